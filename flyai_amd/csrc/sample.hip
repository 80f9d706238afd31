// Token sampling on the logits rows of the lm_head: temperature, top-k, top-p (nucleus) filtering,
// the filtered distribution, the probability of a drafted token, and an inverse-CDF draw -- the
// Sampler of phase0/specsample.py:36-107 (dist, sample_logits, accept's residual draw) on the GPU.
//
// Definition, per logits row x[V] (bf16):
//   z_v = x_v / max(temp, 1e-6) (fp32);
//   top-k (0 < k < V): keep z_v >= the k-th largest z (counted with multiplicity);
//   weights w_v = floor(2^40 * e^(z_v - max z)) as exact integers, 0 for masked tokens, with e^d from
//     samp_exp below (fixed fp64 operations, so every build computes the same integers);
//   top-p (0 < p < 1): with the kept tokens ordered by (z desc, id asc; -0 and +0 are one value),
//     keep a token iff the weight of the tokens before it is <= floor(p * W) (W = the sum of the
//     kept weights, p * W one fp64 product);
//   the distribution is w' / W' over what is kept;
//   a draw with uniform u in [0, 1) is the first id v (ascending) whose inclusive prefix of w'' exceeds
//     floor(u * W''), where w'' is w' with the drafted token's weight removed when a draft is given
//     (the residual of the speculative-sampling rule); when nothing is left (W'' == 0) the draw is the
//     first id of maximal w'.
// Integer weights make every sum independent of the reduction order, so a row's results do not depend
// on the launch shape.  Greedy rows (temp <= 0) draw the first id of maximal x.
#include "common.h"

namespace flyai {

constexpr int kSampThreads = 1024;
constexpr int kSampWaves = kSampThreads / 64;

// order-preserving key of a finite fp32 value: larger value <=> larger key (-0 keyed as +0)
__device__ __forceinline__ uint32_t f32_key(float z) {
  const uint32_t u = z == 0.f ? 0u : __float_as_uint(z);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ float key_f32(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

// floor(2^40 * e^d) for d <= 0, by Cody-Waite range reduction (d = k ln2 + r, |r| <= ln2 / 2, ln2 split
// into a 32-bit head, so k * head is exact, and a tail) and the degree-13 Taylor polynomial of e^r
// (truncation error below 5e-18), each fp64 operation rounded on its own (no fused multiply-add):
// within one unit of the exact floor.  d below -27.75 gives 0 (2^40 e^d < 1 there).
__device__ __forceinline__ uint64_t samp_weight(float z, float zmax) {
#pragma clang fp contract(off)
  const double d = (double)z - (double)zmax;
  if (!(d >= -27.75)) return 0;
  const double k = rint(d * 0x1.71547652b82fep+0);
  const double r = (d - k * 0x1.62e42feep-1) - k * 0x1.a39ef35793c76p-33;
  double p = 0x1.6124613a86d09p-33;
  p = p * r + 0x1.1eed8eff8d898p-29;
  p = p * r + 0x1.ae64567f544e4p-26;
  p = p * r + 0x1.27e4fb7789f5cp-22;
  p = p * r + 0x1.71de3a556c734p-19;
  p = p * r + 0x1.a01a01a01a01ap-16;
  p = p * r + 0x1.a01a01a01a01ap-13;
  p = p * r + 0x1.6c16c16c16c17p-10;
  p = p * r + 0x1.1111111111111p-7;
  p = p * r + 0x1.5555555555555p-5;
  p = p * r + 0x1.5555555555555p-3;
  p = p * r + 0x1p-1;
  p = p * r + 1.0;
  p = p * r + 1.0;
  return (uint64_t)floor(ldexp(p, (int)k + 40));
}

// block sums over the 1024 threads through LDS (one slot per wave)
template <class T>
__device__ __forceinline__ T block_sum(T v, T* red) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) red[wave] = v;
  __syncthreads();
  T s = 0;
#pragma unroll
  for (int w = 0; w < kSampWaves; ++w) s += red[w];
  return s;
}

__device__ __forceinline__ uint32_t block_max_u32(uint32_t v, uint32_t* red) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = max(v, (uint32_t)__shfl_xor((int)v, o, 64));
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) red[wave] = v;
  __syncthreads();
  uint32_t m = 0;
#pragma unroll
  for (int w = 0; w < kSampWaves; ++w) m = max(m, red[w]);
  return m;
}

struct SampShared {
  uint64_t hist[256];
  uint64_t red64[kSampWaves];
  uint32_t red32[kSampWaves];
  uint64_t scan[kSampThreads];
  uint64_t sel_above;  // weight (or count) above the selected bin
  uint32_t sel_prefix;
  int sel_found;
};

// Radix selection over the 32-bit keys of the kept tokens, 8 bits per pass from the top: the key of
// the token where the running total of `mass` (counts for top-k, weights for top-p), taken in
// descending key order, first exceeds `limit`.  Returns the key; *above gets the total mass of the
// kept tokens with larger keys.  If the total never exceeds limit, returns 0 with *above = total.
template <class KeyOf, class MassOf>
__device__ uint32_t radix_select(int V, KeyOf key_of, MassOf mass_of, uint64_t limit, uint64_t* above, SampShared& sh) {
  uint32_t prefix = 0;
  uint64_t run = 0;  // mass of tokens above the current prefix's range
  for (int shift = 24; shift >= 0; shift -= 8) {
    for (int b = threadIdx.x; b < 256; b += kSampThreads) sh.hist[b] = 0;
    __syncthreads();
    const uint32_t hi_mask = shift == 24 ? 0u : (0xffffffffu << (shift + 8));
    for (int v = threadIdx.x; v < V; v += kSampThreads) {
      uint32_t k;
      uint64_t m;
      if (!key_of(v, &k)) continue;
      if ((k & hi_mask) != (prefix & hi_mask)) continue;
      m = mass_of(v);
      if (m) atomicAdd((unsigned long long*)&sh.hist[(k >> shift) & 0xff], (unsigned long long)m);
    }
    __syncthreads();
    if (threadIdx.x == 0) {
      int found = -1;
      uint64_t r = run;
      for (int b = 255; b >= 0; --b) {
        if (r + sh.hist[b] > limit) {
          found = b;
          break;
        }
        r += sh.hist[b];
      }
      sh.sel_found = found;
      sh.sel_above = r;
      sh.sel_prefix = found >= 0 ? (prefix | ((uint32_t)found << shift)) : 0u;
    }
    __syncthreads();
    if (sh.sel_found < 0) {
      *above = sh.sel_above;
      return 0u;
    }
    prefix = sh.sel_prefix;
    run = sh.sel_above;
  }
  *above = run;
  return prefix;
}

__global__ __launch_bounds__(kSampThreads) void sample_rows_kernel(
    const uint16_t* __restrict__ logits, int V, float temp, int top_k, float top_p,
    const int32_t* __restrict__ draft, const double* __restrict__ u, float* __restrict__ p_draft,
    int32_t* __restrict__ draw, float* __restrict__ probs) {
  __shared__ SampShared sh;
  const int row = blockIdx.x;
  const uint16_t* x = logits + (size_t)row * V;
  const int tid = threadIdx.x;
  const int d = draft ? draft[row] : -1;
  const int C = (V + kSampThreads - 1) / kSampThreads;  // ids of thread t for ordered scans: [tC, tC+C)

  if (!(temp > 0.f)) {  // greedy: the first id of maximal x
    uint32_t best = 0;
    for (int v = tid; v < V; v += kSampThreads) best = max(best, f32_key(bf2f(x[v])));
    best = block_max_u32(best, sh.red32);
    int first = V;
    for (int v = tid; v < V; v += kSampThreads)
      if (f32_key(bf2f(x[v])) == best) { first = v; break; }
    // smallest id among the threads' first hits
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) first = min(first, __shfl_xor(first, o, 64));
    __syncthreads();
    if ((tid & 63) == 0) sh.red32[tid >> 6] = (uint32_t)first;
    __syncthreads();
    int arg = V;
    for (int w = 0; w < kSampWaves; ++w) arg = min(arg, (int)sh.red32[w]);
    if (tid == 0) {
      if (draw) draw[row] = arg;
      if (p_draft) p_draft[row] = (d == arg) ? 1.f : 0.f;
    }
    if (probs)
      for (int v = tid; v < V; v += kSampThreads) probs[(size_t)row * V + v] = v == arg ? 1.f : 0.f;
    return;
  }
  const float tdiv = fmaxf(temp, 1e-6f);
  auto zof = [&](int v) __attribute__((always_inline)) { return __fdiv_rn(bf2f(x[v]), tdiv); };

  // top-k: the k-th largest key, counted with multiplicity
  uint32_t kth = 0;
  if (top_k > 0 && top_k < V) {
    uint64_t above = 0;
    kth = radix_select(V, [&](int v, uint32_t* k) { *k = f32_key(zof(v)); return true; },
                       [&](int) { return (uint64_t)1; }, (uint64_t)(top_k - 1), &above, sh);
  }
  auto kept_k = [&](int v, uint32_t* k) __attribute__((always_inline)) {
    *k = f32_key(zof(v));
    return *k >= kth;
  };
  // max z, then the weights' total
  uint32_t mkey = 0;
  for (int v = tid; v < V; v += kSampThreads) mkey = max(mkey, f32_key(zof(v)));
  mkey = block_max_u32(mkey, sh.red32);
  const float zmax = key_f32(mkey);
  uint64_t wsum = 0;
  for (int v = tid; v < V; v += kSampThreads) {
    uint32_t k;
    if (kept_k(v, &k)) wsum += samp_weight(zof(v), zmax);
  }
  const uint64_t W = block_sum(wsum, sh.red64);

  // top-p: the boundary key and how many of its ties (in id order) are kept
  uint32_t pkey = 0;
  uint64_t tie_keep = ~0ull;  // ties at pkey kept (all when top-p is off)
  if (top_p > 0.f && top_p < 1.f) {
    const uint64_t T = (uint64_t)floor((double)top_p * (double)W);
    // the boundary: the first token (descending order) whose inclusive running weight exceeds T; every
    // token above it is kept (its preceding weight is <= T), every token below it is dropped
    uint64_t above = 0;
    pkey = radix_select(V, kept_k, [&](int v) { return samp_weight(zof(v), zmax); }, T, &above, sh);
    if (pkey != 0u) {
      // tie j (0-based, id order) of the boundary value is kept iff above + j * wb <= T (tie 0 always is)
      const uint64_t wb = samp_weight(key_f32(pkey), zmax);
      tie_keep = wb == 0 ? ~0ull : (T - above) / wb + 1;
    }
  }
  // ordered pass 1: per-thread counts of boundary ties (for tie ranks) and kept weights
  const int v0 = tid * C, v1 = min(V, v0 + C);
  uint64_t my_ties = 0;
  if (pkey != 0u)
    for (int v = v0; v < v1; ++v) {
      uint32_t k;
      if (kept_k(v, &k) && k == pkey) ++my_ties;
    }
  __syncthreads();
  sh.scan[tid] = my_ties;
  __syncthreads();
  // exclusive prefix of tie counts (thread 0 serial scan of 1024 values; a small fraction of the work)
  if (tid == 0) {
    uint64_t acc = 0;
    for (int t = 0; t < kSampThreads; ++t) {
      const uint64_t c = sh.scan[t];
      sh.scan[t] = acc;
      acc += c;
    }
  }
  __syncthreads();
  const uint64_t tie_base = sh.scan[tid];
  auto final_w = [&](int v, uint64_t* tie_rank) __attribute__((always_inline)) -> uint64_t {
    uint32_t k;
    if (!kept_k(v, &k)) return 0;
    if (pkey != 0u) {
      if (k < pkey) return 0;
      if (k == pkey) {
        const bool keep = *tie_rank < tie_keep;
        ++*tie_rank;
        if (!keep) return 0;
      }
    }
    return samp_weight(zof(v), zmax);
  };
  // ordered pass 2: kept weights per thread (W'), the draft's weight, the first maximal weight
  uint64_t my_w = 0, wd = 0, best_w = 0;
  int best_v = V;
  {
    uint64_t tr = tie_base;
    for (int v = v0; v < v1; ++v) {
      const uint64_t w = final_w(v, &tr);
      my_w += w;
      if (v == d) wd = w;
      if (w > best_w) { best_w = w; best_v = v; }
    }
  }
  const uint64_t Wk = block_sum(my_w, sh.red64);
  const uint64_t Wd = block_sum(wd, sh.red64);
  if (tid == 0 && p_draft) p_draft[row] = (d >= 0 && Wk > 0) ? (float)((double)Wd / (double)Wk) : 0.f;
  if (probs) {
    uint64_t tr = tie_base;
    for (int v = v0; v < v1; ++v) {
      const uint64_t w = final_w(v, &tr);
      probs[(size_t)row * V + v] = Wk > 0 ? (float)((double)w / (double)Wk) : 0.f;
    }
  }
  if (!(draw && u)) return;
  // the draw: residual weights (draft removed), inverse CDF in id order
  const uint64_t my_r = my_w - wd;
  __syncthreads();
  sh.scan[tid] = my_r;
  __syncthreads();
  if (tid == 0) {
    uint64_t acc = 0;
    for (int t = 0; t < kSampThreads; ++t) {
      const uint64_t c = sh.scan[t];
      sh.scan[t] = acc;
      acc += c;
    }
    sh.sel_above = acc;  // W''
  }
  __syncthreads();
  const uint64_t Wr = sh.sel_above;
  if (Wr == 0) {  // nothing left: the first id of maximal kept weight
    // first maximum across threads: max weight, then the smallest id holding it
    __syncthreads();
    sh.scan[tid] = best_w;
    __syncthreads();
    if (tid == 0) {
      uint64_t bw = 0;
      for (int t = 0; t < kSampThreads; ++t) bw = sh.scan[t] > bw ? sh.scan[t] : bw;
      sh.hist[0] = bw;
    }
    __syncthreads();
    const int cand = best_w == sh.hist[0] ? best_v : V;
    int m = cand;
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) m = min(m, __shfl_xor(m, o, 64));
    __syncthreads();
    if ((tid & 63) == 0) sh.red32[tid >> 6] = (uint32_t)m;
    __syncthreads();
    if (tid == 0) {
      int a = V;
      for (int w = 0; w < kSampWaves; ++w) a = min(a, (int)sh.red32[w]);
      draw[row] = a < V ? a : 0;  // every weight 0 (a non-finite row): the first id, as argmax of zeros
    }
    return;
  }
  double uu = u[row];
  if (!(uu >= 0.0)) uu = 0.0;  // u below 0 (or NaN) draws as 0; u >= 1 is held at Wr - 1 below
  uint64_t target = (uint64_t)(uu * (double)Wr);
  if (target >= Wr) target = Wr - 1;
  const uint64_t base = sh.scan[tid];
  if (target >= base && target < base + my_r) {
    uint64_t acc = base, tr = tie_base;
    for (int v = v0; v < v1; ++v) {
      uint64_t w = final_w(v, &tr);
      if (v == d) w = 0;
      acc += w;
      if (acc > target) {
        draw[row] = v;
        break;
      }
    }
  }
}

// A draw from a given probability vector (the reference's Sampler.sample(probs)): weights
// floor(p_v * 2^40), then the same inverse-CDF rule; all-zero -> the first maximal id (0).
__global__ __launch_bounds__(kSampThreads) void sample_probs_kernel(const float* __restrict__ p, int V, double u,
                                                                    int32_t* __restrict__ out) {
  __shared__ SampShared sh;
  const int tid = threadIdx.x;
  const int C = (V + kSampThreads - 1) / kSampThreads;
  const int v0 = tid * C, v1 = min(V, v0 + C);
  uint64_t my = 0;
  for (int v = v0; v < v1; ++v) my += (uint64_t)((double)fmaxf(p[v], 0.f) * 0x1p40);
  sh.scan[tid] = my;
  __syncthreads();
  if (tid == 0) {
    uint64_t acc = 0;
    for (int t = 0; t < kSampThreads; ++t) {
      const uint64_t c = sh.scan[t];
      sh.scan[t] = acc;
      acc += c;
    }
    sh.sel_above = acc;
  }
  __syncthreads();
  const uint64_t W = sh.sel_above;
  if (W == 0) {
    if (tid == 0) out[0] = 0;
    return;
  }
  uint64_t target = (uint64_t)(u * (double)W);
  if (target >= W) target = W - 1;
  const uint64_t base = sh.scan[tid];
  if (target >= base && target < base + my) {
    uint64_t acc = base;
    for (int v = v0; v < v1; ++v) {
      acc += (uint64_t)((double)fmaxf(p[v], 0.f) * 0x1p40);
      if (acc > target) {
        out[0] = v;
        break;
      }
    }
  }
}

}  // namespace flyai

using namespace flyai;

extern "C" int flyai_sample_rows(const uint16_t* logits, int32_t R, int32_t V, float temp, int32_t top_k,
                                 float top_p, const int32_t* draft, const double* u, float* p_draft,
                                 int32_t* draw, float* probs, flyai_stream_t stream) {
  FLYAI_REQUIRE(R >= 0 && V > 0, "sample_rows: bad shape");
  FLYAI_REQUIRE(logits, "sample_rows: null logits");
  FLYAI_REQUIRE(top_k >= 0, "sample_rows: top_k must be >= 0");
  FLYAI_REQUIRE(!(draw && !u && temp > 0.f), "sample_rows: a sampled draw needs u");
  if (R == 0) return FLYAI_OK;
  hipLaunchKernelGGL(sample_rows_kernel, dim3(R), dim3(kSampThreads), 0, as_stream(stream), logits, V, temp, top_k,
                     top_p, draft, u, p_draft, draw, probs);
  return check_launch("sample_rows");
}

extern "C" int flyai_sample_probs(const float* probs, int32_t V, double u, int32_t* out, flyai_stream_t stream) {
  FLYAI_REQUIRE(probs && out && V > 0, "sample_probs: bad arguments");
  FLYAI_REQUIRE(u >= 0.0 && u < 1.0, "sample_probs: u must be in [0, 1)");
  hipLaunchKernelGGL(sample_probs_kernel, dim3(1), dim3(kSampThreads), 0, as_stream(stream), probs, V, u, out);
  return check_launch("sample_probs");
}
