// Router top-k softmax, expert histogram + stable permute, and unpermute/combine.
// Index outputs are bit-exact against the oracle: the logits use one fixed fp32 summation order
// (64 lane partials over k = lane + 64 j, then a xor butterfly 32,16,8,4,2,1) and ties in top-k
// go to the lower expert id.
#include "common.h"

namespace flyai {

// ------------------------------------------------------------------------------------------------
// Router: one workgroup (4 waves) per TT tokens.  x rows staged in LDS; each wave owns every 4th
// expert; the router weight row is read once per workgroup and reused for all TT tokens.
template <int TT>
__global__ __launch_bounds__(256) void router_topk_softmax_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ w, const uint16_t* __restrict__ b,
    int T, int H, int E, int k, int32_t* __restrict__ topk_ids, float* __restrict__ topk_w,
    float* __restrict__ logits_out) {
  extern __shared__ uint16_t xs[];                  // [TT][H]
  __shared__ float logits[TT][256];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int t0 = blockIdx.x * TT;
  const int nt = min(TT, T - t0);
  // stage x rows (16-byte vectors; H % 64 == 0 so rows are 16-byte aligned)
  const int vecs = H / 8;
  for (int i = tid; i < nt * vecs; i += 256) {
    int t = i / vecs, v = i % vecs;
    reinterpret_cast<uint4*>(xs + t * H)[v] = reinterpret_cast<const uint4*>(x + (size_t)(t0 + t) * H)[v];
  }
  __syncthreads();
  const int J = H / 64;
  for (int e = wave; e < E; e += 4) {
    float acc[TT];
#pragma unroll
    for (int t = 0; t < TT; ++t) acc[t] = 0.f;
    const uint16_t* wr = w + (size_t)e * H + lane;
    for (int j = 0; j < J; ++j) {
      const float wv = bf2f(wr[64 * j]);
#pragma unroll
      for (int t = 0; t < TT; ++t)
        acc[t] = fmaf(bf2f(xs[t * H + lane + 64 * j]), wv, acc[t]);   // exact product: fma == mul+add
    }
    const float bias = bf2f(b[e]);
#pragma unroll
    for (int t = 0; t < TT; ++t) {
      float v = acc[t];
#pragma unroll
      for (int off = 32; off >= 1; off >>= 1) v = v + __shfl_xor(v, off, 64);
      if (lane == 0) logits[t][e] = bf16_round(v + bias);
    }
  }
  __syncthreads();
  // top-k per token: wave w handles tokens w, w+4, ...
  for (int t = wave; t < nt; t += 4) {
    float cv[4];
    int ci[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      ci[c] = lane + 64 * c;
      cv[c] = ci[c] < E ? logits[t][ci[c]] : -INFINITY;
      if (ci[c] >= E) ci[c] = 0x7fffffff;
    }
    if (logits_out) {
      for (int c = 0; c < 4; ++c)
        if (lane + 64 * c < E) logits_out[(size_t)(t0 + t) * E + lane + 64 * c] = cv[c];
    }
    float sv[8];
    int si[8];
    for (int r = 0; r < k; ++r) {
      float bv = -INFINITY;
      int bi = 0x7fffffff;
#pragma unroll
      for (int c = 0; c < 4; ++c)
        if (cv[c] > bv || (cv[c] == bv && ci[c] < bi)) { bv = cv[c]; bi = ci[c]; }
#pragma unroll
      for (int off = 32; off >= 1; off >>= 1) {
        float ov = __shfl_xor(bv, off, 64);
        int oi = __shfl_xor(bi, off, 64);
        if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
      }
      sv[r] = bv;
      si[r] = bi;
#pragma unroll
      for (int c = 0; c < 4; ++c)
        if (ci[c] == bi) { cv[c] = -INFINITY; ci[c] = 0x7fffffff; }
    }
    if (lane == 0) {
      const float m = sv[0];
      float ex[8], sum = 0.f;
      for (int r = 0; r < k; ++r) { ex[r] = expf(sv[r] - m); sum += ex[r]; }
      // ascending ids, weights carried along (insertion sort, k <= 8)
      for (int r = 1; r < k; ++r) {
        int id = si[r];
        float e2 = ex[r];
        int q = r - 1;
        while (q >= 0 && si[q] > id) { si[q + 1] = si[q]; ex[q + 1] = ex[q]; --q; }
        si[q + 1] = id;
        ex[q + 1] = e2;
      }
      for (int r = 0; r < k; ++r) {
        topk_ids[(size_t)(t0 + t) * k + r] = si[r];
        topk_w[(size_t)(t0 + t) * k + r] = ex[r] / sum;
      }
    }
  }
}

int launch_router(const uint16_t* x, const uint16_t* w, const uint16_t* b, int T, int H, int E,
                  int k, int32_t* ids, float* wts, float* logits, hipStream_t s) {
  if (T == 0) return FLYAI_OK;
  if (H <= 3072) {  // 8 rows of x + logits stay under 64 KiB of LDS
    hipLaunchKernelGGL(router_topk_softmax_kernel<8>, dim3(ceil_div(T, 8)), dim3(256),
                       8 * H * sizeof(uint16_t), s, x, w, b, T, H, E, k, ids, wts, logits);
  } else {
    hipLaunchKernelGGL(router_topk_softmax_kernel<4>, dim3(ceil_div(T, 4)), dim3(256),
                       4 * H * sizeof(uint16_t), s, x, w, b, T, H, E, k, ids, wts, logits);
  }
  return check_launch("router_topk_softmax");
}

// ------------------------------------------------------------------------------------------------
// Histogram + exclusive scan + stable permute in one 16-wave workgroup.  Each wave owns a
// contiguous segment of the flattened assignments; within a 64-assignment chunk, lanes with the
// same expert find each other with 8 ballots (one per id bit), rank = popcount of lower peers, and
// the lowest peer updates that wave's per-expert counter.  Pass 1 counts, the scan turns counts
// into per-(wave, expert) cursors, pass 2 scatters.  Order: experts ascending, flat index ascending.
constexpr int kPermWaves = 16;

__device__ __forceinline__ uint64_t match_peers(int e, bool valid, int nbits) {
  uint64_t peers = __ballot(valid);
  for (int bit = 0; bit < nbits; ++bit) {
    const bool set = valid && ((e >> bit) & 1);
    const uint64_t m = __ballot(set);
    peers &= set ? m : ~m;
  }
  return peers;
}

__global__ __launch_bounds__(kPermWaves * 64) void moe_permute_kernel(
    const int32_t* __restrict__ ids, int P, int E, int32_t* __restrict__ hist_out,
    int32_t* __restrict__ off_out, int32_t* __restrict__ perm, int32_t* __restrict__ inv) {
  __shared__ int32_t cnt[kPermWaves][256];
  __shared__ int32_t off[256];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  for (int i = tid; i < kPermWaves * 256; i += kPermWaves * 64) (&cnt[0][0])[i] = 0;
  __syncthreads();
  int nbits = 0;
  while ((1 << nbits) < E) ++nbits;
  const int seg = ((P + kPermWaves * 64 - 1) / (kPermWaves * 64)) * 64;
  const int beg = min(P, wave * seg), end = min(P, beg + seg);
  const uint64_t lt = (lane == 0) ? 0ull : ((~0ull) >> (64 - lane));
  for (int base = beg; base < end; base += 64) {
    const int a = base + lane;
    int e = a < end ? ids[a] : -1;
    const bool valid = e >= 0 && e < E;   // an out-of-range id is dropped, never indexes LDS
    if (!valid) e = 0;
    const uint64_t peers = match_peers(e, valid, nbits);
    if (valid && (peers & lt) == 0) cnt[wave][e] += __popcll(peers);
  }
  __syncthreads();
  if (tid < E) {
    int h = 0;
    for (int w = 0; w < kPermWaves; ++w) h += cnt[w][tid];
    hist_out[tid] = h;
    off[tid] = h;
  }
  __syncthreads();
  if (wave == 0) {  // exclusive scan of off[0..E), 4 entries per lane
    int v[4], s = 0;
    for (int c = 0; c < 4; ++c) { int i = lane * 4 + c; v[c] = i < E ? off[i] : 0; s += v[c]; }
    int incl = s;
    for (int o = 1; o < 64; o <<= 1) { int y = __shfl_up(incl, o, 64); if (lane >= o) incl += y; }
    int run = incl - s;
    for (int c = 0; c < 4; ++c) { int i = lane * 4 + c; if (i < E) off[i] = run; run += v[c]; }
  }
  __syncthreads();
  if (tid < E) {
    int run = off[tid];
    off_out[tid] = run;
    for (int w = 0; w < kPermWaves; ++w) { int c = cnt[w][tid]; cnt[w][tid] = run; run += c; }
  }
  if (tid == 0) off_out[E] = P;
  __syncthreads();
  for (int base = beg; base < end; base += 64) {
    const int a = base + lane;
    int e = a < end ? ids[a] : -1;
    const bool valid = e >= 0 && e < E;
    if (!valid) e = 0;
    const uint64_t peers = match_peers(e, valid, nbits);
    if (valid) {
      const int pos = cnt[wave][e] + __popcll(peers & lt);
      perm[pos] = a;
      inv[a] = pos;
    }
    if (valid && (peers & lt) == 0) cnt[wave][e] += __popcll(peers);
  }
}

int launch_permute(const int32_t* ids, int T, int k, int E, int32_t* hist, int32_t* offsets,
                   int32_t* perm, int32_t* inv, hipStream_t s) {
  hipLaunchKernelGGL(moe_permute_kernel, dim3(1), dim3(kPermWaves * 64), 0, s, ids, T * k, E,
                     hist, offsets, perm, inv);
  return check_launch("moe_permute");
}

// ------------------------------------------------------------------------------------------------
// Combine: out[t] = bf16(sum_s w[t,s] * y_perm[inv[t*k+s]]) (+ residual, rounded again).
__global__ __launch_bounds__(256) void moe_combine_kernel(
    const float* __restrict__ y_perm, const int32_t* __restrict__ inv,
    const float* __restrict__ topk_w, int k, int H, const uint16_t* residual, uint16_t* out) {
  const int t = blockIdx.x;
  int rows[8];
  float wt[8];
  for (int s = 0; s < k; ++s) { rows[s] = inv[t * k + s]; wt[s] = topk_w[t * k + s]; }
  const int H4 = H / 4;
  for (int i = threadIdx.x; i < H4; i += 256) {
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int s = 0; s < k; ++s) {
      const float4 y = reinterpret_cast<const float4*>(y_perm + (size_t)rows[s] * H)[i];
      acc.x = fmaf(wt[s], y.x, acc.x);
      acc.y = fmaf(wt[s], y.y, acc.y);
      acc.z = fmaf(wt[s], y.z, acc.z);
      acc.w = fmaf(wt[s], y.w, acc.w);
    }
    float o[4] = {bf16_round(acc.x), bf16_round(acc.y), bf16_round(acc.z), bf16_round(acc.w)};
    if (residual) {
      const uint2 r = reinterpret_cast<const uint2*>(residual + (size_t)t * H)[i];
      o[0] += bf2f(r.x & 0xffff); o[1] += bf2f(r.x >> 16);
      o[2] += bf2f(r.y & 0xffff); o[3] += bf2f(r.y >> 16);
    }
    uint2 ov;
    ov.x = (uint32_t)f2bf(o[0]) | ((uint32_t)f2bf(o[1]) << 16);
    ov.y = (uint32_t)f2bf(o[2]) | ((uint32_t)f2bf(o[3]) << 16);
    reinterpret_cast<uint2*>(out + (size_t)t * H)[i] = ov;
  }
}

int launch_combine(const float* y_perm, const int32_t* inv, const float* w, int T, int k, int H,
                   const uint16_t* residual, uint16_t* out, hipStream_t s) {
  if (T == 0) return FLYAI_OK;
  hipLaunchKernelGGL(moe_combine_kernel, dim3(T), dim3(256), 0, s, y_perm, inv, w, k, H,
                     residual, out);
  return check_launch("moe_combine");
}

}  // namespace flyai

using namespace flyai;

extern "C" int flyai_router_topk_softmax(const uint16_t* x, const uint16_t* w, const uint16_t* b,
                                         int32_t T, int32_t H, int32_t E, int32_t k,
                                         int32_t* topk_ids, float* topk_w, float* logits_out,
                                         flyai_stream_t stream) {
  FLYAI_REQUIRE(T >= 0 && H > 0 && H % 64 == 0 && H <= 7168, "router: H must be a multiple of 64 <= 7168");
  FLYAI_REQUIRE(E >= 1 && E <= 256 && k >= 1 && k <= 8 && k <= E, "router: need 1<=E<=256, 1<=k<=min(8,E)");
  FLYAI_REQUIRE(x && w && b && topk_ids && topk_w, "router: null pointer");
  return launch_router(x, w, b, T, H, E, k, topk_ids, topk_w, logits_out, as_stream(stream));
}

extern "C" int flyai_moe_permute(const int32_t* topk_ids, int32_t T, int32_t k, int32_t E,
                                 int32_t* hist, int32_t* offsets, int32_t* perm, int32_t* inv,
                                 flyai_stream_t stream) {
  FLYAI_REQUIRE(T >= 0 && k >= 1 && (int64_t)T * k <= 65536, "permute: T*k must be <= 65536");
  FLYAI_REQUIRE(E >= 1 && E <= 256, "permute: E must be in [1, 256]");
  FLYAI_REQUIRE(topk_ids && hist && offsets && perm && inv, "permute: null pointer");
  return launch_permute(topk_ids, T, k, E, hist, offsets, perm, inv, as_stream(stream));
}

extern "C" int flyai_moe_combine(const float* y_perm, const int32_t* inv, const float* topk_w,
                                 int32_t T, int32_t k, int32_t H, const uint16_t* residual,
                                 uint16_t* out, flyai_stream_t stream) {
  FLYAI_REQUIRE(T >= 0 && k >= 1 && k <= 8 && H > 0 && H % 4 == 0, "combine: bad shape");
  FLYAI_REQUIRE(y_perm && inv && topk_w && out, "combine: null pointer");
  return launch_combine(y_perm, inv, topk_w, T, k, H, residual, out, as_stream(stream));
}
