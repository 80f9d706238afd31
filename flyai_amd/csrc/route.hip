// Router top-k softmax, expert histogram + stable permute, and unpermute/combine.
// Index outputs are bit-exact against the oracle: the logits use one fixed fp32 summation order
// (64 lane partials, lane l over k = 512 j + 8 l + i in order, then a xor butterfly 32,16,8,4,2,1)
// and ties in top-k go to the lower expert id.
#include <type_traits>

#include "common.h"

namespace flyai {

// ------------------------------------------------------------------------------------------------
// Router logits: workgroup = (TT tokens, 4*EPW experts); x rows staged in LDS; wave w owns EPW
// experts.  Lane l accumulates k = 512 j + 8 l + i (i = 0..7) in order -- one 16-byte load of the
// weight row and one 16-byte LDS read of x per chunk -- then a xor butterfly (as a reduce-scatter
// over the wave's EPW x TT sums, wave_sum_scatter).  All JMAX weight
// chunks of the wave's experts are loaded before the first FMA (one memory round trip).
// XCD_GROUPED (a 1-D grid): the expert groups of one token group run one after another on one XCD
// (workgroups are dealt to the 8 XCDs round-robin by index), so that XCD's L2 serves their x rows
// after the first; with the 2-D grid they landed on different XCDs and each read x from HBM.
template <int TT, int EPW, int JMAX, bool ROUND_BF16, bool XCD_GROUPED = false>
__global__ __launch_bounds__(256) void router_logits_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ w, const uint16_t* __restrict__ b,
    int T, int H, int E, float* __restrict__ logits) {
  extern __shared__ uint16_t xs[];  // [TT][H]
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  int tg = blockIdx.x, eg = blockIdx.y;
  if (XCD_GROUPED) {
    const int neg = (E + 4 * EPW - 1) / (4 * EPW);
    const int r = (int)blockIdx.x / 8;
    eg = r % neg;
    tg = (r / neg) * 8 + (int)blockIdx.x % 8;
    if (tg * TT >= T) return;  // uniform over the workgroup
  }
  const int t0 = tg * TT;
  const int nt = min(TT, T - t0);
  const int e0 = eg * 4 * EPW + wave * EPW;
  uint4 wv[EPW][JMAX];
#pragma unroll
  for (int c = 0; c < EPW; ++c)
#pragma unroll
    for (int j = 0; j < JMAX; ++j) {
      const int k0 = 512 * j + 8 * lane;
      wv[c][j] = (e0 + c < E && k0 < H) ? *reinterpret_cast<const uint4*>(w + (size_t)(e0 + c) * H + k0)
                                        : make_uint4(0, 0, 0, 0);
    }
  const int vecs = H / 8;
  typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
  // every staging load of the thread goes out (with the weights above) before the first LDS store:
  // one memory round trip for the whole workgroup (H <= JMAX * 512 bounds the count)
  constexpr int kPer = (TT * JMAX * 64 + 255) / 256;
  u32x4 v4[kPer];
  // (token, vector) of element j * 256 + tid, stepped by 256 without integer divisions
  int jt[kPer], jv[kPer];
  {
    int ct = 0, cv = tid;
    while (cv >= vecs) {
      cv -= vecs;
      ++ct;
    }
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      jt[j] = ct;
      jv[j] = cv;
      cv += 256;
      while (cv >= vecs) {
        cv -= vecs;
        ++ct;
      }
    }
  }
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    const int t = jt[j], v = jv[j];
    const bool ok = t < TT && t < nt;  // (t < TT: element index < TT * vecs)
    const u32x4 val = reinterpret_cast<const u32x4*>(x + (ok ? (size_t)(t0 + t) * H : 0))[ok ? v : 0];
    v4[j] = ok ? val : u32x4{0u, 0u, 0u, 0u};
  }
#pragma unroll
  for (int j = 0; j < kPer; ++j)
    if (jt[j] < TT) reinterpret_cast<u32x4*>(xs + jt[j] * H)[jv[j]] = v4[j];
  __syncthreads();
  float acc[EPW][TT];
#pragma unroll
  for (int c = 0; c < EPW; ++c)
#pragma unroll
    for (int t = 0; t < TT; ++t) acc[c][t] = 0.f;
#pragma unroll
  for (int j = 0; j < JMAX; ++j) {
    const int k0 = 512 * j + 8 * lane;
    if (k0 >= H) break;  // lanes past the row end keep their partial unchanged
#pragma unroll
    for (int t = 0; t < TT; ++t) {
      const uint4 xv = *reinterpret_cast<const uint4*>(xs + t * H + k0);
      const uint32_t xw[4] = {xv.x, xv.y, xv.z, xv.w};
#pragma unroll
      for (int c = 0; c < EPW; ++c) {
        const uint32_t ww[4] = {wv[c][j].x, wv[c][j].y, wv[c][j].z, wv[c][j].w};
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const float xf = __uint_as_float((i & 1) ? (xw[i >> 1] & 0xffff0000u) : (xw[i >> 1] << 16));
          const float wf = __uint_as_float((i & 1) ? (ww[i >> 1] & 0xffff0000u) : (ww[i >> 1] << 16));
          acc[c][t] = fmaf(xf, wf, acc[c][t]);  // exact product: fma == mul + add
        }
      }
    }
  }
  // the 64-lane sums of all EPW x TT partials (value c TT + t), the butterfly's additions as a
  // reduce-scatter: lane l ends with value l >> shift
  float part[EPW * TT];
#pragma unroll
  for (int c = 0; c < EPW; ++c)
#pragma unroll
    for (int t = 0; t < TT; ++t) part[c * TT + t] = acc[c][t];
  const float v = wave_sum_scatter<EPW * TT>(part);
  constexpr int shift = wave_sum_scatter_shift<EPW * TT>();
  const int idx = lane >> shift, c = idx / TT, t = idx % TT;
  if ((lane & ((1 << shift) - 1)) == 0 && t < nt && e0 + c < E) {
    const float r = v + (b ? bf2f(b[e0 + c]) : 0.f);
    logits[(size_t)(t0 + t) * E + e0 + c] = ROUND_BF16 ? bf16_round(r) : r;
  }
}

template <int K>
__global__ __launch_bounds__(256) void router_topk_kernel(const float* __restrict__ logits, int T,
                                                          int E, int32_t* __restrict__ topk_ids,
                                                          float* __restrict__ topk_w) {
  const int t = blockIdx.x * 256 + threadIdx.x;
  if (t >= T) return;
  topk_softmax_lane<K>(logits + (size_t)t * E, E, topk_ids + (size_t)t * K, topk_w + (size_t)t * K);
}

// The same selection with 4 lanes per token (64 tokens per workgroup) for E % 16 == 0, E <= 256:
// each lane loads its quarter of the row (E/16 float4, all before the first compare) and parks it in
// LDS (rows of E + 4 floats), then topk_softmax_group<K, 4> merges the quarters -- bit-identical to
// topk_softmax_lane.  A lane reads back only what it wrote itself.
template <int K>
__global__ __launch_bounds__(256) void router_topk4_kernel(const float* __restrict__ logits, int T, int E,
                                                           int32_t* __restrict__ topk_ids,
                                                           float* __restrict__ topk_w) {
  extern __shared__ float4 rows_lds[];  // [64][E + 4] floats
  float* row = reinterpret_cast<float*>(rows_lds) + (threadIdx.x >> 2) * (E + 4);
  const int sub = threadIdx.x & 3, tl = threadIdx.x >> 2;
  const int t = blockIdx.x * 64 + tl;
  const int Q = E / 4;
  float4 v[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int e0 = sub * Q + 4 * i;
    v[i] = (t < T && 4 * i < Q) ? *reinterpret_cast<const float4*>(logits + (size_t)t * E + e0)
                                : make_float4(0.f, 0.f, 0.f, 0.f);
  }
#pragma unroll
  for (int i = 0; i < 16; ++i)
    if (4 * i < Q) *reinterpret_cast<float4*>(row + sub * Q + 4 * i) = v[i];
  if (t < T) topk_softmax_group<K, 4>(row, E, sub, topk_ids + (size_t)t * K, topk_w + (size_t)t * K);
}

int launch_router_logits(const uint16_t* x, const uint16_t* w, const uint16_t* b, int T, int H,
                         int E, float* logits, hipStream_t s) {
  if (H <= 3072 && T >= 256) {  // prefill-sized: 16 experts per workgroup halve the x re-reads
    const int ntg8 = ceil_div(ceil_div(T, 8), 8) * 8;  // token groups, rounded to the 8 XCDs
    hipLaunchKernelGGL((router_logits_kernel<8, 4, 6, true, true>), dim3(ntg8 * ceil_div(E, 16)), dim3(256),
                       8 * H * sizeof(uint16_t), s, x, w, b, T, H, E, logits);
  } else if (H <= 3072) {  // 8 staged rows stay under 48 KiB of LDS; 6 chunks of 512
    hipLaunchKernelGGL((router_logits_kernel<8, 2, 6, true>), dim3(ceil_div(T, 8), ceil_div(E, 8)),
                       dim3(256), 8 * H * sizeof(uint16_t), s, x, w, b, T, H, E, logits);
  } else {
    hipLaunchKernelGGL((router_logits_kernel<4, 1, 14, true>), dim3(ceil_div(T, 4), ceil_div(E, 4)),
                       dim3(256), 4 * H * sizeof(uint16_t), s, x, w, b, T, H, E, logits);
  }
  return check_launch("router_logits");
}

int launch_router(const uint16_t* x, const uint16_t* w, const uint16_t* b, int T, int H, int E,
                  int k, int32_t* ids, float* wts, float* logits, hipStream_t s) {
  if (T == 0) return FLYAI_OK;
  int rc = launch_router_logits(x, w, b, T, H, E, logits, s);
  if (rc) return rc;
  if (E % 16 == 0 && E <= 256 && (k == 4 || k == 8 || k == 2)) {
    if (k == 4)
      hipLaunchKernelGGL(router_topk4_kernel<4>, dim3(ceil_div(T, 64)), dim3(256), 64 * (E + 4) * 4, s, logits, T, E,
                         ids, wts);
    else if (k == 8)
      hipLaunchKernelGGL(router_topk4_kernel<8>, dim3(ceil_div(T, 64)), dim3(256), 64 * (E + 4) * 4, s, logits, T, E,
                         ids, wts);
    else
      hipLaunchKernelGGL(router_topk4_kernel<2>, dim3(ceil_div(T, 64)), dim3(256), 64 * (E + 4) * 4, s, logits, T, E,
                         ids, wts);
    return check_launch("router_topk4");
  }
  if (k == 4)
    hipLaunchKernelGGL(router_topk_kernel<4>, dim3(ceil_div(T, 256)), dim3(256), 0, s, logits, T, E, ids, wts);
  else if (k == 8)
    hipLaunchKernelGGL(router_topk_kernel<8>, dim3(ceil_div(T, 256)), dim3(256), 0, s, logits, T, E, ids, wts);
  else if (k == 2)
    hipLaunchKernelGGL(router_topk_kernel<2>, dim3(ceil_div(T, 256)), dim3(256), 0, s, logits, T, E, ids, wts);
  else
    return set_error(FLYAI_EINVAL, "router: top_k must be 2, 4 or 8");
  return check_launch("router_topk");
}

// ------------------------------------------------------------------------------------------------
// DeepSeek-V3 grouped sigmoid routing (vendor/kimi_k3_ref/modeling_kimi_linear.py:703-759) on fp32
// logits, one wave per token; lane l owns experts 4l .. 4l+3 (E <= 256, a group spans E/n_group
// experts = a power-of-two run of lanes).  scores = sigmoid_det(logit); choice = scores + bias;
// group score = top1 + top2 of the group's choices; the topk_group best groups (ties -> lower group)
// stay; the k best unmasked choices (ties -> lower id) are selected; ids ascending; weights =
// score / (sum in ascending id order + 1e-20) * route_scale, all fp32.
//
// sigmoid_det is exp by Cody-Waite reduction (n = rint(z log2 e); r = (z - n LN2_HI) - n LN2_LO,
// LN2_HI with 12 significant bits) and the degree-7 Taylor polynomial by Horner with separate
// multiplies and adds, times 2^n; then 1 / (1 + e) correctly rounded.  FP contraction is off so
// every operation rounds exactly as the oracle's numpy float32 sequence does.
__device__ __forceinline__ float sigmoid_det(float x) {
#pragma clang fp contract(off)
  const float kLog2e = (float)1.4426950408889634;
  const float kLn2Hi = 0.693145751953125f;
  const float kLn2Lo = (float)(0.69314718055994530942 - 0.693145751953125);
  const float z = fminf(fmaxf(-x, -87.0f), 88.0f);
  const float n = rintf(z * kLog2e);
  float r = z - n * kLn2Hi;
  r = r - n * kLn2Lo;
  float p = (float)(1.0 / 5040.0);
  p = p * r; p = p + (float)(1.0 / 720.0);
  p = p * r; p = p + (float)(1.0 / 120.0);
  p = p * r; p = p + (float)(1.0 / 24.0);
  p = p * r; p = p + (float)(1.0 / 6.0);
  p = p * r; p = p + 0.5f;
  p = p * r; p = p + 1.0f;
  p = p * r; p = p + 1.0f;
  const float e = ldexpf(p, (int)n);
  return __fdiv_rn(1.0f, 1.0f + e);
}

// (value desc, id asc) "a before b"
__device__ __forceinline__ bool route_better(float va, int ia, float vb, int ib) {
  return va > vb || (va == vb && ia < ib);
}

template <int K>
__global__ __launch_bounds__(256) void grouped_topk_kernel(const float* __restrict__ logits,
                                                           const float* __restrict__ e_bias, int T,
                                                           int E, int n_group, int topk_group,
                                                           float route_scale, int32_t* __restrict__ ids,
                                                           float* __restrict__ wts) {
#pragma clang fp contract(off)
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;  // uniform per wave
  const int lane = threadIdx.x & 63;
  const float kNegInf = -__builtin_inff();
  float sc[4], ch[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int e = 4 * lane + j;
    if (e < E) {
      sc[j] = sigmoid_det(logits[(size_t)t * E + e]);
      ch[j] = sc[j] + (e_bias ? e_bias[e] : 0.0f);
    } else {
      sc[j] = 0.0f;
      ch[j] = kNegInf;
    }
  }
  if (n_group > 1 && n_group > topk_group) {
    // top-2 values of the lane's 4 choices, then merged across the group's lanes
    float a1 = kNegInf, a2 = kNegInf;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (ch[j] > a1) { a2 = a1; a1 = ch[j]; } else if (ch[j] > a2) { a2 = ch[j]; }
    }
    const int lpg = E / n_group / 4;  // lanes per group (power of two)
    for (int o = 1; o < lpg; o <<= 1) {
      const float b1 = __shfl_xor(a1, o, 64), b2 = __shfl_xor(a2, o, 64);
      const float n1 = fmaxf(a1, b1);
      const float n2 = fmaxf(fminf(a1, b1), fmaxf(a2, b2));
      a1 = n1; a2 = n2;
    }
    const float gs = a1 + a2;
    const int my_g = lane / lpg;
    int rank = 0;
    for (int gg = 0; gg < n_group; ++gg) {
      const float o = __shfl(gs, gg * lpg, 64);
      rank += route_better(o, gg, gs, my_g) ? 1 : 0;
    }
    if (rank >= topk_group || 4 * lane >= E) {
#pragma unroll
      for (int j = 0; j < 4; ++j) ch[j] = kNegInf;
    }
  }
  // k rounds of a wave-wide argmax over (value desc, id asc)
  int sel[K];
  bool taken[4] = {false, false, false, false};
#pragma unroll
  for (int i = 0; i < K; ++i) {
    float bv = kNegInf;
    int bi = 1 << 30;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int e = 4 * lane + j;
      if (!taken[j] && e < E && route_better(ch[j], e, bv, bi)) { bv = ch[j]; bi = e; }
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
      const float ov = __shfl_xor(bv, o, 64);
      const int oi = __shfl_xor(bi, o, 64);
      if (route_better(ov, oi, bv, bi)) { bv = ov; bi = oi; }
    }
    sel[i] = bi;
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (4 * lane + j == bi) taken[j] = true;
  }
  // ids ascending (static odd-even transposition sort), then their unbiased scores
#pragma unroll
  for (int pass = 0; pass < K; ++pass)
#pragma unroll
    for (int i = pass & 1; i + 1 < K; i += 2)
      if (sel[i] > sel[i + 1]) { const int tmp = sel[i]; sel[i] = sel[i + 1]; sel[i + 1] = tmp; }
  float sv[K];
  float den = 0.0f;
#pragma unroll
  for (int i = 0; i < K; ++i) {
    const int j = sel[i] & 3;
    const float mine = j == 0 ? sc[0] : j == 1 ? sc[1] : j == 2 ? sc[2] : sc[3];
    sv[i] = __shfl(mine, sel[i] >> 2, 64);
    den = den + sv[i];
  }
  den = den + (float)1e-20;  // np.float32(1e-20): the double literal rounded once
  if (lane < K) {
    float v = 0.0f;
    int id = 0;
#pragma unroll
    for (int i = 0; i < K; ++i)
      if (i == lane) { v = sv[i]; id = sel[i]; }
    ids[(size_t)t * K + lane] = id;
    wts[(size_t)t * K + lane] = __fdiv_rn(v, den) * route_scale;
  }
}

int launch_router_grouped(const uint16_t* x, const uint16_t* w, const float* e_bias, int T, int H, int E,
                          int n_group, int topk_group, int k, float route_scale, float* logits,
                          int32_t* ids, float* wts, hipStream_t s) {
  if (T == 0) return FLYAI_OK;
  if (H <= 3072)
    hipLaunchKernelGGL((router_logits_kernel<8, 2, 6, false>), dim3(ceil_div(T, 8), ceil_div(E, 8)),
                       dim3(256), 8 * H * sizeof(uint16_t), s, x, w, nullptr, T, H, E, logits);
  else
    hipLaunchKernelGGL((router_logits_kernel<4, 1, 14, false>), dim3(ceil_div(T, 4), ceil_div(E, 4)),
                       dim3(256), 4 * H * sizeof(uint16_t), s, x, w, nullptr, T, H, E, logits);
  int rc = check_launch("router_logits(fp32)");
  if (rc) return rc;
  const dim3 grid(ceil_div(T, 4));
  if (k == 8)
    hipLaunchKernelGGL(grouped_topk_kernel<8>, grid, dim3(256), 0, s, logits, e_bias, T, E, n_group,
                       topk_group, route_scale, ids, wts);
  else if (k == 4)
    hipLaunchKernelGGL(grouped_topk_kernel<4>, grid, dim3(256), 0, s, logits, e_bias, T, E, n_group,
                       topk_group, route_scale, ids, wts);
  else if (k == 6)
    hipLaunchKernelGGL(grouped_topk_kernel<6>, grid, dim3(256), 0, s, logits, e_bias, T, E, n_group,
                       topk_group, route_scale, ids, wts);
  else
    return set_error(FLYAI_EINVAL, "grouped router: top_k must be 4, 6 or 8");
  return check_launch("grouped_topk");
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

// ids may live in global memory or LDS; called by all kPermWaves*64 threads of the workgroup.
__device__ void permute_block(const int32_t* ids, int P, int E, int32_t* __restrict__ hist_out,
                              int32_t* __restrict__ off_out, int32_t* __restrict__ perm,
                              int32_t* __restrict__ inv, int32_t (*cnt)[256], int32_t* off) {
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
    // an id outside [0, E) (a router row of NaN) counts as expert 0, so the histogram still sums to P
    // and every slot gets a perm and an inv entry: the expert and combine kernels index with those
    int e = a < end ? ids[a] : -1;
    const bool valid = a < end;
    if (e < 0 || e >= E) e = 0;
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
    int v[4], sum = 0;
    for (int c = 0; c < 4; ++c) { int i = lane * 4 + c; v[c] = i < E ? off[i] : 0; sum += v[c]; }
    int incl = sum;
    for (int o = 1; o < 64; o <<= 1) { int y = __shfl_up(incl, o, 64); if (lane >= o) incl += y; }
    int run = incl - sum;
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
    const bool valid = a < end;
    if (e < 0 || e >= E) e = 0;
    const uint64_t peers = match_peers(e, valid, nbits);
    if (valid) {
      const int pos = cnt[wave][e] + __popcll(peers & lt);
      perm[pos] = a;
      inv[a] = pos;
    }
    if (valid && (peers & lt) == 0) cnt[wave][e] += __popcll(peers);
  }
}

__global__ __launch_bounds__(kPermWaves * 64) void moe_permute_kernel(
    const int32_t* __restrict__ ids, int P, int E, int32_t* __restrict__ hist_out,
    int32_t* __restrict__ off_out, int32_t* __restrict__ perm, int32_t* __restrict__ inv) {
  __shared__ int32_t cnt[kPermWaves][256];
  __shared__ int32_t off[256];
  permute_block(ids, P, E, hist_out, off_out, perm, inv, cnt, off);
}

// Small batches: top-k of every token (one lane per token) into LDS, then the permute, in one
// workgroup -- one launch instead of two.
constexpr int kFusedMaxAssign = 4096;

constexpr int kStagedLogits = 8192;  // floats of logits staged in LDS (T * (E + 4) <= this)

template <int K>
__global__ __launch_bounds__(kPermWaves * 64) void moe_topk_permute_kernel(
    const float* __restrict__ logits, int T, int E, int32_t* __restrict__ topk_ids,
    float* __restrict__ topk_w, int32_t* __restrict__ hist_out, int32_t* __restrict__ off_out,
    int32_t* __restrict__ perm, int32_t* __restrict__ inv) {
  __shared__ int32_t cnt[kPermWaves][256];
  __shared__ int32_t off[256];
  __shared__ int32_t ids_s[kFusedMaxAssign];
  __shared__ __align__(16) float lg_s[kStagedLogits];
  // one lane per token (a wave selects for 64 tokens at once); small batches first stage all logits
  // in LDS with coalesced loads (rows padded by 16 bytes), so the selection never waits on memory
  const bool staged = T * (E + 4) <= kStagedLogits;
  if (staged) {
    // every load of the thread goes out before the first LDS store (one round trip, not one per
    // element): T * E < kStagedLogits = 8 per thread
    constexpr int kPer = kStagedLogits / (kPermWaves * 64);
    float v[kPer];
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const int i = threadIdx.x + j * kPermWaves * 64;
      v[j] = i < T * E ? logits[i] : 0.f;
    }
    // row-major into rows of E + 4 floats; (row, column) by a shift and a mask when E is a power
    // of two (128 for GPT-OSS), which keeps 16 integer divisions off the single workgroup's path
    if ((E & (E - 1)) == 0) {
      const int e_shift = __builtin_ctz((unsigned)E);
#pragma unroll
      for (int j = 0; j < kPer; ++j) {
        const int i = threadIdx.x + j * kPermWaves * 64;
        if (i < T * E) lg_s[(i >> e_shift) * (E + 4) + (i & (E - 1))] = v[j];
      }
    } else {
#pragma unroll
      for (int j = 0; j < kPer; ++j) {
        const int i = threadIdx.x + j * kPermWaves * 64;
        if (i < T * E) lg_s[(i / E) * (E + 4) + i % E] = v[j];
      }
    }
    __syncthreads();
  }
  if (staged && E % 16 == 0) {
    // four lanes per token: 256 tokens per pass of the workgroup
    const int sub = threadIdx.x & 3;
    for (int t0 = 0; t0 < T; t0 += kPermWaves * 16) {
      const int t = t0 + (threadIdx.x >> 2);
      // whole quads stay together (T rounds the quad index, never splits one)
      if (t < T) topk_softmax_group<K, 4>(lg_s + t * (E + 4), E, sub, ids_s + t * K, topk_w + (size_t)t * K);
    }
  } else {
    for (int t = threadIdx.x; t < T; t += kPermWaves * 64)
      topk_softmax_lane<K>(staged ? lg_s + t * (E + 4) : logits + (size_t)t * E, E, ids_s + t * K,
                           topk_w + (size_t)t * K);
  }
  __syncthreads();
  for (int i = threadIdx.x; i < T * K; i += kPermWaves * 64) topk_ids[i] = ids_s[i];
  permute_block(ids_s, T * K, E, hist_out, off_out, perm, inv, cnt, off);
}

int launch_permute(const int32_t* ids, int T, int k, int E, int32_t* hist, int32_t* offsets,
                   int32_t* perm, int32_t* inv, hipStream_t s);

int launch_route_permute(const uint16_t* x, const uint16_t* w, const uint16_t* b, int T, int H,
                         int E, int k, int32_t* ids, float* wts, float* logits, int32_t* hist,
                         int32_t* offsets, int32_t* perm, int32_t* inv, hipStream_t s) {
  if (T == 0) return FLYAI_OK;
  if (T * k > kFusedMaxAssign) {
    int rc = launch_router(x, w, b, T, H, E, k, ids, wts, logits, s);
    if (rc) return rc;
    return launch_permute(ids, T, k, E, hist, offsets, perm, inv, s);
  }
  int rc = launch_router_logits(x, w, b, T, H, E, logits, s);
  if (rc) return rc;
  if (k == 4)
    hipLaunchKernelGGL(moe_topk_permute_kernel<4>, dim3(1), dim3(kPermWaves * 64), 0, s, logits, T, E,
                       ids, wts, hist, offsets, perm, inv);
  else if (k == 8)
    hipLaunchKernelGGL(moe_topk_permute_kernel<8>, dim3(1), dim3(kPermWaves * 64), 0, s, logits, T, E,
                       ids, wts, hist, offsets, perm, inv);
  else if (k == 2)
    hipLaunchKernelGGL(moe_topk_permute_kernel<2>, dim3(1), dim3(kPermWaves * 64), 0, s, logits, T, E,
                       ids, wts, hist, offsets, perm, inv);
  else
    return set_error(FLYAI_EINVAL, "route: top_k must be 2, 4 or 8");
  return check_launch("moe_topk_permute");
}

// Top-k + softmax of precomputed logits, then histogram / permute (T*k <= 4096: one workgroup).
int launch_topk_permute(const float* logits, int T, int E, int k, int32_t* ids, float* wts, int32_t* hist,
                        int32_t* offsets, int32_t* perm, int32_t* inv, hipStream_t s) {
  if (T == 0) return FLYAI_OK;
  if ((int64_t)T * k > kFusedMaxAssign) return set_error(FLYAI_EINVAL, "topk_permute: T*k > %d", kFusedMaxAssign);
  if (k == 4)
    hipLaunchKernelGGL(moe_topk_permute_kernel<4>, dim3(1), dim3(kPermWaves * 64), 0, s, logits, T, E, ids,
                       wts, hist, offsets, perm, inv);
  else if (k == 8)
    hipLaunchKernelGGL(moe_topk_permute_kernel<8>, dim3(1), dim3(kPermWaves * 64), 0, s, logits, T, E, ids,
                       wts, hist, offsets, perm, inv);
  else if (k == 2)
    hipLaunchKernelGGL(moe_topk_permute_kernel<2>, dim3(1), dim3(kPermWaves * 64), 0, s, logits, T, E, ids,
                       wts, hist, offsets, perm, inv);
  else
    return set_error(FLYAI_EINVAL, "route: top_k must be 2, 4 or 8");
  return check_launch("moe_topk_permute");
}

int launch_permute(const int32_t* ids, int T, int k, int E, int32_t* hist, int32_t* offsets,
                   int32_t* perm, int32_t* inv, hipStream_t s) {
  hipLaunchKernelGGL(moe_permute_kernel, dim3(1), dim3(kPermWaves * 64), 0, s, ids, T * k, E,
                     hist, offsets, perm, inv);
  return check_launch("moe_permute");
}

// ------------------------------------------------------------------------------------------------
// Combine: out[t] = bf16(sum_s w[t,s] * y_perm[inv[t*k+s]]) (+ residual, rounded again).  When lnw is
// given, the next layer's input RMSNorm of the new row is written to xn as well (fused: the row is
// already in this workgroup's registers).  Each thread owns up to kCombinePer float4 column groups;
// the residual and norm weights are loaded before the slot rows, so the row needs one round trip.
constexpr int kCombineThreads = 1024;
constexpr int kCombinePer = 2;  // H <= 4 * 1024 * 2

template <int K>
__global__ __launch_bounds__(kCombineThreads) void moe_combine_kernel(
    const float* __restrict__ y_perm, const int32_t* __restrict__ inv,
    const float* __restrict__ topk_w, int H, const uint16_t* residual, uint16_t* out,
    const float* __restrict__ lnw, float eps, uint16_t* __restrict__ xn) {
  __shared__ float red[kCombineThreads / 64];
  const int t = blockIdx.x, tid = threadIdx.x;
  const int H4 = H / 4;
  // residual may alias out: it is read here, before any store
  float4 lw[kCombinePer];
  uint2 rsd[kCombinePer];
#pragma unroll
  for (int c = 0; c < kCombinePer; ++c) {
    const int i = tid + c * kCombineThreads;
    lw[c] = (lnw && i < H4) ? reinterpret_cast<const float4*>(lnw)[i] : make_float4(0.f, 0.f, 0.f, 0.f);
    rsd[c] = (residual && i < H4) ? reinterpret_cast<const uint2*>(residual + (size_t)t * H)[i] : make_uint2(0, 0);
  }
  int rows[K];
  float wt[K];
#pragma unroll
  for (int s = 0; s < K; ++s) { rows[s] = inv[t * K + s]; wt[s] = topk_w[t * K + s]; }
  float ss = 0.f;
  uint16_t ob[kCombinePer][4];
#pragma unroll
  for (int c = 0; c < kCombinePer; ++c) {
    const int i = tid + c * kCombineThreads;
    if (i >= H4) continue;
    // the K slot rows' loads all go out before the first add (one round trip); sums in slot order
    float4 yv[K];
#pragma unroll
    for (int s = 0; s < K; ++s) yv[s] = reinterpret_cast<const float4*>(y_perm + (size_t)rows[s] * H)[i];
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int s = 0; s < K; ++s) {
      const float4 y = yv[s];
      acc.x = fmaf(wt[s], y.x, acc.x);
      acc.y = fmaf(wt[s], y.y, acc.y);
      acc.z = fmaf(wt[s], y.z, acc.z);
      acc.w = fmaf(wt[s], y.w, acc.w);
    }
    float o[4] = {bf16_round(acc.x), bf16_round(acc.y), bf16_round(acc.z), bf16_round(acc.w)};
    if (residual) {
      o[0] += bf2f(rsd[c].x & 0xffff); o[1] += bf2f(rsd[c].x >> 16);
      o[2] += bf2f(rsd[c].y & 0xffff); o[3] += bf2f(rsd[c].y >> 16);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      ob[c][j] = f2bf(o[j]);
      const float hf = bf2f(ob[c][j]);
      ss = fmaf(hf, hf, ss);
    }
    reinterpret_cast<uint2*>(out + (size_t)t * H)[i] =
        make_uint2((uint32_t)ob[c][0] | ((uint32_t)ob[c][1] << 16), (uint32_t)ob[c][2] | ((uint32_t)ob[c][3] << 16));
  }
  if (!lnw) return;
  ss = warp_sum(ss);
  if ((tid & 63) == 0) red[tid >> 6] = ss;
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int w = 0; w < kCombineThreads / 64; ++w) tot += red[w];
  const float rr = rsqrtf(tot / (float)H + eps);
#pragma unroll
  for (int c = 0; c < kCombinePer; ++c) {
    const int i = tid + c * kCombineThreads;
    if (i >= H4) continue;
    const float lv[4] = {lw[c].x, lw[c].y, lw[c].z, lw[c].w};
    uint16_t q[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) q[j] = f2bf(lv[j] * (bf2f(ob[c][j]) * rr));
    reinterpret_cast<uint2*>(xn + (size_t)t * H)[i] =
        make_uint2((uint32_t)q[0] | ((uint32_t)q[1] << 16), (uint32_t)q[2] | ((uint32_t)q[3] << 16));
  }
}

int launch_combine(const float* y_perm, const int32_t* inv, const float* w, int T, int k, int H,
                   const uint16_t* residual, uint16_t* out, const float* lnw, float eps,
                   uint16_t* xn, hipStream_t s) {
  if (T == 0) return FLYAI_OK;
  auto go = [&](auto kk) {
    hipLaunchKernelGGL((moe_combine_kernel<decltype(kk)::value>), dim3(T), dim3(kCombineThreads), 0, s, y_perm, inv,
                       w, H, residual, out, lnw, eps, xn);
  };
  switch (k) {
    case 1: go(std::integral_constant<int, 1>{}); break;
    case 2: go(std::integral_constant<int, 2>{}); break;
    case 3: go(std::integral_constant<int, 3>{}); break;
    case 4: go(std::integral_constant<int, 4>{}); break;
    case 5: go(std::integral_constant<int, 5>{}); break;
    case 6: go(std::integral_constant<int, 6>{}); break;
    case 7: go(std::integral_constant<int, 7>{}); break;
    case 8: go(std::integral_constant<int, 8>{}); break;
    default: return set_error(FLYAI_EINVAL, "combine: top_k must be 1..8");
  }
  return check_launch("moe_combine");
}

}  // namespace flyai

using namespace flyai;

extern "C" int flyai_router_topk_softmax(const uint16_t* x, const uint16_t* w, const uint16_t* b,
                                         int32_t T, int32_t H, int32_t E, int32_t k,
                                         int32_t* topk_ids, float* topk_w, float* logits_out,
                                         flyai_stream_t stream) {
  FLYAI_REQUIRE(T >= 0 && H > 0 && H <= 7168, "router: H must be <= 7168");
  FLYAI_REQUIRE(E >= 4 && E <= 256 && E % 4 == 0 && (k == 2 || k == 4 || k == 8) && k <= E,
                "router: need E %% 4 == 0, 4 <= E <= 256, k in {2, 4, 8}");
  FLYAI_REQUIRE(x && w && b && topk_ids && topk_w && logits_out, "router: null pointer");
  FLYAI_REQUIRE(H % 8 == 0, "router: H must be a multiple of 8");
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
  FLYAI_REQUIRE(T >= 0 && k >= 1 && k <= 8 && H > 0 && H % 4 == 0 && H <= 4 * kCombineThreads * kCombinePer,
                "combine: need H %% 4 == 0 and H <= %d", 4 * kCombineThreads * kCombinePer);
  FLYAI_REQUIRE(y_perm && inv && topk_w && out, "combine: null pointer");
  return launch_combine(y_perm, inv, topk_w, T, k, H, residual, out, nullptr, 0.f, nullptr,
                        as_stream(stream));
}

extern "C" int flyai_moe_route_permute(const uint16_t* x, const uint16_t* w, const uint16_t* b,
                                       int32_t T, int32_t H, int32_t E, int32_t k,
                                       int32_t* topk_ids, float* topk_w, float* logits,
                                       int32_t* hist, int32_t* offsets, int32_t* perm, int32_t* inv,
                                       flyai_stream_t stream) {
  FLYAI_REQUIRE(T >= 0 && H > 0 && H <= 7168 && H % 8 == 0, "route_permute: H must be a multiple of 8 <= 7168");
  FLYAI_REQUIRE(E >= 4 && E <= 256 && E % 4 == 0 && (k == 2 || k == 4 || k == 8) && k <= E &&
                    (int64_t)T * k <= 65536,
                "route_permute: need E %% 4 == 0, 4 <= E <= 256, k in {2, 4, 8}, T*k <= 65536");
  FLYAI_REQUIRE(x && w && b && topk_ids && topk_w && logits && hist && offsets && perm && inv,
                "route_permute: null pointer");
  return launch_route_permute(x, w, b, T, H, E, k, topk_ids, topk_w, logits, hist, offsets, perm, inv,
                              as_stream(stream));
}

extern "C" int flyai_router_grouped_sigmoid(const uint16_t* x, const uint16_t* w, const float* e_bias,
                                            int32_t T, int32_t H, int32_t E, int32_t n_group,
                                            int32_t topk_group, int32_t k, float route_scale,
                                            float* logits, int32_t* topk_ids, float* topk_w,
                                            flyai_stream_t stream) {
  FLYAI_REQUIRE(T >= 0 && H > 0 && H <= 7168 && H % 8 == 0, "grouped router: H must be a multiple of 8 <= 7168");
  FLYAI_REQUIRE(E >= 4 && E <= 256 && E % 4 == 0 && (k == 4 || k == 6 || k == 8) && k <= E,
                "grouped router: need E %% 4 == 0, 4 <= E <= 256, k in {4, 6, 8}");
  FLYAI_REQUIRE(n_group >= 1 && E % n_group == 0 && topk_group >= 1 && topk_group <= n_group,
                "grouped router: need n_group | E and 1 <= topk_group <= n_group");
  const int lpg = E / n_group / 4;
  FLYAI_REQUIRE(n_group == 1 || n_group <= topk_group ||
                    ((E / n_group) % 4 == 0 && lpg >= 1 && (lpg & (lpg - 1)) == 0),
                "grouped router: a group must be 4 * 2^j experts");
  FLYAI_REQUIRE(n_group == 1 || n_group <= topk_group || topk_group * (E / n_group) >= k,
                "grouped router: kept groups hold fewer than k experts");
  FLYAI_REQUIRE(x && w && logits && topk_ids && topk_w, "grouped router: null pointer");
  return launch_router_grouped(x, w, e_bias, T, H, E, n_group, topk_group, k, route_scale, logits,
                               topk_ids, topk_w, as_stream(stream));
}
