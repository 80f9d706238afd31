// Layer glue: RMSNorm, bf16 projections with bias (+ residual), RoPE + KV append.
#include <mutex>
#include <type_traits>

#include "common.h"

namespace flyai {

// ---- RMSNorm: y = bf16(w * (x * rsqrt(mean(x^2) + eps))), fp32 weight --------------------------
// (kRowThreads, block_sum_1024 and rmsnorm_row: common.h)
__global__ __launch_bounds__(kRowThreads) void rmsnorm_kernel(const uint16_t* __restrict__ x,
                                                              const float* __restrict__ w, int H,
                                                              float eps, uint16_t* __restrict__ y) {
  rmsnorm_row(x, w, H, eps, y, blockIdx.x);
}

int launch_rmsnorm(const uint16_t* x, const float* w, int T, int H, float eps, uint16_t* y,
                   hipStream_t s) {
  if (T == 0) return FLYAI_OK;
  hipLaunchKernelGGL(rmsnorm_kernel, dim3(T), dim3(kRowThreads), 0, s, x, w, H, eps, y);
  return check_launch("rmsnorm");
}

// ---- bf16 projections: split-K partial GEMM + fused finalize kernels -------------------------------
// gemm_splitk: workgroup = 4 waves on 4 consecutive 16-feature tiles and one K slice of kKQW groups
// of 128.  MFMA step j of group q takes, in lane (r, g), K = 128q + 32j + 8g .. +7 for both operands
// (any K order shared by the two operands is valid), so each weight load instruction reads one
// whole 64-byte run of each of its 16 rows.  The activation slice (64 rows x 512 K, bf16) is staged once in LDS; each wave issues all
// of its weight loads for the slice before its first MFMA (a single HBM round trip per wave) and
// writes fp32 partial sums part[slice][row][feature].  A finalize kernel adds the slices in slice
// order (so the result is independent of timing), the bias, and the fused epilogue.
constexpr int kKQW = 4;       // K groups of 128 per slice
constexpr int kGemmRows = 64; // activation rows per pass

__global__ __launch_bounds__(256) void gemm_splitk_bf16_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ W, int M, int N, int K,
    float* __restrict__ part) {
  __shared__ uint4 as[kGemmRows][kKQW * 16 + 1];  // 64 rows x 512 bf16, +16 B per row vs bank conflicts
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 15, g = lane >> 4;
  const int nt = blockIdx.x * 4 + wave;
  const int slice = blockIdx.y;
  const int KQ = (K + 127) / 128;
  const int kq0 = slice * kKQW;
  const int nkq = min(kKQW, KQ - kq0);
  const bool nval = nt * 16 < N;
  const int feat = nt * 16 + r;
  typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
  if (M <= kGemmRows) {
    // One pass (decode-sized M): the activation slice's loads go out first, then the weights, so the
    // LDS stores wait only for the activations (loads complete in issue order) and the L2 round trip
    // for them overlaps the HBM fetch of the weights; the barrier then waits on LDS only.
    constexpr int kPer = kGemmRows * kKQW * 16 / 256;  // 16-byte vectors per thread
    u32x4 av[kPer];
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const int i = j * 256 + (int)threadIdx.x;
      const int row = i / (kKQW * 16), v = i % (kKQW * 16);
      const int k = 128 * kq0 + 8 * v;
      const bool ok = row < M && k < K;
      av[j] = ok ? *reinterpret_cast<const u32x4*>(x + (size_t)row * K + k) : u32x4{0u, 0u, 0u, 0u};
    }
    asm volatile("" ::: "memory");  // keep the activation loads ahead of the weight loads
    uint4 wv[kKQW][4];
#pragma unroll
    for (int q = 0; q < kKQW; ++q) {
      const int kb = 128 * (kq0 + q);
      const bool ok = nval && q < nkq;
#pragma unroll
      for (int j = 0; j < 4; ++j)  // step j reads K kb + 32j .. +31 (K % 32 == 0)
        wv[q][j] = ok && kb + 32 * j < K ? reinterpret_cast<const uint4*>(W + (size_t)feat * K + kb)[4 * j + g]
                                         : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const int i = j * 256 + (int)threadIdx.x;
      *reinterpret_cast<u32x4*>(&as[i / (kKQW * 16)][i % (kKQW * 16)]) = av[j];
    }
    lds_barrier();
    if (!nval) return;
    const int mt_count = (M + 15) / 16;
    f32x4_t acc[4] = {f32x4_t{0.f, 0.f, 0.f, 0.f}, f32x4_t{0.f, 0.f, 0.f, 0.f},
                      f32x4_t{0.f, 0.f, 0.f, 0.f}, f32x4_t{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
    for (int q = 0; q < kKQW; ++q) {
      if (q >= nkq) break;
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        if (m >= mt_count) break;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint4 av4 = as[16 * m + r][q * 16 + 4 * j + g];
          acc[m] = mfma16x16x32(as_bf16x8(av4), as_bf16x8(wv[q][j]), acc[m]);
        }
      }
    }
    float* pp = part + (size_t)slice * M * N;
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      if (m >= mt_count) break;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int row = 16 * m + 4 * g + v;
        if (row < M) pp[(size_t)row * N + feat] = acc[m][v];
      }
    }
    return;
  }
  // weights for the whole slice, issued up front (reused by every pass of 64 rows)
  uint4 wv[kKQW][4];
#pragma unroll
  for (int q = 0; q < kKQW; ++q) {
    const int kb = 128 * (kq0 + q);
    const bool ok = nval && q < nkq;
#pragma unroll
    for (int j = 0; j < 4; ++j)  // step j reads K kb + 32j .. +31 (K % 32 == 0)
      wv[q][j] = ok && kb + 32 * j < K ? reinterpret_cast<const uint4*>(W + (size_t)feat * K + kb)[4 * j + g]
                                       : make_uint4(0, 0, 0, 0);
  }
  for (int m0 = 0; m0 < M; m0 += kGemmRows) {
    const int rows = min(kGemmRows, M - m0);
    __syncthreads();
    // the slice of A goes to LDS with loads batched 8 per thread (one round trip per batch);
    // rows past the pass and K past the row end are stored as zero
    for (int b0 = 0; b0 < kGemmRows * kKQW * 16; b0 += 8 * 256) {
      u32x4 v8[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int i = b0 + j * 256 + (int)threadIdx.x;
        const int row = i / (kKQW * 16), v = i % (kKQW * 16);
        const int k = 128 * kq0 + 8 * v;
        const bool ok = row < rows && k < K;
        const u32x4 val = *reinterpret_cast<const u32x4*>(x + (ok ? (size_t)(m0 + row) * K + k : 0));
        v8[j] = ok ? val : u32x4{0u, 0u, 0u, 0u};
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int i = b0 + j * 256 + (int)threadIdx.x;
        *reinterpret_cast<u32x4*>(&as[i / (kKQW * 16)][i % (kKQW * 16)]) = v8[j];
      }
    }
    __syncthreads();
    if (!nval) continue;
    const int mt_count = (rows + 15) / 16;
    f32x4_t acc[4] = {f32x4_t{0.f, 0.f, 0.f, 0.f}, f32x4_t{0.f, 0.f, 0.f, 0.f},
                      f32x4_t{0.f, 0.f, 0.f, 0.f}, f32x4_t{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
    for (int q = 0; q < kKQW; ++q) {
      if (q >= nkq) break;
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        if (m >= mt_count) break;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint4 av = as[16 * m + r][q * 16 + 4 * j + g];
          acc[m] = mfma16x16x32(as_bf16x8(av), as_bf16x8(wv[q][j]), acc[m]);
        }
      }
    }
    float* pp = part + (size_t)slice * M * N;
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      if (m >= mt_count) break;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int row = m0 + 16 * m + 4 * g + v;
        if (row < M) pp[(size_t)row * N + feat] = acc[m][v];
      }
    }
  }
}

constexpr int kMaxSlices = 16;  // K <= 8192

// Sum of the split-K partials in slice order; all loads are issued before the first add.
__device__ __forceinline__ float sum_slices(const float* __restrict__ part, int slices, size_t stride,
                                            size_t idx) {
  float v[kMaxSlices];
#pragma unroll
  for (int i = 0; i < kMaxSlices; ++i) v[i] = i < slices ? part[i * stride + idx] : 0.f;
  float s = v[0];
#pragma unroll
  for (int i = 1; i < kMaxSlices; ++i)
    if (i < slices) s += v[i];
  return s;
}

// The thread's ITERS columns (tid + kRowThreads * it) of token row t: the split-K slices summed in
// slice order, + bias, rounded, + the residual, rounded (the sum_slices order).  Every load of the
// first SMAX slices, the bias, the residual and the norm weight is issued before the first add, so
// the row costs one memory round trip instead of one per column; slices past SMAX, if any, are
// added afterwards in order.  Columns past H are clamped for the loads and left out of ss.
template <int ITERS, int SMAX>
__device__ __forceinline__ void row_residual(const float* __restrict__ part, int slices, size_t stride,
                                             const uint16_t* __restrict__ b, const uint16_t* __restrict__ h_in,
                                             const float* __restrict__ lnw, int t, int H,
                                             uint16_t (&hv)[ITERS], float (&lw)[ITERS], float& ss) {
  const int tid = threadIdx.x;
  float pv[ITERS][SMAX], bv[ITERS], hp[ITERS];
#pragma unroll
  for (int it = 0; it < ITERS; ++it) {
    const int i = min(tid + it * kRowThreads, H - 1);
    const size_t idx = (size_t)t * H + i;
#pragma unroll
    for (int q = 0; q < SMAX; ++q) pv[it][q] = part[(size_t)min(q, slices - 1) * stride + idx];
    bv[it] = b ? bf2f(b[i]) : 0.f;
    hp[it] = bf2f(h_in[idx]);
    lw[it] = lnw[i];
  }
  ss = 0.f;
#pragma unroll
  for (int it = 0; it < ITERS; ++it) {
    const int i = tid + it * kRowThreads;
    const size_t idx = (size_t)t * H + min(i, H - 1);
    float o = pv[it][0];
#pragma unroll
    for (int q = 1; q < SMAX; ++q)
      if (q < slices) o += pv[it][q];
    for (int q = SMAX; q < slices; ++q) o += part[(size_t)q * stride + idx];
    hv[it] = f2bf(hp[it] + bf16_round(o + bv[it]));
    const float hf = bf2f(hv[it]);
    if (i < H) ss = fmaf(hf, hf, ss);
  }
}

// y = bf16(sum + b); with residual: residual <- bf16(residual + y)
__global__ __launch_bounds__(256) void linear_finalize_kernel(const float* __restrict__ part, int slices,
                                                              const uint16_t* __restrict__ b, int M,
                                                              int N, uint16_t* __restrict__ y,
                                                              uint16_t* __restrict__ residual) {
  const size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (size_t)M * N) return;
  const int f = idx % N;
  const float o = bf16_round(sum_slices(part, slices, (size_t)M * N, idx) + (b ? bf2f(b[f]) : 0.f));
  if (residual) residual[idx] = f2bf(bf2f(residual[idx]) + o);
  else y[idx] = f2bf(o);
}

// o_proj epilogue fused with the post-attention RMSNorm: h <- bf16(h + bf16(sum + b)),
// xn = bf16(w * (h * rsqrt(mean(h^2) + eps))).  One workgroup per token row.
template <int ITERS, int SMAX>
__global__ __launch_bounds__(kRowThreads) void residual_rmsnorm_finalize_kernel(
    const float* __restrict__ part, int slices, const uint16_t* __restrict__ b, int M, int H,
    uint16_t* __restrict__ h, const float* __restrict__ lnw, float eps, uint16_t* __restrict__ xn) {
  __shared__ float red[kRowThreads / 64];
  const int t = blockIdx.x, tid = threadIdx.x;
  uint16_t hv[ITERS];
  float lw[ITERS], ss;
  row_residual<ITERS, SMAX>(part, slices, (size_t)M * H, b, h, lnw, t, H, hv, lw, ss);
#pragma unroll
  for (int it = 0; it < ITERS; ++it) {
    const int i = tid + it * kRowThreads;
    if (i < H) h[(size_t)t * H + i] = hv[it];
  }
  const float rr = rsqrtf(block_sum_1024(ss, red) / (float)H + eps);
#pragma unroll
  for (int it = 0; it < ITERS; ++it) {
    const int i = tid + it * kRowThreads;
    if (i < H) xn[(size_t)t * H + i] = f2bf(lw[it] * (bf2f(hv[it]) * rr));
  }
}

// Residual + RMSNorm finalize fused with the GPT-OSS router logits of the same token (decode-sized
// batches).  Grid (T, kRouteSplit): every workgroup of a token computes the finalize (the new
// residual stream goes to h_out, never in place, since all of them read h_in; workgroup 0 writes it
// and xn), keeps xn in LDS and computes the logits of its E/kRouteSplit experts with exactly the
// fixed order of router_logits_kernel (lane l sums k = 512 j + 8 l + i in order, then a xor
// butterfly 32..1; bf16(dot + bias)).  The top-k follows in the next kernel: workgroups of one
// kernel never exchange data (a device-scope fence would write back the L2).
constexpr int kRouteSplit = 4;

template <int JMAX, int SMAX>
__global__ __launch_bounds__(kRowThreads) void residual_rmsnorm_logits_kernel(
    const float* __restrict__ part, int slices, const uint16_t* __restrict__ b, int M, int H,
    const uint16_t* __restrict__ h_in, uint16_t* __restrict__ h_out, const float* __restrict__ lnw,
    float eps, uint16_t* __restrict__ xn, const uint16_t* __restrict__ rw,
    const uint16_t* __restrict__ rb, int E, float* __restrict__ logits) {
  __shared__ float red[kRowThreads / 64];
  __shared__ __align__(16) uint16_t xs[JMAX * 512];
  const int t = blockIdx.x, split = blockIdx.y, tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int per = (E + kRouteSplit - 1) / kRouteSplit;
  const int e_lo = split * per, e_hi = min(E, e_lo + per);
  constexpr int kBatch = JMAX <= 6 ? 2 : 1;  // experts per wave in flight
  // the first batch of router weights does not depend on xn: issue it before the finalize
  uint4 wv[kBatch][JMAX];
  auto load_batch = [&](int e0) __attribute__((always_inline)) {
#pragma unroll
    for (int c = 0; c < kBatch; ++c)
#pragma unroll
      for (int j = 0; j < JMAX; ++j) {
        const int k0 = 512 * j + 8 * lane;
        wv[c][j] = (e0 + c < e_hi && k0 < H) ? *reinterpret_cast<const uint4*>(rw + (size_t)(e0 + c) * H + k0)
                                             : make_uint4(0, 0, 0, 0);
      }
  };
  load_batch(e_lo + wave * kBatch);
  constexpr int kIters = (JMAX * 512 + kRowThreads - 1) / kRowThreads;  // columns per thread
  uint16_t hv[kIters];
  float lw[kIters], ss;
  row_residual<kIters, SMAX>(part, slices, (size_t)M * H, b, h_in, lnw, t, H, hv, lw, ss);
#pragma unroll
  for (int it = 0; it < kIters; ++it) {
    const int i = tid + it * kRowThreads;
    if (i < H && split == 0) h_out[(size_t)t * H + i] = hv[it];
  }
  const float rr = rsqrtf(block_sum_1024(ss, red) / (float)H + eps);
#pragma unroll
  for (int it = 0; it < kIters; ++it) {
    const int i = tid + it * kRowThreads;
    if (i < H) {
      const uint16_t v = f2bf(lw[it] * (bf2f(hv[it]) * rr));
      if (split == 0) xn[(size_t)t * H + i] = v;
      xs[i] = v;
    }
  }
  __syncthreads();
  for (int e0 = e_lo + wave * kBatch; e0 < e_hi; e0 += (kRowThreads / 64) * kBatch) {
    if (e0 != e_lo + wave * kBatch) load_batch(e0);
    float acc[kBatch] = {};
#pragma unroll
    for (int j = 0; j < JMAX; ++j) {
      const int k0 = 512 * j + 8 * lane;
      if (k0 >= H) break;  // lanes past the row end keep their partial unchanged
      const uint4 xv = *reinterpret_cast<const uint4*>(xs + k0);
      const uint32_t xw[4] = {xv.x, xv.y, xv.z, xv.w};
#pragma unroll
      for (int c = 0; c < kBatch; ++c) {
        const uint32_t ww[4] = {wv[c][j].x, wv[c][j].y, wv[c][j].z, wv[c][j].w};
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const float xf = __uint_as_float((i & 1) ? (xw[i >> 1] & 0xffff0000u) : (xw[i >> 1] << 16));
          const float wf = __uint_as_float((i & 1) ? (ww[i >> 1] & 0xffff0000u) : (ww[i >> 1] << 16));
          acc[c] = fmaf(xf, wf, acc[c]);  // exact product: fma == mul + add
        }
      }
    }
    // the butterfly's additions as a reduce-scatter over the kBatch sums: lane l ends with l >> shift
    const float v = wave_sum_scatter<kBatch>(acc);
    constexpr int shift = wave_sum_scatter_shift<kBatch>();
    const int c = lane >> shift;
    if ((lane & ((1 << shift) - 1)) == 0 && e0 + c < e_hi)
      logits[(size_t)t * E + e0 + c] = bf16_round(v + bf2f(rb[e0 + c]));
  }
}

// ---- prefill-sized projections: a tiled GEMM with the split-K kernel's per-element arithmetic ------
// For many rows the split-K kernel re-stages its activation slice once per 64-row pass and leaves
// gemm_slices(K) fp32 partial planes for the finalizers.  This kernel tiles M x N instead: a
// workgroup of 4 waves (2 x 2) owns 128 rows x 128 features, each wave 64 x 64 (4 x 4 MFMA tiles).
// Per 128-K group the activation and weight tiles are staged in LDS in MFMA-fragment order (tile t,
// step j: one KiB, lane (r, g) holding row/feature 16t + r, K 32j + 8g .. +7), so every fragment read
// is a lane-contiguous ds_read_b128; the next group's global loads are in flight during the current
// group's MFMAs.  Arithmetic per output element is exactly the split-K kernel's: the same MFMA with
// the same K-to-lane mapping (activations as A, weights as B), each 512-K slice accumulated from zero
// in (group, step) order, and the slices added left to right in fp32 -- so the one folded plane it
// writes equals sum_slices of the split-K planes bit for bit, and a row's result does not depend on
// which kernel the batch size chose.
constexpr int kTileM = 128, kTileN = 128;
constexpr int kTiledWaves = 8;      // 4 (rows) x 2 (features), each wave 32 rows x 64 features
constexpr int kTiledMinRows = 256;  // batches of at least this many rows take the tiled kernel

__global__ __launch_bounds__(64 * kTiledWaves) void gemm_tiled_bf16_kernel(const uint16_t* __restrict__ x,
                                                                           const uint16_t* __restrict__ W,
                                                                           int M, int N, int K,
                                                                           float* __restrict__ out) {
  typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
  __shared__ u32x4 as[kTileM / 16][4][64];  // [row tile][step][lane]
  __shared__ u32x4 ws[kTileN / 16][4][64];  // [feature tile][step][lane]
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int m0 = blockIdx.y * kTileM, n0 = blockIdx.x * kTileN;
  const int wm = wave >> 1, wn = wave & 1;  // the wave's 32 x 64 block: row tiles 2wm, 2wm+1
  const int KG = (K + 127) / 128;
  // staging: each wave fills whole fragment slabs (tile t, step j) -- slab u = 4 wave + i (i < 4) of
  // each operand is tile u / 4, step u % 4 -- so its 64 LDS stores are one contiguous KiB (no bank
  // conflicts); lane (r, g) loads row/feature 16t + r, K 128q + 32j + 8g .. +7
  constexpr int kSlabs = 32 / kTiledWaves;
  const int sr = lane & 15, sg = lane >> 4;
  u32x4 ra[kSlabs], rw[kSlabs];
  auto load_group = [&](int q) {
#pragma unroll
    for (int i = 0; i < kSlabs; ++i) {
      const int u = kSlabs * wave + i, t = u >> 2, j = u & 3;
      const int k = 128 * q + 32 * j + 8 * sg;
      const int row = m0 + 16 * t + sr, feat = n0 + 16 * t + sr;
      ra[i] = (row < M && k < K) ? *reinterpret_cast<const u32x4*>(x + (size_t)row * K + k) : u32x4{0u, 0u, 0u, 0u};
      rw[i] = (feat < N && k < K) ? *reinterpret_cast<const u32x4*>(W + (size_t)feat * K + k) : u32x4{0u, 0u, 0u, 0u};
    }
  };
  auto store_group = [&]() {
#pragma unroll
    for (int i = 0; i < kSlabs; ++i) {
      const int u = kSlabs * wave + i;
      as[u >> 2][u & 3][lane] = ra[i];
      ws[u >> 2][u & 3][lane] = rw[i];
    }
  };
  f32x4_t acc[2][4], tot[2][4];
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      acc[a][b] = f32x4_t{0.f, 0.f, 0.f, 0.f};
      tot[a][b] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    }
  load_group(0);
  for (int q = 0; q < KG; ++q) {
    lds_barrier();  // every wave is done with the previous group's tiles
    store_group();
    if (q + 1 < KG) load_group(q + 1);
    lds_barrier();
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      bf16x8_t af[2], bw[4];
#pragma unroll
      for (int t = 0; t < 2; ++t) af[t] = __builtin_bit_cast(bf16x8_t, as[2 * wm + t][j][lane]);
#pragma unroll
      for (int t = 0; t < 4; ++t) bw[t] = __builtin_bit_cast(bf16x8_t, ws[4 * wn + t][j][lane]);
#pragma unroll
      for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int b = 0; b < 4; ++b) acc[a][b] = mfma16x16x32(af[a], bw[b], acc[a][b]);
    }
    if ((q % kKQW) == kKQW - 1 || q == KG - 1) {  // the end of a 512-K slice: fold it, in slice order
      const bool first = q < kKQW;
#pragma unroll
      for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int b = 0; b < 4; ++b) {
          tot[a][b] = first ? acc[a][b] : tot[a][b] + acc[a][b];
          acc[a][b] = f32x4_t{0.f, 0.f, 0.f, 0.f};
        }
    }
  }
  // lane (r, g) holds rows 16(2wm + a) + 4g + v of feature 16(4wn + b) + r
  const int r = lane & 15, g = lane >> 4;
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const int feat = n0 + 16 * (4 * wn + b) + r;
      if (feat >= N) continue;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int row = m0 + 16 * (2 * wm + a) + 4 * g + v;
        if (row < M) out[(size_t)row * N + feat] = tot[a][b][v];
      }
    }
}

// The tiled GEMM for K % 64 == 0 (every projection of both models): the same 128 x 128 workgroup
// tile, 8 waves of 32 rows x 64 features and per-element arithmetic, but the operand tiles go
// global -> LDS directly (global_load_lds, no register staging) through 4 stages of one 64-K group
// each (A and B: 8 row tiles of 2 KiB per stage, 4 load instructions per wave, each reading whole
// 128-byte rows), a group's loads issued 3 groups ahead.  The stages (A and B apart) are separate
// LDS arrays with compile-time stage numbers, so the compiler can tell a stage's reads from the DMA
// writes into the others; each stage is
// waited for with an explicit vmcnt that leaves the 2 younger groups' loads in flight (vector
// memory loads complete in issue order), then one barrier per group, which also tells the waves
// that the stage just read can be refilled.  The next group's step-0 fragments are read under the
// current group's step-1 MFMAs.  A group is 2 MFMA steps of 32 K; step j of 64-K group q is step
// 2 (q % 2) + j of the split-K kernel's 128-K group q / 2, so the K-to-lane mapping, each slice's
// MFMA chain and the slice-ordered fold are the split-K kernel's, bit for bit.  The group loop is
// unrolled by one 512-K slice (8 groups, twice round the stages), so the fold sits at a fixed place
// and no group carries a branch.  Rows and features past M / N load clamped rows and are never
// stored; the groups issued past the end read the last group and are never computed on.
constexpr int kTlStages = 4;
constexpr int kTlStageBytes = 32 * 1024;  // A and B halves: 8 row tiles x 16 rows x 128 B each
constexpr int kTlLoads = 4;               // load instructions per wave per group
constexpr int kTlGroupsPerSlice = 8;      // 64-K groups per 512-K slice

// The qkv projection's finalize, fused into the tiled GEMM's epilogue (head_dim 64, no tree): the
// qkv_rope_kv_vec_kernel arithmetic on the folded sums -- x = bf16(sum + bias), then q and k rotated
// (first = x1 c - x2 s, second = x2 c + x1 s, each product and sum rounded to bf16) -- q written to
// q_out and k / v to the token's slab slot.  A wave's 64 features are one whole head and lane
// (r, g) holds dims 16b + r of tiles b = 0..3, so each rotation pair (d, d + 32) sits in one lane.
struct QkvEpilogue {
  const uint16_t* bias;
  const int32_t* positions;
  const int32_t* seq_id;
  const uint16_t* cos_tab;
  const uint16_t* sin_tab;
  const int64_t* kv_base;
  const int32_t* kv_cap;
  uint16_t* q_out;
  uint16_t* k_pool;
  uint16_t* v_pool;
  int rope_positions, Hq, Hkv;
};

template <bool QKV>
__global__ __launch_bounds__(64 * kTiledWaves) void gemm_tiled_lds_kernel(const uint16_t* __restrict__ x,
                                                                          const uint16_t* __restrict__ W,
                                                                          int M, int N, int K,
                                                                          float* __restrict__ out,
                                                                          QkvEpilogue ep) {
  typedef __attribute__((address_space(3))) void* lds_ptr;
  // per stage: the A fragment blocks and the B fragment blocks as separate arrays
  __shared__ __align__(1024) char sa0[kTlStageBytes / 2], sb0[kTlStageBytes / 2];
  __shared__ __align__(1024) char sa1[kTlStageBytes / 2], sb1[kTlStageBytes / 2];
  __shared__ __align__(1024) char sa2[kTlStageBytes / 2], sb2[kTlStageBytes / 2];
  __shared__ __align__(1024) char sa3[kTlStageBytes / 2], sb3[kTlStageBytes / 2];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  // XCD-aware tile order: workgroup b runs on XCD b % 8, and XCD x takes tiles x * per .. x * per +
  // per - 1 of the row-fastest order (a band of whole feature columns), so the workgroups that share
  // an XCD's L2 share their weight tiles and the activation rows; without it the output projection
  // (23 feature tiles) read about 11x its operand bytes from HBM
  const int gm_ = (M + kTileM - 1) / kTileM, gn_ = (N + kTileN - 1) / kTileN;
  const int per = (gm_ * gn_ + 7) / 8;
  const int tile = (int)(blockIdx.x % 8) * per + (int)(blockIdx.x / 8);
  if (tile >= gm_ * gn_) return;
  const int m0 = (tile % gm_) * kTileM, n0 = (tile / gm_) * kTileN;
  const int wm = wave >> 1, wn = wave & 1;  // the wave's 32 x 64 block: row tiles 2wm, 2wm+1
  const int KG = K / 64;
  // LDS: a 16-row tile of a 64-K group is 2 KiB, row-major (128 B per row), its eight 16-byte chunks
  // XOR-swizzled by row: chunk c of row rr sits at position c ^ swz(rr), swz(rr) = (rr / 2) % 8.
  // A load instruction fills half a tile (8 whole rows): lane L writes position L % 8 of row L / 8
  // (the DMA's fixed lane order), so it reads chunk (L % 8) ^ swz of that row -- 8 consecutive lanes
  // read one row's 128 contiguous bytes (a fragment-order load, 16 rows x 64 B per instruction,
  // streams from L2 at a third of the rate).  Instruction u = 4 wave + i: u < 16: A half-tile u
  // (tile u / 2, rows 8 (u % 2) ..), else B half-tile u - 16.
  const int r = lane & 15, g = lane >> 4;
  const uint16_t* src[kTlLoads];
#pragma unroll
  for (int i = 0; i < kTlLoads; ++i) {
    const int u = kTlLoads * wave + i, ub = u & 15, t = ub >> 1;
    const int rr = 8 * (ub & 1) + (lane >> 3), chunk = (lane & 7) ^ ((rr >> 1) & 7);
    const bool is_a = u < 16;
    const int row = is_a ? min(m0 + 16 * t + rr, M - 1) : min(n0 + 16 * t + rr, N - 1);
    src[i] = (is_a ? x : W) + (size_t)row * K + 8 * chunk;
  }
  // the MFMA fragment of step j, lane (r, g): row r, K 32j + 8g .. +7 = chunk 4j + g, read from its
  // swizzled position (step 1's chunk is step 0's with bit 2 flipped)
  const int frag0 = r * 128 + ((g ^ ((r >> 1) & 7)) << 4);
  // waves 0-3 fill the A blocks, waves 4-7 the B blocks (wave-uniform)
  auto issue = [&](char* sa, char* sb, int q) __attribute__((always_inline)) {
    const size_t koff = (size_t)min(q, KG - 1) * 64;
    char* dst = wave < 4 ? sa + kTlLoads * wave * 1024 : sb + kTlLoads * (wave - 4) * 1024;
#pragma unroll
    for (int i = 0; i < kTlLoads; ++i)
      __builtin_amdgcn_global_load_lds((const void*)(src[i] + koff), (lds_ptr)(dst + i * 1024), 16, 0, 0);
  };
  // tot starts at -0: -0 + x == x for every x (also -0), so the first fold copies the first slice's
  // sums bit for bit, as the split-K finalizer's first plane
  f32x4_t acc[2][4], tot[2][4];
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      acc[a][b] = f32x4_t{0.f, 0.f, 0.f, 0.f};
      tot[a][b] = f32x4_t{-0.f, -0.f, -0.f, -0.f};
    }
  auto fold = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        tot[a][b] += acc[a][b];
        acc[a][b] = f32x4_t{0.f, 0.f, 0.f, 0.f};
      }
  };
  bf16x8_t a0[2], a1[2], b0[4], b1[4];
  auto read_ab = [&](bf16x8_t (&af)[2], bf16x8_t (&bw)[4], const char* sa, const char* sb, int j) __attribute__((always_inline)) {
    const int fo = frag0 ^ (j << 6);
#pragma unroll
    for (int t = 0; t < 2; ++t) af[t] = as_bf16x8(*reinterpret_cast<const uint4*>(sa + (2 * wm + t) * 2048 + fo));
#pragma unroll
    for (int t = 0; t < 4; ++t) bw[t] = as_bf16x8(*reinterpret_cast<const uint4*>(sb + (4 * wn + t) * 2048 + fo));
  };
  auto mfma_step = [&](const bf16x8_t (&af)[2], const bf16x8_t (&bw)[4]) __attribute__((always_inline)) {
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
      for (int b = 0; b < 4; ++b) acc[a][b] = mfma16x16x32(af[a], bw[b], acc[a][b]);
  };
  // group q from stage (ca, cb) (its step-0 fragments already in a0 / b0); hands over to (na, nb) and
  // refills (ca, cb) with group q + 4
  auto group = [&](char* ca, char* cb, const char* na, const char* nb, int q) __attribute__((always_inline)) {
    read_ab(a1, b1, ca, cb, 1);
    mfma_step(a0, b0);
    __builtin_amdgcn_s_waitcnt(waitcnt_vm((kTlStages - 2) * kTlLoads));  // this wave's part of the next stage landed
    lds_barrier();  // every wave's part of the next stage is in LDS; every wave is done reading this one
    read_ab(a0, b0, na, nb, 0);
    mfma_step(a1, b1);
    issue(ca, cb, q + kTlStages);
  };
  // QKV: the epilogue's per-row data is fetched under the GEMM instead of after it (it took two
  // dependent round trips per workgroup at the end, with nothing else on the CU to hide them).
  // Lane L of wave w fetches row 16 w + L / 4 of the tile: its position and sequence before the
  // prologue (so the first stage wait covers them), then the row's cos / sin (64 bytes each, 16 per
  // lane, global -> LDS) and slab geometry once they have landed.  The epilogue reads all of it
  // from LDS.  (These extra loads only make the later stage waits stricter, never looser.)
  __shared__ __align__(16) uint16_t rot_c[QKV ? kTileM * 32 : 1], rot_s[QKV ? kTileM * 32 : 1];
  __shared__ int row_pos[QKV ? kTileM : 1], row_cap[QKV ? kTileM : 1];
  __shared__ int64_t row_base[QKV ? kTileM : 1];
  const int erow = 16 * wave + (lane >> 2);  // the tile row this lane fetches for
  int e_pos = 0, e_sq = 0;
  float bv[4];
  if constexpr (QKV) {
    const int t = min(m0 + erow, M - 1);
    e_pos = ep.positions[t];
    e_sq = ep.seq_id[t];
    const int fb = min(n0 + 64 * wn, N - 64);
#pragma unroll
    for (int b = 0; b < 4; ++b) bv[b] = ep.bias ? bf2f(ep.bias[fb + 16 * b + r]) : 0.f;
  }
  // the stage waits count loads per group in issue order: no load may move across a group
  asm volatile("" ::: "memory");
  issue(sa0, sb0, 0);
  asm volatile("" ::: "memory");
  issue(sa1, sb1, 1);
  asm volatile("" ::: "memory");
  issue(sa2, sb2, 2);
  asm volatile("" ::: "memory");
  issue(sa3, sb3, 3);
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(waitcnt_vm((kTlStages - 1) * kTlLoads));
  lds_barrier();  // stage 0 is in LDS
  int e_cap = 0;
  int64_t e_base = 0;
  if constexpr (QKV) {
    // e_pos / e_sq landed with stage 0 (issued before it)
    const int pc = min(max(e_pos, 0), ep.rope_positions - 1);
    const size_t roff = (size_t)pc * 32 + 8 * (lane & 3);
    __builtin_amdgcn_global_load_lds((const void*)(ep.cos_tab + roff), (lds_ptr)(rot_c + 16 * wave * 32), 16, 0, 0);
    __builtin_amdgcn_global_load_lds((const void*)(ep.sin_tab + roff), (lds_ptr)(rot_s + 16 * wave * 32), 16, 0, 0);
    e_cap = ep.kv_cap[e_sq];
    e_base = ep.kv_base[e_sq];
    asm volatile("" ::: "memory");
  }
  read_ab(a0, b0, sa0, sb0, 0);
  // whole 512-K slices (8 groups, two turns of the 4 stages), each folded after its last group
  const int full = KG / kTlGroupsPerSlice;
  for (int sl = 0; sl < full; ++sl) {
    const int q = sl * kTlGroupsPerSlice;
    group(sa0, sb0, sa1, sb1, q);
    group(sa1, sb1, sa2, sb2, q + 1);
    group(sa2, sb2, sa3, sb3, q + 2);
    group(sa3, sb3, sa0, sb0, q + 3);
    group(sa0, sb0, sa1, sb1, q + 4);
    group(sa1, sb1, sa2, sb2, q + 5);
    group(sa2, sb2, sa3, sb3, q + 6);
    group(sa3, sb3, sa0, sb0, q + 7);
    fold();
  }
  // the last, partial slice (its first group sits on stage 0)
  const int rem = KG - full * kTlGroupsPerSlice, q = full * kTlGroupsPerSlice;
  if (rem > 0) {
    group(sa0, sb0, sa1, sb1, q);
    if (rem > 1) group(sa1, sb1, sa2, sb2, q + 1);
    if (rem > 2) group(sa2, sb2, sa3, sb3, q + 2);
    if (rem > 3) group(sa3, sb3, sa0, sb0, q + 3);
    if (rem > 4) group(sa0, sb0, sa1, sb1, q + 4);
    if (rem > 5) group(sa1, sb1, sa2, sb2, q + 5);
    if (rem > 6) group(sa2, sb2, sa3, sb3, q + 6);
    fold();
  }
  __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));  // the loads issued past the end have landed
  // lane (r, g) holds rows 16(2wm + a) + 4g + v of feature 16(4wn + b) + r
  if constexpr (!QKV) {
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const int feat = n0 + 16 * (4 * wn + b) + r;
        if (feat >= N) continue;
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int row = m0 + 16 * (2 * wm + a) + 4 * g + v;
          if (row < M) out[(size_t)row * N + feat] = tot[a][b][v];
        }
      }
  } else {
    // every lane's fetched row data to LDS (the rotary rows are there already: vmcnt(0) above)
    if ((lane & 3) == 0) {
      row_pos[erow] = e_pos;
      row_cap[erow] = e_cap;
      row_base[erow] = e_base;
    }
    lds_barrier();
    const int fb = n0 + 64 * wn;  // the wave's head: q heads, then k heads, then v heads
    if (fb >= N) return;
    const int hd = fb / 64;
    const bool rotated = hd < ep.Hq + ep.Hkv;
    int pos[2][4], cap[2][4];
    int64_t base[2][4];
    float cs[2][4][2], sn[2][4][2];
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int tr = 16 * (2 * wm + a) + 4 * g + v;
        pos[a][v] = row_pos[tr];
        cap[a][v] = row_cap[tr];
        base[a][v] = row_base[tr];
#pragma unroll
        for (int b = 0; b < 2; ++b) {
          cs[a][v][b] = bf2f(rot_c[tr * 32 + 16 * b + r]);
          sn[a][v][b] = bf2f(rot_s[tr * 32 + 16 * b + r]);
        }
      }
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int t = m0 + 16 * (2 * wm + a) + 4 * g + v;
        const int p = pos[a][v];
        // rows past M, and positions outside the rotary table, write nothing
        if (t >= M || p < 0 || p >= ep.rope_positions) continue;
        const bool in_cap = p < cap[a][v];
        float xv[4];
#pragma unroll
        for (int b = 0; b < 4; ++b) xv[b] = bf16_round(tot[a][b][v] + bv[b]);
        if (rotated) {
          if (hd >= ep.Hq && !in_cap) continue;
          uint16_t* kh = ep.k_pool + base[a][v] + (size_t)(hd - ep.Hq) * cap[a][v] * 64;
#pragma unroll
          for (int b = 0; b < 2; ++b) {
            const int d = 16 * b + r;
            const float c = cs[a][v][b], s_ = sn[a][v][b];
            const float x1 = xv[b], x2 = xv[b + 2];
            const uint32_t first = f2bf(bf16_round(bf16_round(x1 * c) - bf16_round(x2 * s_)));
            const uint32_t second = f2bf(bf16_round(bf16_round(x2 * c) + bf16_round(x1 * s_)));
            // dims d and d + 1 sit in lanes r and r ^ 1 of the same row (both active or both not):
            // the even lane stores the pair as one dword (q rows and the K slab keep them adjacent)
            const uint32_t pair = __builtin_amdgcn_update_dpp(0, (int)(first | (second << 16)), 0xB1, 0xF, 0xF, false);
            if (r & 1) continue;
            const uint32_t lo = first | (pair << 16), hi = second | (pair & 0xffff0000u);
            uint16_t* d1 = hd < ep.Hq ? ep.q_out + ((size_t)t * ep.Hq + hd) * 64 + d : kh + kv_k_off(p, d);
            uint16_t* d2 = hd < ep.Hq ? ep.q_out + ((size_t)t * ep.Hq + hd) * 64 + d + 32 : kh + kv_k_off(p, d + 32);
            *reinterpret_cast<uint32_t*>(d1) = lo;
            *reinterpret_cast<uint32_t*>(d2) = hi;
          }
        } else if (in_cap) {
          uint16_t* vh = ep.v_pool + base[a][v] + (size_t)(hd - ep.Hq - ep.Hkv) * cap[a][v] * 64;
#pragma unroll
          for (int b = 0; b < 4; ++b) vh[kv_v_off(p, 16 * b + r)] = f2bf(xv[b]);
        }
      }
  }
}

int gemm_slices(int K) { return ((K + 127) / 128 + kKQW - 1) / kKQW; }

size_t linear_partials_bytes(int M, int N, int K) { return (size_t)gemm_slices(K) * M * N * sizeof(float); }

int launch_gemm_splitk(const uint16_t* x, const uint16_t* W, int M, int N, int K, float* part,
                       hipStream_t s) {
  hipLaunchKernelGGL(gemm_splitk_bf16_kernel, dim3(ceil_div(N, 64), gemm_slices(K)), dim3(256), 0, s,
                     x, W, M, N, K, part);
  return check_launch("gemm_splitk_bf16");
}

// x . W^T into fp32 partial planes for a finalizer: the split-K kernel (gemm_slices(K) planes) for
// decode-sized M, the tiled kernel (one folded plane, same bits) from kTiledMinRows rows.
int launch_gemm(const uint16_t* x, const uint16_t* W, int M, int N, int K, float* part, int* slices,
                hipStream_t s) {
  if (M >= kTiledMinRows) {
    *slices = 1;
    if (K % 64 == 0) {
      const int tiles = ceil_div(N, kTileN) * ceil_div(M, kTileM);
      hipLaunchKernelGGL(gemm_tiled_lds_kernel<false>, dim3(8 * ceil_div(tiles, 8)), dim3(64 * kTiledWaves), 0, s, x,
                         W, M, N, K, part, QkvEpilogue{});
      return check_launch("gemm_tiled_lds");
    }
    hipLaunchKernelGGL(gemm_tiled_bf16_kernel, dim3(ceil_div(N, kTileN), ceil_div(M, kTileM)),
                       dim3(64 * kTiledWaves), 0, s,
                       x, W, M, N, K, part);
    return check_launch("gemm_tiled_bf16");
  }
  *slices = gemm_slices(K);
  return launch_gemm_splitk(x, W, M, N, K, part, s);
}

int launch_linear(const uint16_t* x, const uint16_t* W, const uint16_t* b, int M, int N, int K,
                  uint16_t* y, uint16_t* residual, float* part, hipStream_t s) {
  if (M == 0) return FLYAI_OK;
  int slices = 0;
  int rc = launch_gemm(x, W, M, N, K, part, &slices, s);
  if (rc) return rc;
  const size_t total = (size_t)M * N;
  hipLaunchKernelGGL(linear_finalize_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s,
                     part, slices, b, M, N, y, residual);
  return check_launch("linear_finalize");
}

int launch_linear_residual_rmsnorm(const uint16_t* x, const uint16_t* W, const uint16_t* b, int M,
                                   int N, int K, uint16_t* h, const float* lnw, float eps,
                                   uint16_t* xn, float* part, hipStream_t s) {
  if (M == 0) return FLYAI_OK;
  int slices = 0;
  int rc = launch_gemm(x, W, M, N, K, part, &slices, s);
  if (rc) return rc;
  if (N > 7 * kRowThreads) return set_error(FLYAI_EINVAL, "residual_rmsnorm: H <= %d", 7 * kRowThreads);
  auto go = [&](auto iters, auto smax) {
    hipLaunchKernelGGL((residual_rmsnorm_finalize_kernel<decltype(iters)::value, decltype(smax)::value>), dim3(M),
                       dim3(kRowThreads), 0, s, part, slices, b, M, N, h, lnw, eps, xn);
  };
  using I3 = std::integral_constant<int, 3>;
  using I7 = std::integral_constant<int, 7>;
  using S1 = std::integral_constant<int, 1>;
  using S8 = std::integral_constant<int, 8>;
  if (N <= 3 * kRowThreads) {
    if (slices == 1) go(I3{}, S1{}); else go(I3{}, S8{});
  } else {
    if (slices == 1) go(I7{}, S1{}); else go(I7{}, S8{});
  }
  return check_launch("residual_rmsnorm_finalize");
}

// Output projection + residual + RMSNorm + router logits for batches of at most kFusedRouteTokens
// tokens (each token's kRouteSplit workgroups read the router matrix once between them, from L2).
// The new residual stream is written to h_out.
constexpr int kFusedRouteTokens = 256;

int launch_linear_residual_rmsnorm_logits(const uint16_t* x, const uint16_t* W, const uint16_t* b, int M,
                                          int N, int K, const uint16_t* h_in, uint16_t* h_out,
                                          const float* lnw, float eps, uint16_t* xn, float* part,
                                          const uint16_t* rw, const uint16_t* rb, int E, float* logits,
                                          hipStream_t s) {
  if (M == 0) return FLYAI_OK;
  if (M > kFusedRouteTokens || N > 7168 || N % 8 || E > 256)
    return set_error(FLYAI_EINVAL, "fused router logits: needs T <= 256, H %% 8 == 0, H <= 7168, E <= 256");
  int slices = 0;
  int rc = launch_gemm(x, W, M, N, K, part, &slices, s);
  if (rc) return rc;
  auto go = [&](auto jmax, auto smax) {
    hipLaunchKernelGGL((residual_rmsnorm_logits_kernel<decltype(jmax)::value, decltype(smax)::value>),
                       dim3(M, kRouteSplit), dim3(kRowThreads), 0, s, part, slices, b, M, N, h_in, h_out, lnw,
                       eps, xn, rw, rb, E, logits);
  };
  using J6 = std::integral_constant<int, 6>;
  using J14 = std::integral_constant<int, 14>;
  using S1 = std::integral_constant<int, 1>;
  using S8 = std::integral_constant<int, 8>;
  if (N <= 3072) {
    if (slices == 1) go(J6{}, S1{}); else go(J6{}, S8{});
  } else {  // 7 columns per thread and 14 router chunks: more slices in registers would spill
    go(J14{}, S1{});
  }
  return check_launch("residual_rmsnorm_logits");
}

// ---- QKV finalize + RoPE (GPT-OSS half split, per-op bf16 rounding) + K/V append ------------------
// qkv[t][f] = bf16(sum of the split-K partials + bias) -- exactly what the unfused Linear writes --
// then q/k rotate (first = x1 c - x2 s, second = x2 c + x1 s, each product and sum rounded to bf16),
// q goes to q_out and k/v to the sequence's slab at the token's position.  One workgroup per token.
template <bool FROM_PARTIALS>
__global__ __launch_bounds__(256) void rope_kv_append_kernel(
    const uint16_t* __restrict__ qkv, const float* __restrict__ part, int slices, int M,
    const uint16_t* __restrict__ bias, const int32_t* __restrict__ positions,
    const int32_t* __restrict__ seq_id, const uint16_t* __restrict__ cos_tab,
    const uint16_t* __restrict__ sin_tab, int rope_positions, int Hq, int Hkv, int D,
    const int64_t* __restrict__ kv_base, const int32_t* __restrict__ kv_cap,
    uint16_t* __restrict__ q_out, uint16_t* __restrict__ k_pool, uint16_t* __restrict__ v_pool,
    const int32_t* __restrict__ kv_pos) {
  const int t = blockIdx.x;
  const int pos = positions[t];
  if (pos < 0 || pos >= rope_positions) return;  // outside the rotary table: no read, no write
  const int b = seq_id[t];
  const int cap = kv_cap[b];
  const int slot = kv_pos ? kv_pos[t] : pos;  // tree verify writes node i at its own slot
  const bool in_cap = slot >= 0 && slot < cap;
  const int64_t base = kv_base[b];
  const int D2 = D / 2;
  const int width = (Hq + 2 * Hkv) * D;
  const size_t stride = (size_t)M * width;
  auto val = [&](int f) -> float {
    if (FROM_PARTIALS)
      return bf16_round(sum_slices(part, slices, stride, (size_t)t * width + f) + (bias ? bf2f(bias[f]) : 0.f));
    return bf2f(qkv[(size_t)t * width + f]);
  };
  const uint16_t* cr = cos_tab + (size_t)pos * D2;
  const uint16_t* sr = sin_tab + (size_t)pos * D2;
  const int pairs = (Hq + Hkv) * D2;
  const int nthr = blockDim.x * gridDim.y, tid = blockIdx.y * blockDim.x + threadIdx.x;
  for (int i = tid; i < pairs; i += nthr) {
    const int h = i / D2, d = i % D2;
    const float x1 = val(h * D + d), x2 = val(h * D + d + D2);
    const float c = bf2f(cr[d]), s = bf2f(sr[d]);
    const float first = bf16_round(bf16_round(x1 * c) - bf16_round(x2 * s));
    const float second = bf16_round(bf16_round(x2 * c) + bf16_round(x1 * s));
    if (h < Hq) {
      q_out[((size_t)t * Hq + h) * D + d] = f2bf(first);
      q_out[((size_t)t * Hq + h) * D + d + D2] = f2bf(second);
    } else if (in_cap) {
      uint16_t* kh = k_pool + base + (size_t)(h - Hq) * cap * D;  // the head's tiled region
      kh[kv_k_off(slot, d)] = f2bf(first);
      kh[kv_k_off(slot, d + D2)] = f2bf(second);
    }
  }
  if (in_cap) {
    for (int i = tid; i < Hkv * D; i += nthr) {
      const int gv = i / D, d = i % D;
      v_pool[base + (size_t)gv * cap * D + kv_v_off(slot, d)] = f2bf(val((Hq + Hkv) * D + gv * D + d));
    }
  }
}

// The stage's QKV finalize + RoPE + K/V append from the split-K partials, vectorised: each thread
// takes four rotary pairs of one head (features d0..d0+3 and d0+D/2..+3) or four V dims, sums the
// NS-bounded slices with float4 loads all issued before the first add (same slice order and
// per-op bf16 rounding as rope_kv_append_kernel<true>), and writes its q, K or transposed V values.
template <int NS>
__global__ __launch_bounds__(256) void qkv_rope_kv_vec_kernel(
    const float* __restrict__ part, int slices, int M, const uint16_t* __restrict__ bias,
    const int32_t* __restrict__ positions, const int32_t* __restrict__ seq_id,
    const uint16_t* __restrict__ cos_tab, const uint16_t* __restrict__ sin_tab, int rope_positions,
    int Hq, int Hkv, int D, const int64_t* __restrict__ kv_base, const int32_t* __restrict__ kv_cap,
    uint16_t* __restrict__ q_out, uint16_t* __restrict__ k_pool, uint16_t* __restrict__ v_pool,
    const int32_t* __restrict__ kv_pos) {
  const int t = blockIdx.x;
  const int u = blockIdx.y * blockDim.x + threadIdx.x;
  const int D2 = D / 2, Q2 = D2 / 4, QV = D / 4;
  const int rot_units = (Hq + Hkv) * Q2;
  if (u >= rot_units + Hkv * QV) return;
  // Every load that depends only on (t, u) -- the token's indices, the unit's split-K partials and
  // bias -- goes out before the first use, and the rotary table and the sequence's KV geometry in
  // the next batch: two memory round trips in all.  Slices past `slices` are clamped for the load and
  // never added; the sums run in slice order as in sum_slices.
  const int pos = positions[t];
  const int b = seq_id[t];
  const int slot_in = kv_pos ? kv_pos[t] : 0;
  const bool rot = u < rot_units;
  const int h = u / Q2, d0r = (u % Q2) * 4;                       // rotary unit
  const int gv = (u - rot_units) / QV, d0v = ((u - rot_units) % QV) * 4;  // V unit
  const int f1 = rot ? h * D + d0r : (Hq + Hkv) * D + gv * D + d0v;
  const int f2 = rot ? f1 + D2 : f1;
  const int width = (Hq + 2 * Hkv) * D;
  const size_t stride = (size_t)M * width;
  const float* row = part + (size_t)t * width;
  float4 p1[NS], p2[NS];
#pragma unroll
  for (int i = 0; i < NS; ++i) {
    const size_t off = (size_t)min(i, slices - 1) * stride;
    p1[i] = *reinterpret_cast<const float4*>(row + off + f1);
    p2[i] = *reinterpret_cast<const float4*>(row + off + f2);
  }
  float b1[4], b2[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    b1[j] = bias ? bf2f(bias[f1 + j]) : 0.f;
    b2[j] = bias ? bf2f(bias[f2 + j]) : 0.f;
  }
  if (pos < 0 || pos >= rope_positions) return;  // outside the rotary table: no read, no write
  const int cap = kv_cap[b];
  const int64_t base = kv_base[b];
  // the K/V slot: the position itself, or the tree node's slot in tree verify
  const int slot = kv_pos ? slot_in : pos;
  const bool in_cap = slot >= 0 && slot < cap;
  auto sum4 = [&](const float4 (&pv)[NS], const float (&bv)[4], float (&o)[4]) __attribute__((always_inline)) {
    float4 a = pv[0];
#pragma unroll
    for (int i = 1; i < NS; ++i)
      if (i < slices) { a.x += pv[i].x; a.y += pv[i].y; a.z += pv[i].z; a.w += pv[i].w; }
    const float av[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) o[j] = bf16_round(av[j] + bv[j]);
  };
  if (rot) {
    const int d0 = d0r;
    if (h >= Hq && !in_cap) return;
    const uint16_t* cr = cos_tab + (size_t)pos * D2 + d0;
    const uint16_t* sr = sin_tab + (size_t)pos * D2 + d0;
    float cv[4], sv[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) { cv[j] = bf2f(cr[j]); sv[j] = bf2f(sr[j]); }
    float x1[4], x2[4];
    sum4(p1, b1, x1);
    sum4(p2, b2, x2);
    uint16_t first[4], second[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float c = cv[j], sn = sv[j];
      first[j] = f2bf(bf16_round(bf16_round(x1[j] * c) - bf16_round(x2[j] * sn)));
      second[j] = f2bf(bf16_round(bf16_round(x2[j] * c) + bf16_round(x1[j] * sn)));
    }
    // four consecutive dims from a multiple of 4 stay contiguous in the tiled K layout
    uint16_t* kh = k_pool + base + (size_t)(h - Hq) * cap * D;
    uint16_t* d1 = h < Hq ? q_out + ((size_t)t * Hq + h) * D + d0 : kh + kv_k_off(slot, d0);
    uint16_t* d2 = h < Hq ? q_out + ((size_t)t * Hq + h) * D + d0 + D2 : kh + kv_k_off(slot, d0 + D2);
    *reinterpret_cast<uint2*>(d1) = make_uint2(first[0] | ((uint32_t)first[1] << 16),
                                               first[2] | ((uint32_t)first[3] << 16));
    *reinterpret_cast<uint2*>(d2) = make_uint2(second[0] | ((uint32_t)second[1] << 16),
                                               second[2] | ((uint32_t)second[3] << 16));
  } else if (in_cap) {
    float o[4];
    sum4(p1, b1, o);
#pragma unroll
    for (int j = 0; j < 4; ++j) v_pool[base + (size_t)gv * cap * D + kv_v_off(slot, d0v + j)] = f2bf(o[j]);
  }
}

int launch_rope_kv(const uint16_t* qkv, const int32_t* positions, const int32_t* seq_id,
                   const uint16_t* cos_tab, const uint16_t* sin_tab, int rope_positions, int T,
                   int Hq, int Hkv, int D, const int64_t* kv_base, const int32_t* kv_cap,
                   uint16_t* q_out, uint16_t* k_pool, uint16_t* v_pool, hipStream_t s) {
  if (T == 0) return FLYAI_OK;
  hipLaunchKernelGGL(rope_kv_append_kernel<false>, dim3(T), dim3(256), 0, s, qkv, nullptr, 0, T,
                     nullptr, positions, seq_id, cos_tab, sin_tab, rope_positions, Hq, Hkv, D, kv_base,
                     kv_cap, q_out, k_pool, v_pool, nullptr);
  return check_launch("rope_kv_append");
}

// QKV projection + RoPE + KV append: split-K GEMM, then the fused finalize.  kv_pos (nullable) gives
// each token's K/V slot when it differs from its rotary position (tree verify).
int launch_qkv_rope_kv(const uint16_t* x, const uint16_t* Wqkv, const uint16_t* bqkv, float* part,
                       const int32_t* positions, const int32_t* seq_id, const uint16_t* cos_tab,
                       const uint16_t* sin_tab, int rope_positions, int T, int H, int Hq, int Hkv,
                       int D, const int64_t* kv_base, const int32_t* kv_cap, uint16_t* q_out,
                       uint16_t* k_pool, uint16_t* v_pool, const int32_t* kv_pos, hipStream_t s) {
  if (T == 0) return FLYAI_OK;
  const int width = (Hq + 2 * Hkv) * D;
  if (T >= kTiledMinRows && H % 64 == 0 && D == 64 && !kv_pos) {
    // prefill-sized: the finalize, RoPE and KV append in the tiled GEMM's epilogue (no fp32 plane)
    const int tiles = ceil_div(width, kTileN) * ceil_div(T, kTileM);
    const QkvEpilogue ep{bqkv, positions, seq_id, cos_tab, sin_tab, kv_base, kv_cap, q_out, k_pool, v_pool,
                         rope_positions, Hq, Hkv};
    hipLaunchKernelGGL(gemm_tiled_lds_kernel<true>, dim3(8 * ceil_div(tiles, 8)), dim3(64 * kTiledWaves), 0, s, x,
                       Wqkv, T, width, H, part, ep);
    return check_launch("gemm_tiled_lds_qkv");
  }
  int slices = 0;
  int rc = launch_gemm(x, Wqkv, T, width, H, part, &slices, s);
  if (rc) return rc;
  if (D % 8 == 0 && slices <= 16) {
    const int units = (Hq + Hkv) * (D / 8) + Hkv * (D / 4);
    const dim3 grid(T, ceil_div(units, 256));
    // the slice count the kernel loads unconditionally: exact for the tiled GEMM's one plane and for
    // K = 2880 (6 planes), rounded up otherwise (clamped loads past `slices` are never added)
    auto go = [&](auto ns) {
      hipLaunchKernelGGL((qkv_rope_kv_vec_kernel<decltype(ns)::value>), grid, dim3(256), 0, s, part, slices, T,
                         bqkv, positions, seq_id, cos_tab, sin_tab, rope_positions, Hq, Hkv, D, kv_base, kv_cap,
                         q_out, k_pool, v_pool, kv_pos);
    };
    if (slices == 1) go(std::integral_constant<int, 1>{});
    else if (slices <= 6) go(std::integral_constant<int, 6>{});
    else if (slices <= 8) go(std::integral_constant<int, 8>{});
    else go(std::integral_constant<int, 16>{});
  } else {
    hipLaunchKernelGGL(rope_kv_append_kernel<true>, dim3(T, 4), dim3(256), 0, s, nullptr, part, slices, T,
                       bqkv, positions, seq_id, cos_tab, sin_tab, rope_positions, Hq, Hkv, D, kv_base,
                       kv_cap, q_out, k_pool, v_pool, kv_pos);
  }
  return check_launch("qkv_rope_kv_append");
}

}  // namespace flyai

using namespace flyai;

extern "C" int flyai_rmsnorm(const uint16_t* x, const float* w, int32_t T, int32_t H, float eps,
                             uint16_t* y, flyai_stream_t stream) {
  FLYAI_REQUIRE(T >= 0 && H > 0, "rmsnorm: bad shape");
  FLYAI_REQUIRE(x && w && y, "rmsnorm: null pointer");
  return launch_rmsnorm(x, w, T, H, eps, y, as_stream(stream));
}

extern "C" size_t flyai_linear_workspace_bytes(int32_t M, int32_t N, int32_t K) {
  if (M <= 0 || N <= 0 || K <= 0) return 0;
  return linear_partials_bytes(M, N, K);
}

extern "C" int flyai_linear_bf16(const uint16_t* x, const uint16_t* w, const uint16_t* b, int32_t M,
                                 int32_t N, int32_t K, uint16_t* y, uint16_t* residual,
                                 float* workspace, flyai_stream_t stream) {
  FLYAI_REQUIRE(M >= 0 && N > 0 && K > 0 && N % 16 == 0 && K % 32 == 0 && K <= 8192,
                "linear: need N %% 16 == 0, K %% 32 == 0, K <= 8192");
  FLYAI_REQUIRE(x && w && (y || residual) && workspace, "linear: null pointer");
  return launch_linear(x, w, b, M, N, K, y, residual, workspace, as_stream(stream));
}

// ---- the linear without allocation --------------------------------------------------------------
// The split-K partial planes (or the tiled kernel's one folded plane) live in this file-scope device
// array instead of a caller workspace.  Every GPU the library runs on holds its own copy, at its own
// address, until the process ends.  In host code the name `scratch` is only a host-side stand-in: its
// device address comes from hipGetSymbolAddress, resolved once per device with that device current and
// kept in g_scratch_dev[]; kernels receive that address, never the name.
constexpr size_t kLinearScratchBytes = (size_t)16 << 20;
static __device__ __align__(256) float scratch[kLinearScratchBytes / sizeof(float)];

constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mu;
static float* g_scratch_dev[kMaxDevices] = {};

static int linear_scratch(float** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return set_error(FLYAI_EHIP, "hipGetDevice: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices) return set_error(FLYAI_EINVAL, "linear_noalloc: device %d >= %d", dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_dev[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return set_error(FLYAI_EHIP, "hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
    g_scratch_dev[dev] = static_cast<float*>(p);
  }
  *out = g_scratch_dev[dev];
  return FLYAI_OK;
}

// bytes of partial planes launch_gemm writes and the finalizer reads for this shape
static size_t linear_partials_used(int M, int N, int K) {
  const int planes = M >= kTiledMinRows ? 1 : gemm_slices(K);
  return (size_t)planes * M * N * sizeof(float);
}

extern "C" size_t flyai_linear_noalloc_max_bytes(void) { return kLinearScratchBytes; }

extern "C" int flyai_linear_bf16_noalloc(const uint16_t* x, const uint16_t* w, const uint16_t* b, int32_t M,
                                         int32_t N, int32_t K, uint16_t* y, uint16_t* residual,
                                         flyai_stream_t stream) {
  FLYAI_REQUIRE(M >= 0 && N > 0 && K > 0 && N % 16 == 0 && K % 32 == 0 && K <= 8192,
                "linear: need N %% 16 == 0, K %% 32 == 0, K <= 8192");
  FLYAI_REQUIRE(x && w && (y || residual), "linear: null pointer");
  const size_t need = linear_partials_used(M, N, K);
  FLYAI_REQUIRE(need <= kLinearScratchBytes,
                "linear_noalloc: M=%d N=%d K=%d needs %zu partial bytes > the %zu-byte static scratch", M, N, K,
                need, kLinearScratchBytes);
  if (M == 0) return FLYAI_OK;
  float* part = nullptr;
  const int rc = linear_scratch(&part);
  if (rc) return rc;
  // every partial the finalizer reads is written by this call's GEMM first: nothing needs clearing
  return launch_linear(x, w, b, M, N, K, y, residual, part, as_stream(stream));
}

extern "C" int flyai_rope_kv_append(const uint16_t* qkv, const int32_t* positions,
                                    const int32_t* seq_id, const uint16_t* cos_tab,
                                    const uint16_t* sin_tab, int32_t rope_positions, int32_t T,
                                    int32_t Hq, int32_t Hkv, int32_t D, const int64_t* kv_base,
                                    const int32_t* kv_cap, uint16_t* q_out, uint16_t* k_pool,
                                    uint16_t* v_pool, flyai_stream_t stream) {
  FLYAI_REQUIRE(T >= 0 && Hq > 0 && Hkv > 0 && D == 64 && rope_positions > 0,
                "rope_kv: bad shape (the tiled KV layout needs head_dim 64)");
  FLYAI_REQUIRE(qkv && positions && seq_id && cos_tab && sin_tab && kv_base && kv_cap && q_out &&
                    k_pool && v_pool,
                "rope_kv: null pointer");
  return launch_rope_kv(qkv, positions, seq_id, cos_tab, sin_tab, rope_positions, T, Hq, Hkv, D,
                        kv_base, kv_cap, q_out, k_pool, v_pool, as_stream(stream));
}
