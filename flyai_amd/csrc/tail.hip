// Head and tail of a served model on one GPU: token embedding gather, and the tail's final-norm
// output -> lm_head logits -> greedy argmax (phase0/specpipe.py:595-616, :779-801: embed(token_ids);
// lm_head(norm(h)) then argmax(-1), the greedy path of Sampler.sample_logits / accept,
// phase0/specsample.py:78-100).
//
// lm_head weights are re-packed once (flyai_bf16_tile_repack) from the nn.Linear layout W[V][H]
// into 16-row tiles in MFMA-fragment order: tile t, K step s (32 inputs) is one contiguous KiB in
// which lane l = 16g + r holds W[16t + r][32s + 8g .. 32s + 8g + 7].  A wave's 16-byte load per
// lane is then one contiguous KiB, and that register is directly the A operand of
// v_mfma_f32_16x16x32_bf16 (vocab rows x K); the normed hidden rows are the B operand (K x tokens),
// staged in LDS per 128-K chunk in the same fragment order.  The weights stream once from HBM
// through a register ring; the hidden rows (a few hundred KB) stay in L2.
#include "common.h"

namespace flyai {

constexpr int kTailWaves = 4;
constexpr int kTailNTW = 2;                                   // vocab tiles per wave
constexpr int kTailRowsPerWG = kTailWaves * kTailNTW * 16;    // 128 vocab rows per workgroup
constexpr int kTailMaxRows = 64;                              // token rows per launch (4 tiles)

typedef unsigned int tail_u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint4 tail_ld_nt(const uint8_t* p) {
  const tail_u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const tail_u32x4*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}

// (value desc, id asc): the first maximal index, as torch.argmax returns it
__device__ __forceinline__ bool tail_better(float v, int i, float bv, int bi) {
  return v > bv || (v == bv && i < bi);
}

// ---- re-pack W[N][K] bf16 -> [N/16][K/32][64 lanes][16 B] -----------------------------------------
__global__ __launch_bounds__(256) void bf16_tile_repack_kernel(const uint16_t* __restrict__ w, int N, int K,
                                                               uint8_t* __restrict__ packed) {
  const size_t S = K / 32;
  const size_t total = (size_t)(N / 16) * S * 64;
  const size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= total) return;
  const int lane = idx % 64;
  const size_t s = (idx / 64) % S;
  const size_t t = idx / 64 / S;
  const int r = lane & 15, g = lane >> 4;
  const uint4 v = *reinterpret_cast<const uint4*>(w + (t * 16 + r) * (size_t)K + s * 32 + 8 * g);
  *reinterpret_cast<uint4*>(packed + idx * 16) = v;
}

// ---- embedding gather: out[t] = table[ids[t]] (ids outside [0, V) give a zero row) -------------
__global__ __launch_bounds__(256) void embed_gather_kernel(const uint16_t* __restrict__ table,
                                                           const int32_t* __restrict__ ids, int H, int V,
                                                           uint16_t* __restrict__ out) {
  const int t = blockIdx.x;
  const int id = ids[t];
  const bool ok = id >= 0 && id < V;
  const uint4* src = reinterpret_cast<const uint4*>(table + (size_t)(ok ? id : 0) * H);
  uint4* dst = reinterpret_cast<uint4*>(out + (size_t)t * H);
  for (int i = threadIdx.x; i < H / 8; i += 256) dst[i] = ok ? src[i] : make_uint4(0, 0, 0, 0);
}

// ---- lm_head + argmax --------------------------------------------------------------------------
// Workgroup = 4 waves x 2 vocab tiles = 128 vocab rows, all TT token tiles (16 token rows each).
// K advances in chunks of 4 MFMA steps (128 K): the chunk's hidden fragments live in one of two
// LDS buffers (TT KiB per step), the next chunk's are loaded into registers one chunk ahead, and
// the weights go through a 4-deep register ring (3 steps in flight while one computes).  One
// workgroup barrier per chunk.  Logits are rounded to bf16 (the reference's bf16 lm_head output)
// and reduced to (max, lowest id) per token over the workgroup; argmax_finish_kernel folds the
// workgroups.
template <int TT>
__global__ __launch_bounds__(256) void lm_head_argmax_kernel(
    const uint16_t* __restrict__ x, const int32_t* __restrict__ rows, int n_rows, int K,
    const uint8_t* __restrict__ wp, int V, float* __restrict__ part_val, int32_t* __restrict__ part_id,
    uint16_t* __restrict__ logits_out) {
  __shared__ uint4 xs[2][TT][4][64];
  __shared__ float red_v[kTailWaves][TT * 16];
  __shared__ int red_i[kTailWaves][TT * 16];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int n = lane & 15, g = lane >> 4;
  const int S = K / 32;                 // MFMA steps
  const int NC = (S + 3) / 4;           // chunks of 4 steps
  const int n_tiles = V / 16;
  const int t0 = (blockIdx.x * kTailWaves + wave) * kTailNTW;

  // staging: thread tid covers, for each token tile tt, step j = tid/64 of the chunk, fragment lane
  // tid%64 -> token row 16tt + (tid & 15), K 32*(4c + j) + 8*((tid & 63) >> 4)
  const int sj = tid >> 6, sn = tid & 15, sg = (tid & 63) >> 4;
  const uint16_t* srow[TT];
#pragma unroll
  for (int tt = 0; tt < TT; ++tt) {
    const int rr = 16 * tt + sn;
    srow[tt] = rr < n_rows ? x + (size_t)(rows ? rows[rr] : rr) * K : nullptr;
  }
  auto load_x = [&](uint4 (&xr)[TT], int c) {
    const int s = 4 * c + sj;
#pragma unroll
    for (int tt = 0; tt < TT; ++tt)
      xr[tt] = (srow[tt] && s < S) ? *reinterpret_cast<const uint4*>(srow[tt] + 32 * s + 8 * sg)
                                   : make_uint4(0, 0, 0, 0);
  };
  auto store_x = [&](const uint4 (&xr)[TT], int buf) {
#pragma unroll
    for (int tt = 0; tt < TT; ++tt) xs[buf][tt][sj][lane] = xr[tt];
  };

  const uint8_t* wbase = wp + (size_t)t0 * S * 1024 + lane * 16;
  auto load_w = [&](uint4 (&w)[kTailNTW], int s) {
#pragma unroll
    for (int nn = 0; nn < kTailNTW; ++nn)
      w[nn] = (t0 + nn < n_tiles && s < S) ? tail_ld_nt(wbase + ((size_t)nn * S + s) * 1024)
                                            : make_uint4(0, 0, 0, 0);
  };
  f32x4_t acc[kTailNTW][TT];
#pragma unroll
  for (int nn = 0; nn < kTailNTW; ++nn)
#pragma unroll
    for (int tt = 0; tt < TT; ++tt) acc[nn][tt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  auto compute = [&](const uint4 (&w)[kTailNTW], int buf, int j) {
#pragma unroll
    for (int tt = 0; tt < TT; ++tt) {
      const bf16x8_t b = as_bf16x8(xs[buf][tt][j][lane]);
#pragma unroll
      for (int nn = 0; nn < kTailNTW; ++nn) acc[nn][tt] = mfma16x16x32(as_bf16x8(w[nn]), b, acc[nn][tt]);
    }
  };

  uint4 xr[TT];
  load_x(xr, 0);
  store_x(xr, 0);
  load_x(xr, 1);
  uint4 w0[kTailNTW], w1[kTailNTW], w2[kTailNTW], w3[kTailNTW];
  load_w(w0, 0);
  load_w(w1, 1);
  load_w(w2, 2);
  lds_barrier();
  for (int c = 0; c < NC; ++c) {
    const int buf = c & 1, s0 = 4 * c;
    load_w(w3, s0 + 3);
    compute(w0, buf, 0);
    load_w(w0, s0 + 4);
    compute(w1, buf, 1);
    load_w(w1, s0 + 5);
    compute(w2, buf, 2);
    load_w(w2, s0 + 6);
    compute(w3, buf, 3);
    // the next chunk's fragments go to the other buffer: every wave finished reading it before the
    // previous barrier, and the barrier below publishes it
    store_x(xr, buf ^ 1);
    load_x(xr, c + 2);
    lds_barrier();
  }

  // lane (n, g) holds the logits of vocab rows 16(t0+nn) + 4g + v for token row 16tt + n
#pragma unroll
  for (int tt = 0; tt < TT; ++tt) {
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    const int row = 16 * tt + n;
#pragma unroll
    for (int nn = 0; nn < kTailNTW; ++nn) {
      if (t0 + nn >= n_tiles) continue;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int id = (t0 + nn) * 16 + 4 * g + v;
        const uint16_t lb = f2bf(acc[nn][tt][v]);
        const float lv = bf2f(lb);
        if (logits_out && row < n_rows) logits_out[(size_t)row * V + id] = lb;
        if (tail_better(lv, id, bv, bi)) { bv = lv; bi = id; }
      }
    }
#pragma unroll
    for (int o = 16; o <= 32; o <<= 1) {
      const float ov = __shfl_xor(bv, o, 64);
      const int oi = __shfl_xor(bi, o, 64);
      if (tail_better(ov, oi, bv, bi)) { bv = ov; bi = oi; }
    }
    if (g == 0) {
      red_v[wave][16 * tt + n] = bv;
      red_i[wave][16 * tt + n] = bi;
    }
  }
  __syncthreads();
  if (tid < n_rows) {
    float bv = red_v[0][tid];
    int bi = red_i[0][tid];
    for (int w = 1; w < kTailWaves; ++w)
      if (tail_better(red_v[w][tid], red_i[w][tid], bv, bi)) { bv = red_v[w][tid]; bi = red_i[w][tid]; }
    part_val[(size_t)blockIdx.x * n_rows + tid] = bv;
    part_id[(size_t)blockIdx.x * n_rows + tid] = bi;
  }
}

// One workgroup per token row: the (max, lowest id) over every workgroup's partial.
__global__ __launch_bounds__(256) void argmax_finish_kernel(const float* __restrict__ part_val,
                                                            const int32_t* __restrict__ part_id, int n_parts,
                                                            int n_rows, int32_t* __restrict__ ids) {
  __shared__ float sv[4];
  __shared__ int si[4];
  const int row = blockIdx.x, tid = threadIdx.x;
  float bv = -INFINITY;
  int bi = 0x7fffffff;
  for (int p = tid; p < n_parts; p += 256) {
    const float v = part_val[(size_t)p * n_rows + row];
    const int i = part_id[(size_t)p * n_rows + row];
    if (tail_better(v, i, bv, bi)) { bv = v; bi = i; }
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    const float ov = __shfl_xor(bv, o, 64);
    const int oi = __shfl_xor(bi, o, 64);
    if (tail_better(ov, oi, bv, bi)) { bv = ov; bi = oi; }
  }
  if ((tid & 63) == 0) { sv[tid >> 6] = bv; si[tid >> 6] = bi; }
  __syncthreads();
  if (tid == 0) {
    for (int w = 1; w < 4; ++w)
      if (tail_better(sv[w], si[w], bv, bi)) { bv = sv[w]; bi = si[w]; }
    ids[row] = bi;
  }
}

static int lm_head_parts(int V) { return (V + kTailRowsPerWG - 1) / kTailRowsPerWG; }

}  // namespace flyai

using namespace flyai;

extern "C" size_t flyai_bf16_tile_packed_bytes(int32_t N, int32_t K) {
  if (N <= 0 || K <= 0 || N % 16 || K % 32) return 0;
  return (size_t)N * K * 2;
}

extern "C" int flyai_bf16_tile_repack(const uint16_t* w, int32_t N, int32_t K, uint8_t* packed,
                                      flyai_stream_t stream) {
  FLYAI_REQUIRE(N > 0 && K > 0 && N % 16 == 0 && K % 32 == 0, "bf16_tile_repack: need N %% 16 == 0, K %% 32 == 0");
  FLYAI_REQUIRE(w && packed, "bf16_tile_repack: null pointer");
  const size_t total = (size_t)(N / 16) * (K / 32) * 64;
  hipLaunchKernelGGL(bf16_tile_repack_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                     as_stream(stream), w, N, K, packed);
  return check_launch("bf16_tile_repack");
}

extern "C" int flyai_embed_gather(const uint16_t* table, const int32_t* ids, int32_t T, int32_t H, int32_t V,
                                  uint16_t* out, flyai_stream_t stream) {
  FLYAI_REQUIRE(T >= 0 && H > 0 && H % 8 == 0 && V > 0, "embed_gather: need H %% 8 == 0");
  FLYAI_REQUIRE(table && ids && out, "embed_gather: null pointer");
  if (T == 0) return FLYAI_OK;
  hipLaunchKernelGGL(embed_gather_kernel, dim3(T), dim3(256), 0, as_stream(stream), table, ids, H, V, out);
  return check_launch("embed_gather");
}

extern "C" size_t flyai_lm_head_workspace_bytes(int32_t n_rows, int32_t V) {
  if (n_rows <= 0 || V <= 0) return 0;
  return (size_t)lm_head_parts(V) * n_rows * (sizeof(float) + sizeof(int32_t));
}

extern "C" int flyai_lm_head_argmax(const uint16_t* x, const int32_t* rows, int32_t n_rows, int32_t H,
                                    const uint8_t* w_packed, int32_t V, int32_t* ids, uint16_t* logits,
                                    void* workspace, flyai_stream_t stream) {
  FLYAI_REQUIRE(n_rows >= 0 && n_rows <= kTailMaxRows, "lm_head_argmax: n_rows %d outside [0, %d]", n_rows,
                kTailMaxRows);
  FLYAI_REQUIRE(H > 0 && H % 32 == 0 && V > 0 && V % 16 == 0, "lm_head_argmax: need H %% 32 == 0, V %% 16 == 0");
  FLYAI_REQUIRE(x && w_packed && ids && workspace, "lm_head_argmax: null pointer");
  if (n_rows == 0) return FLYAI_OK;
  hipStream_t s = as_stream(stream);
  const int parts = lm_head_parts(V);
  float* pv = static_cast<float*>(workspace);
  int32_t* pi = reinterpret_cast<int32_t*>(pv + (size_t)parts * n_rows);
  const int TT = (n_rows + 15) / 16;
  switch (TT) {
    case 1: hipLaunchKernelGGL(lm_head_argmax_kernel<1>, dim3(parts), dim3(256), 0, s, x, rows, n_rows, H, w_packed, V, pv, pi, logits); break;
    case 2: hipLaunchKernelGGL(lm_head_argmax_kernel<2>, dim3(parts), dim3(256), 0, s, x, rows, n_rows, H, w_packed, V, pv, pi, logits); break;
    case 3: hipLaunchKernelGGL(lm_head_argmax_kernel<3>, dim3(parts), dim3(256), 0, s, x, rows, n_rows, H, w_packed, V, pv, pi, logits); break;
    default: hipLaunchKernelGGL(lm_head_argmax_kernel<4>, dim3(parts), dim3(256), 0, s, x, rows, n_rows, H, w_packed, V, pv, pi, logits); break;
  }
  int rc = check_launch("lm_head_argmax");
  if (rc) return rc;
  hipLaunchKernelGGL(argmax_finish_kernel, dim3(n_rows), dim3(256), 0, s, pv, pi, parts, n_rows, ids);
  return check_launch("argmax_finish");
}
