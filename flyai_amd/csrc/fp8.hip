// FP8 (e4m3) 128x128 block-scaled MoE experts for the DeepSeek-V3-shaped stage: activation
// quantiser, weight re-pack, grouped expert GEMM on the gfx950 scaled MFMA, and the combine that
// adds the shared expert.
//
// Semantics (vendor/deepseek_v4_ref/inference/model.py:114-124 linear, :592-611 Expert, :634-650
// MoE; kernel.py:204-254 fp8_gemm; engines/deepseek_v4/v4_kernels_cpu.py:89-104 act_quant):
//   * activations are quantised per row per 128-K block: s = 2^ceil(log2(max(amax,1e-4)/448)),
//     q = e4m3_rne(clamp(x / s, -448, 448)); s is a power of two, stored as its E8M0 byte;
//   * weights are e4m3 with one power-of-two (E8M0) scale per 128x128 block;
//   * C[m][n] = sum_kb (q_a[m, kb] . q_w[n, kb]) * s_a[m, kb] * s_w[n/128, kb], fp32, bf16 out.
// Both scales being powers of two is what lets v_mfma_scale_f32_16x16x128_f8f6f4 apply them
// inside the MFMA: one instruction covers one 128-K block of 16 rows x 16 columns, with the
// activation row's scale and the weight row's scale as its E8M0 operands.
//
// Packed weight layout of W[E][N][K] (K % 1024 == 0, N % 16 == 0), KB = K/128 steps:
//   data  : [E][N/16][KB][2048 B]; in step kb of tile nt, byte h*1024 + l*16 + i (h = 0, 1;
//           lane l = 16g + r) holds row r, K = 128 kb + 32 g + 16 h + i.  A lane's two 16-byte
//           loads give it the 32 contiguous K values of row r that the MFMA takes from it, and
//           each load instruction of a wave reads one contiguous KiB.
//   scales: after all data, [E][N/16][KB/4][64] dwords; dword (kb4, l) holds the E8M0 scales of
//           row r for steps 4kb4 .. 4kb4+3 in bytes 0..3.
//   gate_up packs w1 and w3 interleaved: packed row 2j = w1 row j, 2j+1 = w3 row j, so the gate and
//   up of one unit land in neighbouring lanes of the MFMA output.
#include <type_traits>

#include "common.h"

namespace flyai {

typedef int v8i_t __attribute__((ext_vector_type(8)));

// Calls f(integral_constant<int, I>) for I = B .. N-1: register arrays indexed this way keep
// constant indices from the start, so they stay in registers.
template <int B, int N, class F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (B < N) {
    f(std::integral_constant<int, B>{});
    static_for<B + 1, N>(f);
  }
}

struct Fp8Geom {
  int NT, KB, KB4;
  size_t data_bytes;
};

__host__ __device__ inline Fp8Geom fp8_geom(int E, int N, int K) {
  Fp8Geom g;
  g.NT = N / 16;
  g.KB = K / 128;
  g.KB4 = (g.KB + 3) / 4;
  g.data_bytes = (size_t)E * g.NT * g.KB * 2048;
  return g;
}

// ---- activation quantiser ------------------------------------------------------------------------
// One wave per (row, 128-block): 2 elements per lane, wave-wide amax, E8M0 scale, RNE to e4m3 with
// v_cvt_pk_fp8_f32 (OCP e4m3fn on gfx950).
__global__ __launch_bounds__(256) void act_quant_fp8_kernel(const uint16_t* __restrict__ x, int M, int K,
                                                            uint8_t* __restrict__ q,
                                                            uint8_t* __restrict__ s) {
  const int KB = K / 128;
  const int item = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (item >= M * KB) return;  // uniform per wave
  const int lane = threadIdx.x & 63;
  const int row = item / KB, kb = item % KB;
  const size_t off = (size_t)row * K + kb * 128 + 2 * lane;
  const uint32_t xv = *reinterpret_cast<const uint32_t*>(x + off);
  const float x0 = bf2f(xv & 0xffff), x1 = bf2f(xv >> 16);
  float amax = fmaxf(fabsf(x0), fabsf(x1));
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o, 64));
  amax = fmaxf(amax, 1e-4f);
  // ceil(log2(amax / 448)) from the bits of amax * (1/448) (a normal number: amax >= 1e-4)
  const uint32_t bits = __float_as_uint(amax * (1.0f / 448.0f));
  const int e = (int)((bits >> 23) & 0xff) - 127 + ((bits & 0x7fffffu) ? 1 : 0);
  const float y0 = fminf(fmaxf(ldexpf(x0, -e), -448.0f), 448.0f);
  const float y1 = fminf(fmaxf(ldexpf(x1, -e), -448.0f), 448.0f);
  const int packed = __builtin_amdgcn_cvt_pk_fp8_f32(y0, y1, 0, false);
  *reinterpret_cast<uint16_t*>(q + off) = (uint16_t)(packed & 0xffff);
  if (lane == 0) s[(size_t)row * KB + kb] = (uint8_t)(e + 127);
}

int launch_act_quant_fp8(const uint16_t* x, int M, int K, uint8_t* q, uint8_t* s, hipStream_t st) {
  if (M == 0) return FLYAI_OK;
  const int items = M * (K / 128);
  hipLaunchKernelGGL(act_quant_fp8_kernel, dim3(ceil_div(items, 4)), dim3(256), 0, st, x, M, K, q, s);
  return check_launch("act_quant_fp8");
}

// ---- re-pack ---------------------------------------------------------------------------------------
// w [E][Nsrc][K] e4m3 bytes, s [E][ceil(Nsrc/128)][K/128] E8M0 bytes; with w3 given, the packed N is
// 2*Nsrc, rows interleaved w1/w3.  One thread per (e, tile, step, lane).
__global__ __launch_bounds__(256) void fp8_repack_kernel(const uint8_t* __restrict__ w1,
                                                         const uint8_t* __restrict__ s1,
                                                         const uint8_t* __restrict__ w3,
                                                         const uint8_t* __restrict__ s3, int E,
                                                         int Nsrc, int K, uint8_t* __restrict__ packed) {
  const int N = w3 ? 2 * Nsrc : Nsrc;
  const Fp8Geom gm = fp8_geom(E, N, K);
  const size_t total = (size_t)E * gm.NT * gm.KB * 64;
  const size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= total) return;
  const int lane = idx % 64;
  const int kb = (idx / 64) % gm.KB;
  const size_t et = idx / 64 / gm.KB;  // e * NT + nt
  const int nt = et % gm.NT, e = et / gm.NT;
  const int r = lane & 15, g = lane >> 4;
  const int prow = nt * 16 + r;
  const bool second = w3 && (prow & 1);
  const int srow = w3 ? prow >> 1 : prow;
  const uint8_t* w = second ? w3 : w1;
  const uint8_t* sc = second ? s3 : s1;
  const int SB = (Nsrc + 127) / 128;
  const uint8_t* src = w + ((size_t)e * Nsrc + srow) * K + kb * 128 + 32 * g;
  uint8_t* dst = packed + (et * gm.KB + kb) * 2048 + lane * 16;
  *reinterpret_cast<uint4*>(dst) = *reinterpret_cast<const uint4*>(src);
  *reinterpret_cast<uint4*>(dst + 1024) = *reinterpret_cast<const uint4*>(src + 16);
  if ((kb & 3) == 0) {
    uint32_t word = 0;
    for (int i = 0; i < 4 && kb + i < gm.KB; ++i)
      word |= (uint32_t)sc[((size_t)e * SB + srow / 128) * gm.KB + kb + i] << (8 * i);
    reinterpret_cast<uint32_t*>(packed + gm.data_bytes)[(et * gm.KB4 + kb / 4) * 64 + lane] = word;
  }
}

// ---- grouped expert GEMM ------------------------------------------------------------------------------
// Workgroup = 4 waves x NTW tiles of 16 weight rows of one expert.  The expert's activation rows
// (up to MT*16 per pass) are staged in LDS one KC-byte K chunk at a time, with their E8M0 scales
// for the whole K staged once per pass; the weights stream once per pass through a 4-deep register
// ring of non-temporal loads (3 steps in flight while one computes, the next body's scale dword
// one body ahead).  Every weight step is used by all MT row tiles.
//
// Vector-memory waits complete in issue order, so a wait on staging loads issued after the ring's
// loads would drain the ring.  The staging loads of chunk c+1 are therefore issued into registers
// at the top of chunk c, before that chunk's ring loads, and stored to LDS at the next chunk
// boundary; all loads are unconditional (step, tile and row clamped to valid ones: a clamped load
// only feeds a step that is never computed or an output that is never stored), and scheduling
// barriers keep the ring's order.
//
// GATE_UP: rows are tokens (act row = perm[p] / k, or p when perm is null); the epilogue rounds gate
// and up to bf16 (w1(x), w3(x) are bf16 Linear outputs), h = silu(gate) * up * routing weight,
// written as bf16 [P][N/2].  DOWN: rows are the permuted h rows; y = bf16 [P][N].
// With n_shared > 0, expert E (packed after the E routed ones) is the shared expert: its rows
// P .. P+n_shared-1 (P = offsets[E]) take tokens 0 .. n_shared-1 with weight 1, so one launch
// covers routed and shared experts.
// Experts with fewer than min_rows or more than max_rows rows are left to another launch.
__host__ __device__ constexpr int fp8_chunk(int MT) { return MT == 1 ? 1024 : 256; }

__host__ __device__ inline int fp8_lds_bytes(int MT, int K) {
  return MT * 16 * (fp8_chunk(MT) + 16 + K / 128);
}

__device__ __forceinline__ v8i_t ld_nt_v8(const uint8_t* p) {
  typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
  const u32x4 a = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  const u32x4 b = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p + 1024));
  return v8i_t{(int)a.x, (int)a.y, (int)a.z, (int)a.w, (int)b.x, (int)b.y, (int)b.z, (int)b.w};
}

// One workgroup's work (`bid`: its index among the launch's workgroups of this shape).
template <bool GATE_UP, int MT, int NTW>
__device__ __forceinline__ void moe_fp8_body(
    int bid, const uint8_t* __restrict__ aq, const uint8_t* __restrict__ as, const int32_t* __restrict__ perm,
    const int32_t* __restrict__ offsets, int k_top, const float* __restrict__ row_w,
    const uint8_t* __restrict__ packed, int E, int n_shared, int N, int K, int min_rows,
    int max_rows, uint16_t* __restrict__ out) {
  extern __shared__ uint4 f8_lds[];
  constexpr int KC = fp8_chunk(MT);          // K bytes per LDS chunk
  constexpr int SPC = KC / 128;              // MFMA steps per chunk
  constexpr int ROWB = KC + 16;              // padded LDS row
  constexpr int VPR = KC / 16;               // 16-byte vectors per row chunk
  constexpr int SREG = MT * 16 * VPR / 256;  // staging vectors per thread
  const Fp8Geom gm = fp8_geom(E + (n_shared > 0), N, K);
  constexpr int kTilesPerWG = 4 * NTW;
  const int wg_per_e = (gm.NT + kTilesPerWG - 1) / kTilesPerWG;
  const int e = bid / wg_per_e;
  const int wgi = bid % wg_per_e;
  const bool shared = e == E;
  const int row_lo = offsets[e];
  const int n_e = shared ? n_shared : offsets[e + 1] - row_lo;
  if (n_e <= 0 || n_e < min_rows || n_e > max_rows) return;  // uniform over the workgroup
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nt0 = wgi * kTilesPerWG + wave * NTW;
  const int ntw = max(0, min(NTW, gm.NT - nt0));  // waves past the last tile still join barriers
  const int r = lane & 15, g = lane >> 4;
  const int KB = gm.KB;
  char* lds_a = reinterpret_cast<char*>(f8_lds);                          // [MT*16][ROWB]
  uint8_t* lds_s = reinterpret_cast<uint8_t*>(lds_a + MT * 16 * ROWB);    // [MT*16][KB]

  const uint8_t* data = packed + ((size_t)e * gm.NT + nt0) * KB * 2048 + lane * 16;
  const uint32_t* scl = reinterpret_cast<const uint32_t*>(packed + gm.data_bytes) +
                        ((size_t)e * gm.NT + nt0) * gm.KB4 * 64 + lane;
  const size_t tile_stride = (size_t)KB * 2048;
  const size_t scale_stride = (size_t)gm.KB4 * 64;

  auto src_row = [&](int p) __attribute__((always_inline)) -> int {
    if (!GATE_UP) return p;
    if (shared) return p - row_lo;
    return perm ? perm[p] / k_top : p;
  };

  for (int m0 = 0; m0 < n_e; m0 += MT * 16) {
    const int rows = min(MT * 16, n_e - m0);
    // activation source rows of this thread's staging vectors (rows past the pass clamp to row 0)
    const uint8_t* asrc[SREG];
    static_for<0, SREG>([&](auto J) {
      const int i = J * 256 + tid;
      const int rr = i / VPR;
      asrc[J] = aq + (size_t)src_row(row_lo + m0 + (rr < rows ? rr : 0)) * K + (i % VPR) * 16;
    });
    lds_barrier();  // the previous pass is done with LDS (the weight ring stays in flight)
    for (int i = tid; i < MT * 16 * KB; i += 256) {
      const int rr = i / KB, kb = i % KB;
      lds_s[i] = rr < rows ? as[(size_t)src_row(row_lo + m0 + rr) * KB + kb] : (uint8_t)127;
    }
    typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));  // plain loads, no struct copies
    u32x4 stg[SREG];
    static_for<0, SREG>([&](auto J) { stg[J] = *reinterpret_cast<const u32x4*>(asrc[J]); });

    auto load_w = [&](v8i_t (&w)[NTW], int kb) __attribute__((always_inline)) {
      const size_t kk = (size_t)min(kb, KB - 1) * 2048;
#pragma unroll
      for (int n = 0; n < NTW; ++n) w[n] = ld_nt_v8(data + min(n, ntw - 1) * tile_stride + kk);
    };
    auto load_sc = [&](uint32_t (&sc)[NTW], int kb4) __attribute__((always_inline)) {
      const int kk = min(kb4, gm.KB4 - 1) * 64;
#pragma unroll
      for (int n = 0; n < NTW; ++n) sc[n] = scl[min(n, ntw - 1) * scale_stride + kk];
    };
    f32x4_t acc[MT][NTW];
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
      for (int n = 0; n < NTW; ++n) acc[m][n] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    auto compute = [&](const v8i_t (&w)[NTW], const uint32_t (&sc)[NTW], int kb, int b) __attribute__((always_inline)) {
      const int kc = (kb % SPC) * 128 + 32 * g;  // byte offset in the LDS chunk row
#pragma unroll
      for (int m = 0; m < MT; ++m) {
        {  // every row tile, valid or not: rows past the pass hold a clamped row, never stored
          const char* ap = lds_a + (m * 16 + r) * ROWB + kc;
          const uint4 lo = *reinterpret_cast<const uint4*>(ap);
          const uint4 hi = *reinterpret_cast<const uint4*>(ap + 16);
          const v8i_t a = v8i_t{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
          const int sa = lds_s[(m * 16 + r) * KB + kb];
#pragma unroll
          for (int n = 0; n < NTW; ++n)
            acc[m][n] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
                a, w[n], acc[m][n], 0, 0, 0, sa, 0, (int)((sc[n] >> (8 * b)) & 0xffu));
        }
      }
    };

    // The ring runs in static bodies of 4 steps over the whole K; a step that opens a new LDS chunk
    // first switches chunks (every wave takes part, so waves without tiles still meet the barriers).
    const int nchunks = K / KC;
    auto next_chunk = [&](int c) __attribute__((always_inline)) {
      lds_barrier();  // every wave is done with the previous chunk (the weight ring stays in flight)
      static_for<0, SREG>([&](auto J) {
        const int i = J * 256 + tid;
        *reinterpret_cast<u32x4*>(lds_a + (i / VPR) * ROWB + (i % VPR) * 16) = stg[J];
      });
      lds_barrier();
      if (c + 1 < nchunks)
        static_for<0, SREG>([&](auto J) { stg[J] = *reinterpret_cast<const u32x4*>(asrc[J] + (size_t)(c + 1) * KC); });
    };
    v8i_t w0[NTW], w1[NTW], w2[NTW], w3[NTW];
    uint32_t sc_cur[NTW], sc_nxt[NTW];
    const bool has_tiles = ntw > 0;
    if (has_tiles) {
      load_sc(sc_cur, 0);
      load_w(w0, 0);
      load_w(w1, 1);
      load_w(w2, 2);
    }
    for (int kb = 0; kb < KB; kb += 4) {
      if (kb % SPC == 0) next_chunk(kb / SPC);
      if (has_tiles) {
        load_sc(sc_nxt, kb / 4 + 1);
        load_w(w3, kb + 3);
        __builtin_amdgcn_sched_barrier(0);
        compute(w0, sc_cur, kb, 0);
        __builtin_amdgcn_sched_barrier(0);
        load_w(w0, kb + 4);
      }
      if ((kb + 1) % SPC == 0) next_chunk((kb + 1) / SPC);
      if (has_tiles) {
        __builtin_amdgcn_sched_barrier(0);
        compute(w1, sc_cur, kb + 1, 1);
        __builtin_amdgcn_sched_barrier(0);
        load_w(w1, kb + 5);
      }
      if ((kb + 2) % SPC == 0) next_chunk((kb + 2) / SPC);
      if (has_tiles) {
        __builtin_amdgcn_sched_barrier(0);
        compute(w2, sc_cur, kb + 2, 2);
        __builtin_amdgcn_sched_barrier(0);
        load_w(w2, kb + 6);
      }
      if ((kb + 3) % SPC == 0) next_chunk((kb + 3) / SPC);
      if (has_tiles) {
        __builtin_amdgcn_sched_barrier(0);
        compute(w3, sc_cur, kb + 3, 3);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int n = 0; n < NTW; ++n) sc_cur[n] = sc_nxt[n];
      }
    }

    // epilogue: acc[m][n][v] = C[act row m*16 + 4g + v][weight row (nt0+n)*16 + r]
#pragma unroll
    for (int m = 0; m < MT; ++m) {
#pragma unroll
      for (int n = 0; n < NTW; ++n) {
        const int col = (nt0 + n) * 16 + r;
        const bool nval = n < ntw;
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int orow = m * 16 + 4 * g + v;
          const int p = row_lo + m0 + orow;
          if (GATE_UP) {
            const float val = bf16_round(acc[m][n][v]);
            const float up = __shfl_xor(val, 1, 64);
            if (nval && (r & 1) == 0 && orow < rows) {
              const float wt = (row_w && !shared) ? row_w[perm ? perm[p] : p] : 1.0f;
              const float hval = val / (1.0f + expf(-val)) * up * wt;
              out[(size_t)p * (N / 2) + col / 2] = f2bf(hval);
            }
          } else {
            if (nval && orow < rows) out[(size_t)p * N + col] = f2bf(acc[m][n][v]);
          }
        }
      }
    }
  }
}

// Experts with at most kF8TailRows rows take the one-row-tile body (two weight tiles per wave,
// small LDS); larger groups take the 8-row-tile body (one weight tile per wave, 128 rows per pass,
// so groups up to that size stream their weights once).  Both run in one launch, the dense
// workgroups first: the few hot experts' long, latency-bound workgroups start at once and run
// beside the bandwidth-bound row-pass workgroups instead of after them.  Both bodies fit two waves
// per SIMD (at most 244 registers) and the launch's LDS is the larger body's.
constexpr int kF8TailRows = 16;
constexpr int kF8DenseMT = 8;

template <bool GATE_UP>
__global__ __launch_bounds__(256) void moe_fp8_kernel(
    const uint8_t* __restrict__ aq, const uint8_t* __restrict__ as, const int32_t* __restrict__ perm,
    const int32_t* __restrict__ offsets, int k_top, const float* __restrict__ row_w,
    const uint8_t* __restrict__ packed, int E, int n_shared, int N, int K, int dense_wgs,
    uint16_t* __restrict__ out) {
  if ((int)blockIdx.x < dense_wgs)
    moe_fp8_body<GATE_UP, kF8DenseMT, 1>(blockIdx.x, aq, as, perm, offsets, k_top, row_w, packed, E, n_shared,
                                         N, K, kF8TailRows + 1, 1 << 30, out);
  else
    moe_fp8_body<GATE_UP, 1, 2>(blockIdx.x - dense_wgs, aq, as, perm, offsets, k_top, row_w, packed, E,
                                n_shared, N, K, 1, kF8TailRows, out);
}

template <bool GATE_UP>
int launch_moe_fp8(const uint8_t* aq, const uint8_t* as, const int32_t* perm, const int32_t* offsets,
                   int k_top, const float* row_w, const uint8_t* packed, int E, int n_shared, int N,
                   int K, uint16_t* out, hipStream_t s) {
  const Fp8Geom gm = fp8_geom(E, N, K);
  const int groups = E + (n_shared > 0);
  const int dense_wgs = groups * ceil_div(gm.NT, 4), tail_wgs = groups * ceil_div(gm.NT, 8);
  const int lds = std::max(fp8_lds_bytes(kF8DenseMT, K), fp8_lds_bytes(1, K));
  hipLaunchKernelGGL((moe_fp8_kernel<GATE_UP>), dim3(dense_wgs + tail_wgs), dim3(256), lds, s, aq, as, perm,
                     offsets, k_top, row_w, packed, E, n_shared, N, K, dense_wgs, out);
  return check_launch(GATE_UP ? "moe_gate_up_fp8" : "moe_down_fp8");
}

// ---- combine: out[t] = bf16(residual + bf16(sum_s y[inv[t*k+s]] + shared[t])) ------------------------
__global__ __launch_bounds__(256) void moe_combine_sum_kernel(const uint16_t* __restrict__ y,
                                                              const int32_t* __restrict__ inv, int k,
                                                              int H, const uint16_t* __restrict__ shared,
                                                              const uint16_t* residual, uint16_t* out) {
  const int t = blockIdx.x;
  int rows[8];
  for (int s = 0; s < k; ++s) rows[s] = inv[t * k + s];
  for (int i = threadIdx.x; i < H / 4; i += 256) {
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    for (int s = 0; s < k; ++s) {
      const uint2 v = reinterpret_cast<const uint2*>(y + (size_t)rows[s] * H)[i];
      acc[0] += bf2f(v.x & 0xffff); acc[1] += bf2f(v.x >> 16);
      acc[2] += bf2f(v.y & 0xffff); acc[3] += bf2f(v.y >> 16);
    }
    if (shared) {
      const uint2 v = reinterpret_cast<const uint2*>(shared + (size_t)t * H)[i];
      acc[0] += bf2f(v.x & 0xffff); acc[1] += bf2f(v.x >> 16);
      acc[2] += bf2f(v.y & 0xffff); acc[3] += bf2f(v.y >> 16);
    }
    uint16_t o[4];
    if (residual) {
      const uint2 v = reinterpret_cast<const uint2*>(residual + (size_t)t * H)[i];
      const float rv[4] = {bf2f(v.x & 0xffff), bf2f(v.x >> 16), bf2f(v.y & 0xffff), bf2f(v.y >> 16)};
#pragma unroll
      for (int c = 0; c < 4; ++c) o[c] = f2bf(rv[c] + bf16_round(acc[c]));
    } else {
#pragma unroll
      for (int c = 0; c < 4; ++c) o[c] = f2bf(acc[c]);
    }
    uint2 ov;
    ov.x = (uint32_t)o[0] | ((uint32_t)o[1] << 16);
    ov.y = (uint32_t)o[2] | ((uint32_t)o[3] << 16);
    reinterpret_cast<uint2*>(out + (size_t)t * H)[i] = ov;
  }
}

}  // namespace flyai

using namespace flyai;

extern "C" int flyai_fp8_act_quant(const uint16_t* x, int32_t M, int32_t K, uint8_t* q, uint8_t* s,
                                   flyai_stream_t stream) {
  FLYAI_REQUIRE(M >= 0 && K > 0 && K % 128 == 0, "act_quant: need K %% 128 == 0");
  FLYAI_REQUIRE(x && q && s, "act_quant: null pointer");
  return launch_act_quant_fp8(x, M, K, q, s, as_stream(stream));
}

extern "C" size_t flyai_fp8_packed_bytes(int32_t E, int32_t N, int32_t K) {
  if (E <= 0 || N <= 0 || K <= 0 || N % 16 || K % 1024) return 0;
  const Fp8Geom g = fp8_geom(E, N, K);
  return g.data_bytes + (size_t)E * g.NT * g.KB4 * 256;
}

extern "C" int flyai_fp8_repack(const uint8_t* w1, const uint8_t* s1, const uint8_t* w3,
                                const uint8_t* s3, int32_t E, int32_t N, int32_t K, uint8_t* packed,
                                flyai_stream_t stream) {
  FLYAI_REQUIRE(E > 0 && N > 0 && K > 0 && N % 16 == 0 && K % 1024 == 0 && K <= 8192,
                "fp8_repack: need N %% 16 == 0, K %% 1024 == 0, K <= 8192");
  FLYAI_REQUIRE(w1 && s1 && packed && ((w3 == nullptr) == (s3 == nullptr)), "fp8_repack: null pointer");
  const int Np = w3 ? 2 * N : N;
  const Fp8Geom gm = fp8_geom(E, Np, K);
  const size_t total = (size_t)E * gm.NT * gm.KB * 64;
  hipLaunchKernelGGL(fp8_repack_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                     as_stream(stream), w1, s1, w3, s3, E, N, K, packed);
  return check_launch("fp8_repack");
}

extern "C" int flyai_moe_gate_up_fp8(const uint8_t* xq, const uint8_t* xs, const int32_t* perm,
                                     const int32_t* offsets, int32_t k, const float* topk_w,
                                     const uint8_t* w13_packed, int32_t E, int32_t H, int32_t I,
                                     int32_t n_shared, uint16_t* h, flyai_stream_t stream) {
  FLYAI_REQUIRE(E > 0 && H > 0 && I > 0 && H % 1024 == 0 && H <= 8192 && I % 8 == 0 && k >= 1 &&
                    n_shared >= 0,
                "gate_up_fp8: need H %% 1024 == 0, H <= 8192, I %% 8 == 0, n_shared >= 0");
  FLYAI_REQUIRE(xq && xs && offsets && w13_packed && h, "gate_up_fp8: null pointer");
  return launch_moe_fp8<true>(xq, xs, perm, offsets, k, topk_w, w13_packed, E, n_shared, 2 * I, H, h,
                              as_stream(stream));
}

extern "C" int flyai_moe_down_fp8(const uint8_t* hq, const uint8_t* hs, const int32_t* offsets,
                                  const uint8_t* w2_packed, int32_t E, int32_t H, int32_t I,
                                  int32_t n_shared, uint16_t* y, flyai_stream_t stream) {
  FLYAI_REQUIRE(E > 0 && H > 0 && I > 0 && I % 1024 == 0 && I <= 8192 && H % 16 == 0 && n_shared >= 0,
                "down_fp8: need I %% 1024 == 0, I <= 8192, H %% 16 == 0, n_shared >= 0");
  FLYAI_REQUIRE(hq && hs && offsets && w2_packed && y, "down_fp8: null pointer");
  return launch_moe_fp8<false>(hq, hs, nullptr, offsets, 1, nullptr, w2_packed, E, n_shared, H, I, y,
                               as_stream(stream));
}

extern "C" int flyai_moe_combine_sum(const uint16_t* y_perm, const int32_t* inv, int32_t T, int32_t k,
                                     int32_t H, const uint16_t* shared, const uint16_t* residual,
                                     uint16_t* out, flyai_stream_t stream) {
  FLYAI_REQUIRE(T >= 0 && k >= 1 && k <= 8 && H > 0 && H % 4 == 0, "combine_sum: bad shape");
  FLYAI_REQUIRE(y_perm && inv && out, "combine_sum: null pointer");
  if (T == 0) return FLYAI_OK;
  hipLaunchKernelGGL(moe_combine_sum_kernel, dim3(T), dim3(256), 0, as_stream(stream), y_perm, inv, k, H,
                     shared, residual, out);
  return check_launch("moe_combine_sum");
}
