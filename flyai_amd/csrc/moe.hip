// MXFP4 expert FFN for GPT-OSS: re-pack, gate_up (+ fused SwiGLU) and down kernels.
//
// Packed layout of one MXFP4 weight W[E][N][K] (N output rows, K inputs, G = K/32 blocks/row):
//   data   : [E][N/16 tiles][G*256 bytes].  Within a tile, group kg covers blocks 4kg..4kg+3 and
//            sits at byte kg*1024: lane l = 16*g + r holds the 16 bytes (32 E2M1 codes) of row r,
//            block 4kg+g.  A wave's 16-byte load per lane therefore reads one contiguous KiB.  The
//            last group holds only the G-4*(KG-1) existing blocks (no padding in the data).
//   scales : [E][N/16][KG4*256 bytes] after all data; dword (kg4, lane) holds the E8M0 scales of
//            (row r, block 4kg+g) for kg = 4kg4 .. 4kg4+3 in bytes 0..3 (0 past the end).
//
// The MFMA (v_mfma_f32_16x16x32_bf16) sees activations as A (16 rows x 32 K) and dequantised
// weights as B (32 K x 16 output features).  Because any consistent permutation of K is allowed
// in a dot product, lane (r, g) supplies, at MFMA step j of group kg, the 8 K values
// 32*(4kg+g) + 8j .. +7 for BOTH operands: the lane's 16 weight bytes feed four MFMA steps and
// its activation bytes are the matching 64 contiguous bytes of the activation row.
#include <type_traits>

#include "common.h"

namespace flyai {

struct MxGeom {
  int NT, G, KG, KG4;
  size_t data_bytes;  // whole data region (all experts)
};

__host__ __device__ inline MxGeom mx_geom(int E, int N, int K) {
  MxGeom g;
  g.NT = N / 16;
  g.G = K / 32;
  g.KG = (g.G + 3) / 4;
  g.KG4 = (g.KG + 3) / 4;
  g.data_bytes = (size_t)E * g.NT * g.G * 256;
  return g;
}

// ---- re-pack: HF blocks [E][N][G][16] + scales [E][N][G] -> tile layout -------------------------
__global__ __launch_bounds__(256) void mxfp4_repack_kernel(const uint8_t* __restrict__ blocks,
                                                           const uint8_t* __restrict__ scales,
                                                           int E, int N, int K,
                                                           uint8_t* __restrict__ packed) {
  const MxGeom gm = mx_geom(E, N, K);
  const size_t total = (size_t)E * gm.NT * gm.KG * 64;
  const size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= total) return;
  const int lane = idx % 64;
  const int kg = (idx / 64) % gm.KG;
  const size_t et = idx / 64 / gm.KG;  // e * NT + nt
  const int nt = et % gm.NT;
  const int e = et / gm.NT;
  const int r = lane & 15, g = lane >> 4;
  const int row = nt * 16 + r, blk = kg * 4 + g;
  if (blk < gm.G) {
    const uint4 v = *reinterpret_cast<const uint4*>(blocks + (((size_t)e * N + row) * gm.G + blk) * 16);
    *reinterpret_cast<uint4*>(packed + et * gm.G * 256 + (size_t)kg * 1024 + lane * 16) = v;
  }
  if ((kg & 3) == 0) {
    uint32_t word = 0;
    for (int i = 0; i < 4; ++i) {
      const int b2 = (kg + i) * 4 + g;
      if (kg + i < gm.KG && b2 < gm.G)
        word |= (uint32_t)scales[((size_t)e * N + row) * gm.G + b2] << (8 * i);
    }
    reinterpret_cast<uint32_t*>(packed + gm.data_bytes + et * gm.KG4 * 256)[(kg / 4) * 64 + lane] = word;
  }
}

// ---- expert kernels ---------------------------------------------------------------------------
// Workgroup = 4 waves = 4*NTW weight tiles (16 output rows each) of one expert, full K.  The
// expert's activation rows are staged in LDS, kRowsPerPass at a time, with fully coalesced loads
// (one pass serves every tile of the workgroup), so the only vector-memory loads in the K loop are
// the weights: 1 KiB per tile per group of 128 K, streamed through a 4-deep register ring with
// non-temporal loads (3 groups in flight while one computes).  Each group is dequantised in registers (gfx950 v_cvt_scalef32_pk_bf16_fp4,
// E8M0 scale in the exponent field) and fed to v_mfma_f32_16x16x32_bf16 with the activation
// fragment read from LDS (rows >= the pass's row count read as zero).  Larger groups take further
// passes over the weights.
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint4 ld_nt(const uint8_t* p) {
  const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ float swiglu_gptoss(float gate, float up) {
  // modeling_gpt_oss.py:82-88: gate clamped above at 7, up clamped to [-7, 7]
  const float g = fminf(gate, 7.0f);
  const float u = fminf(fmaxf(up, -7.0f), 7.0f);
  const float glu = g * (1.0f / (1.0f + __expf(-1.702f * g)));
  return (u + 1.0f) * glu;
}

constexpr int kRowsPerPass = 8;

__host__ __device__ inline int mx_lds_row_bytes(int K) { return K * 2 + 16; }  // +16 B vs bank conflicts

template <bool GATE_UP, int NTW>
__global__ __launch_bounds__(256) void moe_mxfp4_kernel(
    const uint16_t* __restrict__ act, const int32_t* __restrict__ perm,
    const int32_t* __restrict__ offsets, int k_top, const uint8_t* __restrict__ packed,
    const float* __restrict__ bias, int E, int N, int K, int min_rows, int max_rows,
    void* __restrict__ out) {
  extern __shared__ uint4 xs_lds[];  // [kRowsPerPass][K*2+16 bytes]
  const MxGeom gm = mx_geom(E, N, K);
  constexpr int kTilesPerWG = 4 * NTW;
  const int wg_per_e = (gm.NT + kTilesPerWG - 1) / kTilesPerWG;
  const int e = blockIdx.x / wg_per_e;
  const int wgi = blockIdx.x % wg_per_e;
  const int row_lo = offsets[e];
  const int n_e = offsets[e + 1] - row_lo;
  if (n_e <= 0 || n_e < min_rows || n_e > max_rows) return;  // uniform over the workgroup
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nt0 = wgi * kTilesPerWG + wave * NTW;
  const int ntw = max(0, min(NTW, gm.NT - nt0));  // waves past the last tile still join the barriers
  const int r = lane & 15, g = lane >> 4;
  const int row_bytes = mx_lds_row_bytes(K);
  const int row_vecs = K / 8;  // 16-byte vectors per activation row

  const uint8_t* data = packed + ((size_t)e * gm.NT + nt0) * gm.G * 256 + lane * 16;
  const uint32_t* scl = reinterpret_cast<const uint32_t*>(
                            packed + gm.data_bytes + ((size_t)e * gm.NT + nt0) * gm.KG4 * 256) + lane;
  const size_t tile_stride = (size_t)gm.G * 256;
  const size_t scale_stride = (size_t)gm.KG4 * 64;
  const char* lds = reinterpret_cast<const char*>(xs_lds);

  for (int m0 = 0; m0 < n_e; m0 += kRowsPerPass) {
    const int rows = min(kRowsPerPass, n_e - m0);
    __syncthreads();  // the previous pass is done with the LDS rows
    // staging loads go out in batches of 4 per thread (one round trip per batch, not per vector);
    // indices past the end are clamped for the load and not stored
    const int total = rows * row_vecs;
    for (int b0 = 0; b0 < total; b0 += 4 * 256) {
      u32x4_t v4[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int i = min(b0 + j * 256 + (int)threadIdx.x, total - 1);
        const int rr = i / row_vecs, v = i % row_vecs;
        const int p = row_lo + m0 + rr;
        const int src = GATE_UP ? perm[p] / k_top : p;
        v4[j] = reinterpret_cast<const u32x4_t*>(act + (size_t)src * K)[v];
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int i = b0 + j * 256 + (int)threadIdx.x;
        if (i < total)
          *reinterpret_cast<u32x4_t*>(const_cast<char*>(lds) + (i / row_vecs) * row_bytes + (i % row_vecs) * 16) = v4[j];
      }
    }
    __syncthreads();
    if (ntw == 0) continue;
    const bool aval = r < rows;
    const char* arow = lds + r * row_bytes + 64 * g;

    auto load_w = [&](uint4 (&w)[NTW], int kg) {
      const bool bvalid = kg < gm.KG && 4 * kg + g < gm.G;
#pragma unroll
      for (int n = 0; n < NTW; ++n)
        w[n] = (bvalid && n < ntw) ? ld_nt(data + n * tile_stride + (size_t)kg * 1024) : make_uint4(0, 0, 0, 0);
    };
    auto load_sc = [&](uint32_t (&sc)[NTW], int kg4) {
#pragma unroll
      for (int n = 0; n < NTW; ++n) sc[n] = (kg4 < gm.KG4 && n < ntw) ? scl[n * scale_stride + kg4 * 64] : 0u;
    };
    f32x4_t acc[NTW];
#pragma unroll
    for (int n = 0; n < NTW; ++n) acc[n] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    // byte b of sc[n] is the E8M0 scale of group 4*kg4 + b
    auto compute = [&](const uint4 (&w)[NTW], const uint32_t (&sc)[NTW], int kg, int b) {
      uint4 a[4];
      const bool ok = aval && kg < gm.KG && 4 * kg + g < gm.G;
#pragma unroll
      for (int j = 0; j < 4; ++j)
        a[j] = ok ? *reinterpret_cast<const uint4*>(arow + 256 * kg + 16 * j) : make_uint4(0, 0, 0, 0);
#pragma unroll
      for (int n = 0; n < NTW; ++n) {
        const float scale = e8m0_operand((sc[n] >> (8 * b)) & 0xffu);
        const uint32_t wd[4] = {w[n].x, w[n].y, w[n].z, w[n].w};
#pragma unroll
        for (int j = 0; j < 4; ++j)
          acc[n] = mfma16x16x32(as_bf16x8(a[j]), fp4x8_to_bf16x8(wd[j], scale), acc[n]);
      }
    };

    // Static bodies of 4 groups: a 4-deep weight ring (3 groups in flight while one computes) and
    // the next body's scale dword loaded one body ahead, so no wait ever drains the ring.
    uint4 w0[NTW], w1[NTW], w2[NTW], w3[NTW];
    uint32_t sc_cur[NTW], sc_nxt[NTW];
    load_sc(sc_cur, 0);
    load_w(w0, 0);
    load_w(w1, 1);
    load_w(w2, 2);
    for (int kg4 = 0; kg4 < gm.KG4; ++kg4) {
      const int kg = 4 * kg4;
      load_sc(sc_nxt, kg4 + 1);
      load_w(w3, kg + 3);
      compute(w0, sc_cur, kg, 0);
      load_w(w0, kg + 4);
      compute(w1, sc_cur, kg + 1, 1);
      load_w(w1, kg + 5);
      compute(w2, sc_cur, kg + 2, 2);
      load_w(w2, kg + 6);
      compute(w3, sc_cur, kg + 3, 3);
#pragma unroll
      for (int n = 0; n < NTW; ++n) sc_cur[n] = sc_nxt[n];
    }

    // epilogue: lane holds D[act row 4g+v][feature r] of each tile
#pragma unroll
    for (int n = 0; n < NTW; ++n) {
      const int feat = (nt0 + n) * 16 + r;
      const bool nval = n < ntw;
      const float bsum = nval ? bias[(size_t)e * N + feat] : 0.f;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int orow = 4 * g + v;
        const float val = acc[n][v] + bsum;
        if (GATE_UP) {
          const float partner = __shfl_xor(val, 1, 64);
          if (nval && (r & 1) == 0 && orow < rows)
            reinterpret_cast<uint16_t*>(out)[(size_t)(row_lo + m0 + orow) * (N / 2) + feat / 2] =
                f2bf(swiglu_gptoss(val, partner));
        } else {
          if (nval && orow < rows)
            reinterpret_cast<float*>(out)[(size_t)(row_lo + m0 + orow) * N + feat] = val;
        }
      }
    }
  }
}

constexpr int kNTW = 2;  // weight tiles per wave

// ---- dense groups ------------------------------------------------------------------------------
// Groups of many rows (chunked prefill, skewed routing) take MT row tiles per pass so the expert's
// weights stream once per MT*16 rows: one weight tile per wave, the same 4-deep non-temporal ring
// and scale prefetch as above, and the bf16 activation rows staged in LDS one 128-K group at a
// time.  The staging loads of group c+1 are issued into registers before group c's ring loads
// (vector-memory waits complete in issue order, so a later wait on them never drains the ring) and
// stored at the next group boundary.  Loads are unconditional with clamped addresses: weight lanes
// past the last block of a row are zeroed by select, activation loads past the row end read a
// valid element of the row (multiplied by those zero weights); rows past the pass read row 0 and
// are never stored.
template <int B, int N, class F>
__device__ __forceinline__ void mx_static_for(F&& f) {
  if constexpr (B < N) {
    f(std::integral_constant<int, B>{});
    mx_static_for<B + 1, N>(f);
  }
}

template <bool GATE_UP, int MT>
__global__ __launch_bounds__(256) void moe_mxfp4_dense_kernel(
    const uint16_t* __restrict__ act, const int32_t* __restrict__ perm,
    const int32_t* __restrict__ offsets, int k_top, const uint8_t* __restrict__ packed,
    const float* __restrict__ bias, int E, int N, int K, int min_rows, void* __restrict__ out) {
  typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
  extern __shared__ uint4 xd_lds[];
  constexpr int KC = 256;                    // bytes of a bf16 row per chunk: one group of 128 K
  constexpr int ROWB = KC + 16;              // padded LDS row
  constexpr int VPR = KC / 16;               // 16-byte vectors per row chunk
  constexpr int SREG = MT * 16 * VPR / 256;  // staging vectors per thread
  const MxGeom gm = mx_geom(E, N, K);
  const int wg_per_e = (gm.NT + 3) / 4;
  const int e = blockIdx.x / wg_per_e;
  const int wgi = blockIdx.x % wg_per_e;
  const int row_lo = offsets[e];
  const int n_e = offsets[e + 1] - row_lo;
  if (n_e <= 0 || n_e < min_rows) return;  // uniform over the workgroup
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nt = wgi * 4 + wave;
  const bool has_tile = nt < gm.NT;         // waves past the last tile still join the barriers
  const int ntc = min(nt, gm.NT - 1);
  const int r = lane & 15, g = lane >> 4;
  char* lds = reinterpret_cast<char*>(xd_lds);
  const uint8_t* data = packed + ((size_t)e * gm.NT + ntc) * gm.G * 256 + lane * 16;
  const uint32_t* scl = reinterpret_cast<const uint32_t*>(packed + gm.data_bytes + ((size_t)e * gm.NT + ntc) * gm.KG4 * 256) + lane;

  for (int m0 = 0; m0 < n_e; m0 += MT * 16) {
    const int rows = min(MT * 16, n_e - m0);
    const uint16_t* asrc[SREG];
    int acol[SREG];
    mx_static_for<0, SREG>([&](auto J) {
      const int i = J * 256 + tid;
      const int rr = i / VPR;
      const int p = row_lo + m0 + (rr < rows ? rr : 0);
      asrc[J] = act + (size_t)(GATE_UP ? perm[p] / k_top : p) * K;
      acol[J] = (i % VPR) * 8;   // element offset within the chunk
    });
    auto stage_load = [&](u32x4 (&st)[SREG], int c) __attribute__((always_inline)) {
      mx_static_for<0, SREG>([&](auto J) {
        const int col = c * 128 + acol[J];
        st[J] = *reinterpret_cast<const u32x4*>(asrc[J] + (col < K ? col : acol[J]));
      });
    };
    u32x4 stg[SREG];
    stage_load(stg, 0);
    auto next_chunk = [&](int c) __attribute__((always_inline)) {
      __syncthreads();  // every wave is done with the previous chunk
      mx_static_for<0, SREG>([&](auto J) {
        const int i = J * 256 + tid;
        *reinterpret_cast<u32x4*>(lds + (i / VPR) * ROWB + (i % VPR) * 16) = stg[J];
      });
      __syncthreads();
      if (c + 1 < gm.KG) stage_load(stg, c + 1);
    };
    auto load_w = [&](int kg) __attribute__((always_inline)) -> uint4 {
      // lanes past the row's last block (and look-ahead past K) load group 0 and are zeroed
      const bool ok = kg < gm.KG && 4 * kg + g < gm.G;
      const uint4 v = ld_nt(data + (ok ? (size_t)kg * 1024 : 0));
      return ok ? v : make_uint4(0, 0, 0, 0);
    };
    auto load_sc = [&](int kg4) __attribute__((always_inline)) -> uint32_t {
      return scl[min(kg4, gm.KG4 - 1) * 64];
    };
    f32x4_t acc[MT];
#pragma unroll
    for (int m = 0; m < MT; ++m) acc[m] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    auto compute = [&](uint4 w, uint32_t sc, int b) __attribute__((always_inline)) {
      const float scale = e8m0_operand((sc >> (8 * b)) & 0xffu);
      const uint32_t wd[4] = {w.x, w.y, w.z, w.w};
      bf16x8_t bw[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) bw[j] = fp4x8_to_bf16x8(wd[j], scale);
#pragma unroll
      for (int m = 0; m < MT; ++m) {
        const char* ap = lds + (m * 16 + r) * ROWB + 64 * g;
#pragma unroll
        for (int j = 0; j < 4; ++j)
          acc[m] = mfma16x16x32(as_bf16x8(*reinterpret_cast<const uint4*>(ap + 16 * j)), bw[j], acc[m]);
      }
    };

    uint4 w0, w1, w2, w3;
    uint32_t sc_cur = 0, sc_nxt = 0;
    if (has_tile) {
      sc_cur = load_sc(0);
      w0 = load_w(0);
      w1 = load_w(1);
      w2 = load_w(2);
    }
    for (int kg = 0; kg < gm.KG4 * 4; kg += 4) {
      // chunk switches happen for every existing group; groups past KG (the last body's tail) skip
      if (kg < gm.KG) next_chunk(kg);
      if (has_tile) {
        sc_nxt = load_sc(kg / 4 + 1);
        w3 = load_w(kg + 3);
        if (kg < gm.KG) compute(w0, sc_cur, 0);
        w0 = load_w(kg + 4);
      }
      if (kg + 1 < gm.KG) next_chunk(kg + 1);
      if (has_tile) {
        if (kg + 1 < gm.KG) compute(w1, sc_cur, 1);
        w1 = load_w(kg + 5);
      }
      if (kg + 2 < gm.KG) next_chunk(kg + 2);
      if (has_tile) {
        if (kg + 2 < gm.KG) compute(w2, sc_cur, 2);
        w2 = load_w(kg + 6);
      }
      if (kg + 3 < gm.KG) next_chunk(kg + 3);
      if (has_tile) {
        if (kg + 3 < gm.KG) compute(w3, sc_cur, 3);
        sc_cur = sc_nxt;
      }
    }

    // epilogue: acc[m][v] = D[act row m*16 + 4g + v][feature nt*16 + r]
    const int feat = ntc * 16 + r;
    const float bsum = bias[(size_t)e * N + feat];
#pragma unroll
    for (int m = 0; m < MT; ++m) {
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int orow = m * 16 + 4 * g + v;
        const float val = acc[m][v] + bsum;
        if (GATE_UP) {
          const float partner = __shfl_xor(val, 1, 64);
          if (has_tile && (r & 1) == 0 && orow < rows)
            reinterpret_cast<uint16_t*>(out)[(size_t)(row_lo + m0 + orow) * (N / 2) + feat / 2] =
                f2bf(swiglu_gptoss(val, partner));
        } else {
          if (has_tile && orow < rows)
            reinterpret_cast<float*>(out)[(size_t)(row_lo + m0 + orow) * N + feat] = val;
        }
      }
    }
  }
}

// Groups of more than kDenseFrom rows take the dense kernel when the batch averages at least that
// many rows per expert (otherwise the row-pass kernel serves every group: a rare large group costs
// extra passes, not a launch of mostly idle workgroups).  Both kernels are correct for any count.
constexpr int kDenseFrom = 8;
constexpr int kDenseMT = 6;  // 96 rows per pass

inline bool use_dense(int rows_total, int E) { return (int64_t)rows_total >= (int64_t)kDenseFrom * E; }

int launch_moe_gate_up(const uint16_t* x, const int32_t* perm, const int32_t* offsets, int k_top,
                       const uint8_t* w13, const float* b13, int T, int E, int H, int I, uint16_t* h,
                       hipStream_t s) {
  const MxGeom gm = mx_geom(E, 2 * I, H);
  const bool dense = use_dense(T * k_top, E);
  if (H <= 4064) {
    const int wg_per_e = ceil_div(gm.NT, 4 * kNTW);
    hipLaunchKernelGGL((moe_mxfp4_kernel<true, kNTW>), dim3(E * wg_per_e), dim3(256),
                       kRowsPerPass * mx_lds_row_bytes(H), s, x, perm, offsets, k_top, w13, b13, E,
                       2 * I, H, 1, dense ? kDenseFrom : (1 << 30), (void*)h);
    int rc = check_launch("moe_gate_up_mxfp4");
    if (rc) return rc;
  }
  if (dense || H > 4064) {
    hipLaunchKernelGGL((moe_mxfp4_dense_kernel<true, kDenseMT>), dim3(E * ceil_div(gm.NT, 4)), dim3(256),
                       kDenseMT * 16 * 272, s, x, perm, offsets, k_top, w13, b13, E, 2 * I, H,
                       H > 4064 ? 1 : kDenseFrom + 1, (void*)h);
    return check_launch("moe_gate_up_mxfp4(dense)");
  }
  return FLYAI_OK;
}

int launch_moe_down(const uint16_t* h, const int32_t* offsets, const uint8_t* w2, const float* b2,
                    int rows_total, int E, int H, int I, float* y, hipStream_t s) {
  const MxGeom gm = mx_geom(E, H, I);
  const bool dense = use_dense(rows_total, E);
  if (I <= 4064) {
    const int wg_per_e = ceil_div(gm.NT, 4 * kNTW);
    hipLaunchKernelGGL((moe_mxfp4_kernel<false, kNTW>), dim3(E * wg_per_e), dim3(256),
                       kRowsPerPass * mx_lds_row_bytes(I), s, h, nullptr, offsets, 1, w2, b2, E, H, I, 1,
                       dense ? kDenseFrom : (1 << 30), (void*)y);
    int rc = check_launch("moe_down_mxfp4");
    if (rc) return rc;
  }
  if (dense || I > 4064) {
    hipLaunchKernelGGL((moe_mxfp4_dense_kernel<false, kDenseMT>), dim3(E * ceil_div(gm.NT, 4)), dim3(256),
                       kDenseMT * 16 * 272, s, h, nullptr, offsets, 1, w2, b2, E, H, I,
                       I > 4064 ? 1 : kDenseFrom + 1, (void*)y);
    return check_launch("moe_down_mxfp4(dense)");
  }
  return FLYAI_OK;
}

}  // namespace flyai

using namespace flyai;

extern "C" size_t flyai_mxfp4_packed_bytes(int32_t E, int32_t N, int32_t K) {
  if (E <= 0 || N <= 0 || K <= 0 || N % 16 || K % 32) return 0;
  const MxGeom g = mx_geom(E, N, K);
  return g.data_bytes + (size_t)E * g.NT * g.KG4 * 256;
}

extern "C" int flyai_mxfp4_repack(const uint8_t* blocks, const uint8_t* scales, int32_t E, int32_t N,
                                  int32_t K, uint8_t* packed, flyai_stream_t stream) {
  FLYAI_REQUIRE(E > 0 && N > 0 && K > 0 && N % 16 == 0 && K % 32 == 0,
                "repack: need N %% 16 == 0 and K %% 32 == 0");
  FLYAI_REQUIRE(blocks && scales && packed, "repack: null pointer");
  const MxGeom gm = mx_geom(E, N, K);
  const size_t total = (size_t)E * gm.NT * gm.KG * 64;
  hipLaunchKernelGGL(mxfp4_repack_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                     as_stream(stream), blocks, scales, E, N, K, packed);
  return check_launch("mxfp4_repack");
}

extern "C" int flyai_moe_gate_up_mxfp4(const uint16_t* x, const int32_t* perm,
                                       const int32_t* offsets, int32_t T, int32_t k,
                                       const uint8_t* w13_packed, const float* b13, int32_t E,
                                       int32_t H, int32_t I, uint16_t* h, flyai_stream_t stream) {
  FLYAI_REQUIRE(T >= 0 && E > 0 && H > 0 && I > 0 && H % 32 == 0 && (2 * I) % 16 == 0 && k >= 1,
                "gate_up: need H %% 32 == 0, 2I %% 16 == 0");
  FLYAI_REQUIRE(x && perm && offsets && w13_packed && b13 && h, "gate_up: null pointer");
  return launch_moe_gate_up(x, perm, offsets, k, w13_packed, b13, T, E, H, I, h, as_stream(stream));
}

extern "C" int flyai_moe_down_mxfp4(const uint16_t* h, const int32_t* offsets, int32_t rows,
                                    const uint8_t* w2_packed, const float* b2, int32_t E, int32_t H,
                                    int32_t I, float* y_perm, flyai_stream_t stream) {
  FLYAI_REQUIRE(rows >= 0 && E > 0 && H > 0 && I > 0 && I % 32 == 0 && H % 16 == 0,
                "down: need I %% 32 == 0, H %% 16 == 0");
  FLYAI_REQUIRE(h && offsets && w2_packed && b2 && y_perm, "down: null pointer");
  return launch_moe_down(h, offsets, w2_packed, b2, rows, E, H, I, y_perm, as_stream(stream));
}
