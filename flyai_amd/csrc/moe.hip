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
constexpr int kMT = 2;   // 16-row activation tiles per pass (32 rows)
constexpr int kNTW = 2;  // 16-row weight tiles per wave

__device__ __forceinline__ float swiglu_gptoss(float gate, float up) {
  // modeling_gpt_oss.py:82-88: gate clamped above at 7, up clamped to [-7, 7]
  const float g = fminf(gate, 7.0f);
  const float u = fminf(fmaxf(up, -7.0f), 7.0f);
  const float glu = g * (1.0f / (1.0f + __expf(-1.702f * g)));
  return (u + 1.0f) * glu;
}

template <bool GATE_UP>
__global__ __launch_bounds__(256) void moe_mxfp4_kernel(
    const uint16_t* __restrict__ act, const int32_t* __restrict__ perm,
    const int32_t* __restrict__ offsets, int k_top, const uint8_t* __restrict__ packed,
    const float* __restrict__ bias, int E, int N, int K, void* __restrict__ out) {
  const MxGeom gm = mx_geom(E, N, K);
  constexpr int kTilesPerWG = 4 * kNTW;
  const int wg_per_e = (gm.NT + kTilesPerWG - 1) / kTilesPerWG;
  const int e = blockIdx.x / wg_per_e;
  const int wgi = blockIdx.x % wg_per_e;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nt0 = wgi * kTilesPerWG + wave * kNTW;
  if (nt0 >= gm.NT) return;
  const int row_lo = offsets[e];
  const int n_e = offsets[e + 1] - row_lo;
  if (n_e <= 0) return;
  const int r = lane & 15, g = lane >> 4;
  const int ntw = min(kNTW, gm.NT - nt0);

  const uint8_t* data = packed + ((size_t)e * gm.NT + nt0) * gm.G * 256 + lane * 16;
  const uint32_t* scl = reinterpret_cast<const uint32_t*>(
                            packed + gm.data_bytes + ((size_t)e * gm.NT + nt0) * gm.KG4 * 256) + lane;
  const size_t tile_stride = (size_t)gm.G * 256;
  const size_t scale_stride = (size_t)gm.KG4 * 64;

  for (int m0 = 0; m0 < n_e; m0 += 16 * kMT) {
    const int mt_count = min(kMT, (n_e - m0 + 15) / 16);
    const uint16_t* arow[kMT];
    bool aval[kMT];
#pragma unroll
    for (int m = 0; m < kMT; ++m) {
      const int row = m0 + 16 * m + r;
      aval[m] = row < n_e;
      int src = 0;
      if (aval[m]) src = GATE_UP ? perm[row_lo + row] / k_top : row_lo + row;
      arow[m] = act + (size_t)src * K;
    }
    f32x4_t acc[kMT][kNTW];
#pragma unroll
    for (int m = 0; m < kMT; ++m)
#pragma unroll
      for (int n = 0; n < kNTW; ++n) acc[m][n] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    uint4 wq[kNTW], wq_next[kNTW];
    uint32_t scw[kNTW];
    {
      const bool bv = g < gm.G;
#pragma unroll
      for (int n = 0; n < kNTW; ++n)
        wq[n] = (bv && n < ntw) ? *reinterpret_cast<const uint4*>(data + n * tile_stride)
                                : make_uint4(0, 0, 0, 0);
    }
    for (int kg = 0; kg < gm.KG; ++kg) {
      const int blk = 4 * kg + g;
      const bool bvalid = blk < gm.G;
      // prefetch next group's weights
      if (kg + 1 < gm.KG) {
        const bool nv = (blk + 4) < gm.G;
#pragma unroll
        for (int n = 0; n < kNTW; ++n)
          wq_next[n] = (nv && n < ntw)
                           ? *reinterpret_cast<const uint4*>(data + n * tile_stride + (size_t)(kg + 1) * 1024)
                           : make_uint4(0, 0, 0, 0);
      }
      if ((kg & 3) == 0) {
#pragma unroll
        for (int n = 0; n < kNTW; ++n) scw[n] = (n < ntw) ? scl[n * scale_stride + (kg >> 2) * 64] : 0u;
      }
      uint4 a[kMT][4];
#pragma unroll
      for (int m = 0; m < kMT; ++m) {
        if (aval[m] && bvalid) {
          const uint4* ap = reinterpret_cast<const uint4*>(arow[m] + blk * 32);
#pragma unroll
          for (int j = 0; j < 4; ++j) a[m][j] = ap[j];
        } else {
#pragma unroll
          for (int j = 0; j < 4; ++j) a[m][j] = make_uint4(0, 0, 0, 0);
        }
      }
      float sc[kNTW];
#pragma unroll
      for (int n = 0; n < kNTW; ++n) sc[n] = e8m0_operand((scw[n] >> (8 * (kg & 3))) & 0xffu);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
#pragma unroll
        for (int n = 0; n < kNTW; ++n) {
          const uint32_t word = j == 0 ? wq[n].x : j == 1 ? wq[n].y : j == 2 ? wq[n].z : wq[n].w;
          const bf16x8_t bw = fp4x8_to_bf16x8(word, sc[n]);
#pragma unroll
          for (int m = 0; m < kMT; ++m)
            if (m < mt_count) acc[m][n] = mfma16x16x32(as_bf16x8(a[m][j]), bw, acc[m][n]);
        }
      }
#pragma unroll
      for (int n = 0; n < kNTW; ++n) wq[n] = wq_next[n];
    }
    // epilogue: lane holds D[act row 4g+v][feature r] of each (m, n) tile
#pragma unroll
    for (int n = 0; n < kNTW; ++n) {
      const int feat = (nt0 + n) * 16 + r;
      const bool nval = n < ntw;
      const float bsum = nval ? bias[(size_t)e * N + feat] : 0.f;
#pragma unroll
      for (int m = 0; m < kMT; ++m) {
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int row = m0 + 16 * m + 4 * g + v;
          const float val = acc[m][n][v] + bsum;
          if (GATE_UP) {
            const float partner = __shfl_xor(val, 1, 64);
            if (nval && (r & 1) == 0 && row < n_e && m < mt_count) {
              const float hval = swiglu_gptoss(val, partner);
              reinterpret_cast<uint16_t*>(out)[(size_t)(row_lo + row) * (N / 2) + feat / 2] = f2bf(hval);
            }
          } else {
            if (nval && row < n_e && m < mt_count)
              reinterpret_cast<float*>(out)[(size_t)(row_lo + row) * N + feat] = val;
          }
        }
      }
    }
  }
}

int launch_moe_gate_up(const uint16_t* x, const int32_t* perm, const int32_t* offsets, int k_top,
                       const uint8_t* w13, const float* b13, int E, int H, int I, uint16_t* h,
                       hipStream_t s) {
  const MxGeom gm = mx_geom(E, 2 * I, H);
  const int wg_per_e = ceil_div(gm.NT, 4 * kNTW);
  hipLaunchKernelGGL(moe_mxfp4_kernel<true>, dim3(E * wg_per_e), dim3(256), 0, s, x, perm, offsets,
                     k_top, w13, b13, E, 2 * I, H, (void*)h);
  return check_launch("moe_gate_up_mxfp4");
}

int launch_moe_down(const uint16_t* h, const int32_t* offsets, const uint8_t* w2, const float* b2,
                    int E, int H, int I, float* y, hipStream_t s) {
  const MxGeom gm = mx_geom(E, H, I);
  const int wg_per_e = ceil_div(gm.NT, 4 * kNTW);
  hipLaunchKernelGGL(moe_mxfp4_kernel<false>, dim3(E * wg_per_e), dim3(256), 0, s, h, nullptr,
                     offsets, 1, w2, b2, E, H, I, (void*)y);
  return check_launch("moe_down_mxfp4");
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
                                       const int32_t* offsets, int32_t k, const uint8_t* w13_packed,
                                       const float* b13, int32_t E, int32_t H, int32_t I,
                                       uint16_t* h, flyai_stream_t stream) {
  FLYAI_REQUIRE(E > 0 && H > 0 && I > 0 && H % 32 == 0 && (2 * I) % 16 == 0 && k >= 1,
                "gate_up: need H %% 32 == 0, 2I %% 16 == 0");
  FLYAI_REQUIRE(x && perm && offsets && w13_packed && b13 && h, "gate_up: null pointer");
  return launch_moe_gate_up(x, perm, offsets, k, w13_packed, b13, E, H, I, h, as_stream(stream));
}

extern "C" int flyai_moe_down_mxfp4(const uint16_t* h, const int32_t* offsets,
                                    const uint8_t* w2_packed, const float* b2, int32_t E, int32_t H,
                                    int32_t I, float* y_perm, flyai_stream_t stream) {
  FLYAI_REQUIRE(E > 0 && H > 0 && I > 0 && I % 32 == 0 && H % 16 == 0,
                "down: need I %% 32 == 0, H %% 16 == 0");
  FLYAI_REQUIRE(h && offsets && w2_packed && b2 && y_perm, "down: null pointer");
  return launch_moe_down(h, offsets, w2_packed, b2, E, H, I, y_perm, as_stream(stream));
}
