// Layer glue: RMSNorm, bf16 projections with bias (+ residual), RoPE + KV append.
#include "common.h"

namespace flyai {

// ---- RMSNorm: y = bf16(w * (x * rsqrt(mean(x^2) + eps))), fp32 weight --------------------------
__global__ __launch_bounds__(256) void rmsnorm_kernel(const uint16_t* __restrict__ x,
                                                      const float* __restrict__ w, int H, float eps,
                                                      uint16_t* __restrict__ y) {
  __shared__ float red[4];
  const int t = blockIdx.x, tid = threadIdx.x;
  const uint16_t* xr = x + (size_t)t * H;
  float ss = 0.f;
  for (int i = tid; i < H; i += 256) {
    const float v = bf2f(xr[i]);
    ss = fmaf(v, v, ss);
  }
  ss = warp_sum(ss);
  if ((tid & 63) == 0) red[tid >> 6] = ss;
  __syncthreads();
  const float total = red[0] + red[1] + red[2] + red[3];
  const float r = rsqrtf(total / (float)H + eps);
  uint16_t* yr = y + (size_t)t * H;
  for (int i = tid; i < H; i += 256) {
    const float hs = bf2f(xr[i]) * r;
    yr[i] = f2bf(w[i] * hs);
  }
}

int launch_rmsnorm(const uint16_t* x, const float* w, int T, int H, float eps, uint16_t* y,
                   hipStream_t s) {
  if (T == 0) return FLYAI_OK;
  hipLaunchKernelGGL(rmsnorm_kernel, dim3(T), dim3(256), 0, s, x, w, H, eps, y);
  return check_launch("rmsnorm");
}

// ---- bf16 linear: y[M,N] = bf16(x[M,K] W[N,K]^T + b), split-K over the waves of a workgroup --------
// Workgroup = KS waves on one 16-feature tile; wave w takes K groups of 128 (w, w+KS, ...); lane
// (r, g) supplies K values 128*kq + 32*g + 8*j .. +7 at MFMA step j for both operands.  Partial
// accumulators are reduced through LDS and wave 0 applies bias / residual.
constexpr int kLinMT = 4;  // 64 activation rows per pass

template <int KS>
__global__ __launch_bounds__(KS * 64) void linear_bf16_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ W, const uint16_t* __restrict__ b,
    int M, int N, int K, uint16_t* __restrict__ y, uint16_t* __restrict__ residual) {
  __shared__ f32x4_t red[KS][kLinMT][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 15, g = lane >> 4;
  const int nt = blockIdx.x;
  const int feat = nt * 16 + r;
  const int KQ = (K + 127) / 128;
  const uint16_t* wrow = W + (size_t)feat * K + 32 * g;
  for (int m0 = 0; m0 < M; m0 += 16 * kLinMT) {
    const int mt_count = min(kLinMT, (M - m0 + 15) / 16);
    f32x4_t acc[kLinMT];
#pragma unroll
    for (int m = 0; m < kLinMT; ++m) acc[m] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    for (int kq = wave; kq < KQ; kq += KS) {
      const int k0 = 128 * kq + 32 * g;
      const bool kv = k0 < K;
      uint4 wv[4];
#pragma unroll
      for (int j = 0; j < 4; ++j)
        wv[j] = kv ? reinterpret_cast<const uint4*>(wrow + 128 * kq)[j] : make_uint4(0, 0, 0, 0);
#pragma unroll
      for (int m = 0; m < kLinMT; ++m) {
        if (m < mt_count) {
          const int row = m0 + 16 * m + r;
          uint4 av[4];
          if (kv && row < M) {
            const uint4* ap = reinterpret_cast<const uint4*>(x + (size_t)row * K + k0);
#pragma unroll
            for (int j = 0; j < 4; ++j) av[j] = ap[j];
          } else {
#pragma unroll
            for (int j = 0; j < 4; ++j) av[j] = make_uint4(0, 0, 0, 0);
          }
#pragma unroll
          for (int j = 0; j < 4; ++j) acc[m] = mfma16x16x32(as_bf16x8(av[j]), as_bf16x8(wv[j]), acc[m]);
        }
      }
    }
#pragma unroll
    for (int m = 0; m < kLinMT; ++m) red[wave][m][lane] = acc[m];
    __syncthreads();
    if (wave == 0) {
      const float bias = b ? bf2f(b[feat]) : 0.f;
      for (int m = 0; m < mt_count; ++m) {
        f32x4_t s = red[0][m][lane];
#pragma unroll
        for (int w = 1; w < KS; ++w) s += red[w][m][lane];
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int row = m0 + 16 * m + 4 * g + v;
          if (row < M) {
            const float o = bf16_round(s[v] + bias);
            if (residual) {
              uint16_t* rp = residual + (size_t)row * N + feat;
              *rp = f2bf(bf2f(*rp) + o);
            } else {
              y[(size_t)row * N + feat] = f2bf(o);
            }
          }
        }
      }
    }
    __syncthreads();
  }
}

int launch_linear(const uint16_t* x, const uint16_t* W, const uint16_t* b, int M, int N, int K,
                  uint16_t* y, uint16_t* residual, hipStream_t s) {
  if (M == 0) return FLYAI_OK;
  hipLaunchKernelGGL(linear_bf16_kernel<8>, dim3(N / 16), dim3(8 * 64), 0, s, x, W, b, M, N, K, y,
                     residual);
  return check_launch("linear_bf16");
}

// ---- RoPE (GPT-OSS half split, per-op bf16 rounding) + K/V append --------------------------------
__global__ __launch_bounds__(256) void rope_kv_append_kernel(
    const uint16_t* __restrict__ qkv, const int32_t* __restrict__ positions,
    const int32_t* __restrict__ seq_id, const uint16_t* __restrict__ cos_tab,
    const uint16_t* __restrict__ sin_tab, int rope_positions, int Hq, int Hkv, int D,
    const int64_t* __restrict__ kv_base,
    const int32_t* __restrict__ kv_cap, uint16_t* __restrict__ q_out, uint16_t* __restrict__ k_pool,
    uint16_t* __restrict__ v_pool) {
  const int t = blockIdx.x;
  const int pos = positions[t];
  if (pos < 0 || pos >= rope_positions) return;  // outside the rotary table: no read, no write
  const int b = seq_id[t];
  const int cap = kv_cap[b];
  const bool in_cap = pos >= 0 && pos < cap;
  const int64_t base = kv_base[b];
  const int D2 = D / 2;
  const int width = (Hq + 2 * Hkv) * D;
  const uint16_t* row = qkv + (size_t)t * width;
  const uint16_t* cr = cos_tab + (size_t)pos * D2;
  const uint16_t* sr = sin_tab + (size_t)pos * D2;
  const int pairs = (Hq + Hkv) * D2;
  for (int i = threadIdx.x; i < pairs; i += blockDim.x) {
    const int h = i / D2, d = i % D2;
    const float x1 = bf2f(row[h * D + d]), x2 = bf2f(row[h * D + d + D2]);
    const float c = bf2f(cr[d]), s = bf2f(sr[d]);
    const float first = bf16_round(bf16_round(x1 * c) - bf16_round(x2 * s));
    const float second = bf16_round(bf16_round(x2 * c) + bf16_round(x1 * s));
    if (h < Hq) {
      q_out[((size_t)t * Hq + h) * D + d] = f2bf(first);
      q_out[((size_t)t * Hq + h) * D + d + D2] = f2bf(second);
    } else if (in_cap) {
      const int gk = h - Hq;
      uint16_t* kp = k_pool + base + ((size_t)gk * cap + pos) * D;
      kp[d] = f2bf(first);
      kp[d + D2] = f2bf(second);
    }
  }
  if (in_cap) {
    for (int i = threadIdx.x; i < Hkv * D; i += blockDim.x) {
      const int gv = i / D, d = i % D;
      v_pool[base + ((size_t)gv * D + d) * cap + pos] = row[(Hq + Hkv) * D + gv * D + d];
    }
  }
}

int launch_rope_kv(const uint16_t* qkv, const int32_t* positions, const int32_t* seq_id,
                   const uint16_t* cos_tab, const uint16_t* sin_tab, int rope_positions, int T,
                   int Hq, int Hkv, int D,
                   const int64_t* kv_base, const int32_t* kv_cap, uint16_t* q_out,
                   uint16_t* k_pool, uint16_t* v_pool, hipStream_t s) {
  if (T == 0) return FLYAI_OK;
  hipLaunchKernelGGL(rope_kv_append_kernel, dim3(T), dim3(256), 0, s, qkv, positions, seq_id,
                     cos_tab, sin_tab, rope_positions, Hq, Hkv, D, kv_base, kv_cap, q_out, k_pool,
                     v_pool);
  return check_launch("rope_kv_append");
}

}  // namespace flyai

using namespace flyai;

extern "C" int flyai_rmsnorm(const uint16_t* x, const float* w, int32_t T, int32_t H, float eps,
                             uint16_t* y, flyai_stream_t stream) {
  FLYAI_REQUIRE(T >= 0 && H > 0, "rmsnorm: bad shape");
  FLYAI_REQUIRE(x && w && y, "rmsnorm: null pointer");
  return launch_rmsnorm(x, w, T, H, eps, y, as_stream(stream));
}

extern "C" int flyai_linear_bf16(const uint16_t* x, const uint16_t* w, const uint16_t* b, int32_t M,
                                 int32_t N, int32_t K, uint16_t* y, uint16_t* residual,
                                 flyai_stream_t stream) {
  FLYAI_REQUIRE(M >= 0 && N > 0 && K > 0 && N % 16 == 0 && K % 32 == 0,
                "linear: need N %% 16 == 0 and K %% 32 == 0");
  FLYAI_REQUIRE(x && w && (y || residual), "linear: null pointer");
  return launch_linear(x, w, b, M, N, K, y, residual, as_stream(stream));
}

extern "C" int flyai_rope_kv_append(const uint16_t* qkv, const int32_t* positions,
                                    const int32_t* seq_id, const uint16_t* cos_tab,
                                    const uint16_t* sin_tab, int32_t rope_positions, int32_t T,
                                    int32_t Hq, int32_t Hkv, int32_t D, const int64_t* kv_base,
                                    const int32_t* kv_cap, uint16_t* q_out, uint16_t* k_pool,
                                    uint16_t* v_pool, flyai_stream_t stream) {
  FLYAI_REQUIRE(T >= 0 && Hq > 0 && Hkv > 0 && D > 0 && D % 2 == 0 && rope_positions > 0,
                "rope_kv: bad shape");
  FLYAI_REQUIRE(qkv && positions && seq_id && cos_tab && sin_tab && kv_base && kv_cap && q_out &&
                    k_pool && v_pool,
                "rope_kv: null pointer");
  return launch_rope_kv(qkv, positions, seq_id, cos_tab, sin_tab, rope_positions, T, Hq, Hkv, D,
                        kv_base, kv_cap, q_out, k_pool, v_pool, as_stream(stream));
}
