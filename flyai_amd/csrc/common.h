// Shared device/host helpers for the gfx950 stage kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

#include "flyai_stage.h"

namespace flyai {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

// ---- error reporting (thread-local last error, C-ABI returns negative codes) ------------------
int set_error(int code, const char* fmt, ...);
int check_launch(const char* what);

#define FLYAI_REQUIRE(cond, ...)                                   \
  do {                                                             \
    if (!(cond)) return ::flyai::set_error(FLYAI_EINVAL, __VA_ARGS__); \
  } while (0)

// ---- bf16 <-> fp32 -----------------------------------------------------------------------------
__device__ __forceinline__ float bf2f(uint16_t v) { return __uint_as_float(((uint32_t)v) << 16); }

// round-to-nearest-even fp32 -> bf16 bits, NaN made quiet (high 16 bits | 0x40): gfx950's
// v_cvt_pk_bf16_f32 (the __bf16 cast), one instruction for two values.  Checked against the integer
// formulation ((u + 0x7fff + ((u >> 16) & 1)) >> 16, NaN -> (u >> 16) | 0x40) on 1.1 million inputs
// (random words, every special class, 65,536 denormals): no bit differs.
__device__ __forceinline__ uint16_t f2bf(float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }

__device__ __forceinline__ float bf16_round(float f) { return bf2f(f2bf(f)); }

// E8M0 scale byte -> the fp32 whose exponent field is that byte (the form gfx950's scaled
// conversions read: only the exponent bits of the scale operand are used).
__device__ __forceinline__ float e8m0_operand(uint32_t byte) { return __uint_as_float(byte << 23); }

// Eight fp4 (E2M1) values held in one dword -> eight bf16 values scaled by 2^(scale-127).
// Byte b of `packed` holds elements 2b (low nibble) and 2b+1 (high nibble).
__device__ __forceinline__ bf16x8_t fp4x8_to_bf16x8(uint32_t packed, float scale) {
  bf16x2_t p0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(packed, scale, 0);
  bf16x2_t p1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(packed, scale, 1);
  bf16x2_t p2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(packed, scale, 2);
  bf16x2_t p3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(packed, scale, 3);
  bf16x8_t r;
  r[0] = p0[0]; r[1] = p0[1]; r[2] = p1[0]; r[3] = p1[1];
  r[4] = p2[0]; r[5] = p2[1]; r[6] = p3[0]; r[7] = p3[1];
  return r;
}

__device__ __forceinline__ bf16x8_t as_bf16x8(uint4 v) { return __builtin_bit_cast(bf16x8_t, v); }

__device__ __forceinline__ f32x4_t mfma16x16x32(bf16x8_t a, bf16x8_t b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// s_waitcnt immediates (vmcnt in bits 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8)
constexpr int waitcnt_vm(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }
constexpr int kWaitLgkm0 = 15 | (3 << 14) | (7 << 4);

// Workgroup barrier that waits only for the wave's own LDS operations.  __syncthreads() is also a
// release fence, which on gfx950 waits for every outstanding global load (s_waitcnt vmcnt(0)): it
// would drain a kernel's prefetch ring at every barrier.  Global loads stay in flight here.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

__device__ __forceinline__ float warp_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

constexpr int kRowThreads = 1024;  // one workgroup per token row: ~3 elements per thread at H = 2880

__device__ __forceinline__ float block_sum_1024(float v, float* red) {
  v = warp_sum(v);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  float s = 0.f;
#pragma unroll
  for (int w = 0; w < kRowThreads / 64; ++w) s += red[w];
  return s;
}

// RMSNorm of token row t by one kRowThreads workgroup: y = bf16(w * (x * rsqrt(mean(x^2) + eps)))
__device__ __forceinline__ void rmsnorm_row(const uint16_t* __restrict__ x, const float* __restrict__ w, int H,
                                            float eps, uint16_t* __restrict__ y, int t) {
  __shared__ float red[kRowThreads / 64];
  const int tid = threadIdx.x;
  const uint16_t* xr = x + (size_t)t * H;
  float ss = 0.f;
  for (int i = tid; i < H; i += kRowThreads) {
    const float v = bf2f(xr[i]);
    ss = fmaf(v, v, ss);
  }
  const float total = block_sum_1024(ss, red);
  const float r = rsqrtf(total / (float)H + eps);
  uint16_t* yr = y + (size_t)t * H;
  for (int i = tid; i < H; i += kRowThreads) {
    const float hs = bf2f(xr[i]) * r;
    yr[i] = f2bf(w[i] * hs);
  }
}

__device__ __forceinline__ float warp_max(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}

// ---- wave sums of many values at once ------------------------------------------------------------
// The xor butterfly v += shfl_xor(v, off), off = 32, 16, ..., 1, leaves every lane with the wave's
// sum.  For N = 2^n values per lane, wave_sum_scatter computes the same N sums with the same
// additions (each step adds a lane's partial to its partner's, and a + b == b + a bit for bit), but
// as a reduce-scatter: the step with offset off halves the values a lane carries -- the lane with
// that bit clear keeps the lower half, its partner the upper -- so the N sums take N - 1 exchanges
// per lane instead of 6 N.  Offsets 32 and 16 use gfx950's v_permlane32_swap / v_permlane16_swap
// (which pair value j with value j + half directly), the smaller ones ds_swizzle in its xor bit mode.
// Lane i ends with the sum of value i >> (6 - n) (2^(6-n) lanes hold each).  Every lane of the wave
// must be active.
template <int OFF>
__device__ __forceinline__ float swizzle_xor(float v) {
  static_assert(OFF >= 1 && OFF <= 16, "ds_swizzle's bit mode stays within 32 lanes");
  return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x1f | (OFF << 10)));
}

template <int OFF, int CNT, int N>
__device__ __forceinline__ void wave_sum_step(float (&a)[N], int lane) {
  if constexpr (CNT == 1) {  // one value left: the plain butterfly step
    if constexpr (OFF == 32 || OFF == 16) {
      const uint32_t u = __float_as_uint(a[0]);
      const auto r = OFF == 32 ? __builtin_amdgcn_permlane32_swap(u, u, false, false)
                               : __builtin_amdgcn_permlane16_swap(u, u, false, false);
      a[0] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    } else {
      a[0] = a[0] + swizzle_xor<OFF>(a[0]);
    }
  } else {
    constexpr int H = CNT / 2;
    if constexpr (OFF == 32 || OFF == 16) {
#pragma unroll
      for (int j = 0; j < H; ++j) {
        const auto r = OFF == 32
                           ? __builtin_amdgcn_permlane32_swap(__float_as_uint(a[j]), __float_as_uint(a[j + H]), false, false)
                           : __builtin_amdgcn_permlane16_swap(__float_as_uint(a[j]), __float_as_uint(a[j + H]), false, false);
        a[j] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
      }
    } else {
      const bool upper = (lane & OFF) != 0;
#pragma unroll
      for (int j = 0; j < H; ++j) {
        const float send = upper ? a[j] : a[j + H];
        const float keep = upper ? a[j + H] : a[j];
        a[j] = keep + swizzle_xor<OFF>(send);
      }
    }
  }
}

template <int N>
__device__ __forceinline__ float wave_sum_scatter(float (&a)[N]) {
  static_assert(N >= 1 && N <= 64 && (N & (N - 1)) == 0, "N must be a power of two <= 64");
  const int lane = threadIdx.x & 63;
  constexpr int c1 = N, c2 = c1 > 1 ? c1 / 2 : 1, c3 = c2 > 1 ? c2 / 2 : 1, c4 = c3 > 1 ? c3 / 2 : 1,
                c5 = c4 > 1 ? c4 / 2 : 1, c6 = c5 > 1 ? c5 / 2 : 1;
  wave_sum_step<32, c1>(a, lane);
  wave_sum_step<16, c2>(a, lane);
  wave_sum_step<8, c3>(a, lane);
  wave_sum_step<4, c4>(a, lane);
  wave_sum_step<2, c5>(a, lane);
  wave_sum_step<1, c6>(a, lane);
  return a[0];
}

template <int N>
constexpr int wave_sum_scatter_shift() {
  return N >= 64 ? 0 : N >= 32 ? 1 : N >= 16 ? 2 : N >= 8 ? 3 : N >= 4 ? 4 : N >= 2 ? 5 : 6;
}

// ---- KV slab layout (head_dim 64) ----------------------------------------------------------------
// A sequence's slab holds, per kv head, a region of cap x 64 bf16 (cap % 64 == 0) made of 64-key
// blocks of 4096 elements in the attention kernel's MFMA-fragment order, so that every 16-byte-per-
// lane load of a wave reads one contiguous KiB:
//   K: [kt 4][step 2][lane 64][8]  lane = 16 gd + n holds key tile_key(kt, n) of the block and dims
//      32 step + 8 gd .. +7, where tile_key(kt, m) = 32 (kt / 2) + 8 (m / 4) + 4 (kt % 2) + m % 4;
//   V: [h 2][dt 4][lane 64][8]  lane = 16 gk + n holds dim 16 dt + n and keys 32 h + 8 gk .. +7.
// kv_k_off / kv_v_off give the element offset of (key position p, dim d) within a head region.
__host__ __device__ inline int64_t kv_k_off(int p, int d) {
  const int kk = p & 63;
  const int kt = 2 * (kk >> 5) + ((kk & 7) >> 2);
  const int n = 4 * ((kk & 31) >> 3) + (kk & 3);
  return (int64_t)(p >> 6) * 4096 + kt * 1024 + (d >> 5) * 512 + (16 * ((d & 31) >> 3) + n) * 8 + (d & 7);
}
__host__ __device__ inline int64_t kv_v_off(int p, int d) {
  const int kk = p & 63;
  return (int64_t)(p >> 6) * 4096 + (kk >> 5) * 2048 + (d >> 4) * 512 + (16 * ((kk & 31) >> 3) + (d & 15)) * 8 +
         (kk & 7);
}

// query tokens per chunked-prefill attention item (4 waves x 4 tokens)
constexpr int kPrefillTokens = 16;

inline hipStream_t as_stream(flyai_stream_t s) { return reinterpret_cast<hipStream_t>(s); }

inline int ceil_div(int a, int b) { return (a + b - 1) / b; }

// Sorted top-K list helpers, branch-free (compare + select), so lanes of a wave never diverge.
// topk_insert_strict: (v, id) enters in front of the first entry it strictly exceeds and every
// entry behind it moves down one place (the last falls off) -- equal values keep the earlier (lower)
// id ahead, the same list a strict-greater insertion at the end followed by bubbling past strictly
// smaller values gives.  Every comparison is of the new entry (comparing a displaced entry again
// would swap two equal values), and no comparison waits on another.  topk_insert_ordered: the same under (value desc, id asc).
template <int K>
__device__ __forceinline__ void topk_insert_at(float (&sv)[K], int (&si)[K], float v, int id, const bool (&gt)[K]) {
  // gt[] is monotonic over the sorted list (false ... false, true ... true): the new entry goes to
  // the first true position and the entries from there on shift down one place; slot j reads only
  // slot j-1, so walking down from the end overwrites nothing still needed
#pragma unroll
  for (int j = K - 1; j >= 0; --j) {
    const bool prev = j > 0 && gt[j - 1];
    const float pv = j > 0 ? sv[j - 1] : v;
    const int pi = j > 0 ? si[j - 1] : id;
    sv[j] = gt[j] ? (prev ? pv : v) : sv[j];
    si[j] = gt[j] ? (prev ? pi : id) : si[j];
  }
}

template <int K>
__device__ __forceinline__ void topk_insert_strict(float (&sv)[K], int (&si)[K], float v, int id) {
  bool gt[K];
#pragma unroll
  for (int j = 0; j < K; ++j) gt[j] = v > sv[j];
  topk_insert_at<K>(sv, si, v, id, gt);
}

template <int K>
__device__ __forceinline__ void topk_insert_ordered(float (&sv)[K], int (&si)[K], float v, int id) {
  bool gt[K];
#pragma unroll
  for (int j = 0; j < K; ++j) gt[j] = v > sv[j] || (v == sv[j] && id < si[j]);
  topk_insert_at<K>(sv, si, v, id, gt);
}

// ids ascending, carrying their weights (odd-even transposition sort, K passes, branch-free)
template <int K>
__device__ __forceinline__ void sort_ids_with_weights(int (&si)[K], float (&ex)[K]) {
#pragma unroll
  for (int pass = 0; pass < K; ++pass)
#pragma unroll
    for (int j = pass & 1; j + 1 < K; j += 2) {
      const bool sw = si[j] > si[j + 1];
      const int a = si[j], b = si[j + 1];
      const float x = ex[j], y = ex[j + 1];
      si[j] = sw ? b : a;
      si[j + 1] = sw ? a : b;
      ex[j] = sw ? y : x;
      ex[j + 1] = sw ? x : y;
    }
}

// Top-k + softmax of one token by one lane.  The lane streams its token's logits in ascending expert
// id and keeps a sorted list of K (value, id); a value enters only if strictly greater than the
// current K-th and bubbles up past strictly smaller values, so equal values keep ascending ids --
// the (value desc, id asc) order.  Softmax over the K selected values in fp32, then ids sorted
// ascending carrying their weights.  Logit rows are 16-byte aligned (E % 4 == 0).
template <int K>
__device__ __forceinline__ void topk_softmax_lane(const float* __restrict__ lrow, int E,
                                                  int32_t* ids_out, float* w_out) {
  float sv[K];
  int si[K];
#pragma unroll
  for (int j = 0; j < K; ++j) { sv[j] = -INFINITY; si[j] = 0x7fffffff; }
  for (int e0 = 0; e0 < E; e0 += 16) {
    float4 v4[4];
#pragma unroll
    for (int c = 0; c < 4; ++c)
      v4[c] = (e0 + 4 * c < E) ? reinterpret_cast<const float4*>(lrow + e0)[c]
                               : make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const float4& q = v4[i >> 2];
      const float v = (i & 3) == 0 ? q.x : (i & 3) == 1 ? q.y : (i & 3) == 2 ? q.z : q.w;
      const int id = e0 + i;
      topk_insert_strict<K>(sv, si, id < E ? v : -INFINITY, id);
    }
  }
  float ex[K], sum = 0.f;
#pragma unroll
  for (int j = 0; j < K; ++j) { ex[j] = expf(sv[j] - sv[0]); sum += ex[j]; }
  sort_ids_with_weights<K>(si, ex);
#pragma unroll
  for (int j = 0; j < K; ++j) {
    ids_out[j] = (unsigned)si[j] < (unsigned)E ? si[j] : 0;  // a NaN row selects nothing: expert 0
    w_out[j] = ex[j] / sum;
  }
}

// The same top-k + softmax by a whole wave (E <= 256): each lane holds E/64 logits; K rounds of a
// wave-wide argmax over (value desc, id asc) give the same selection in the same order as
// topk_softmax_lane, and every lane then does the identical softmax / id sort, so ids and weights
// are bit-identical to it.  Lanes 0..K-1 write the outputs.
template <int K>
__device__ __forceinline__ void topk_softmax_wave_vals(const float (&v)[4], int E, int lane,
                                                       int32_t* ids_out, float* w_out) {
  bool taken[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) taken[j] = 4 * lane + j >= E;
  float sv[K];
  int si[K];
#pragma unroll
  for (int r = 0; r < K; ++r) {
    float bv = -INFINITY;
    int bi = 0x7fffffff;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int e = 4 * lane + j;
      if (!taken[j] && (v[j] > bv || (v[j] == bv && e < bi))) { bv = v[j]; bi = e; }
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
      const float ov = __shfl_xor(bv, o, 64);
      const int oi = __shfl_xor(bi, o, 64);
      if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
    }
    sv[r] = bv;
    si[r] = bi;
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (4 * lane + j == bi) taken[j] = true;
  }
  float ex[K], sum = 0.f;
#pragma unroll
  for (int j = 0; j < K; ++j) { ex[j] = expf(sv[j] - sv[0]); sum += ex[j]; }
  sort_ids_with_weights<K>(si, ex);
#pragma unroll
  for (int j = 0; j < K; ++j)
    if (lane == j) {
      ids_out[j] = (unsigned)si[j] < (unsigned)E ? si[j] : 0;  // a NaN row selects nothing: expert 0
      w_out[j] = ex[j] / sum;
    }
}

// lane l's logits of a row: experts 4l .. 4l+3 (-inf past E)
__device__ __forceinline__ void load_logits_lane(const float* __restrict__ lrow, int E, int lane, float (&v)[4]) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int e = 4 * lane + j;
    v[j] = e < E ? lrow[e] : -INFINITY;
  }
}

template <int K>
__device__ __forceinline__ void topk_softmax_wave(const float* __restrict__ lrow, int E, int lane,
                                                  int32_t* ids_out, float* w_out) {
  float v[4];
  load_logits_lane(lrow, E, lane, v);
  topk_softmax_wave_vals<K>(v, E, lane, ids_out, w_out);
}

// The same top-k + softmax with LANES lanes per token (lanes LANES*t .. LANES*t + LANES-1, `sub` =
// lane % LANES): each lane keeps the sorted top K of its 1/LANES of the logits (ascending ids,
// strict > insertion), then log2(LANES) xor-shuffle rounds merge the lists under (value desc, id
// asc), so all lanes of the group hold the same sorted selection as topk_softmax_lane and compute
// the identical softmax; sub 0 writes.  lrow must be 16-byte aligned and the share Q = E/LANES a
// multiple of 4 (E % (4*LANES) == 0).
template <int K, int LANES>
__device__ __forceinline__ void topk_softmax_group(const float* __restrict__ lrow, int E, int sub,
                                                   int32_t* ids_out, float* w_out) {
  float sv[K];
  int si[K];
#pragma unroll
  for (int j = 0; j < K; ++j) { sv[j] = -INFINITY; si[j] = 0x7fffffff; }
  const int Q = E / LANES;
  for (int e0 = sub * Q; e0 < (sub + 1) * Q; e0 += 4) {
    const float4 q = *reinterpret_cast<const float4*>(lrow + e0);
    const float vv[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) topk_insert_strict<K>(sv, si, vv[i], e0 + i);
  }
#pragma unroll
  for (int o = 1; o < LANES; o <<= 1) {
    float pv[K];
    int pi[K];
#pragma unroll
    for (int j = 0; j < K; ++j) { pv[j] = __shfl_xor(sv[j], o, 64); pi[j] = __shfl_xor(si[j], o, 64); }
#pragma unroll
    for (int m = 0; m < K; ++m) topk_insert_ordered<K>(sv, si, pv[m], pi[m]);
  }
  float ex[K], sum = 0.f;
#pragma unroll
  for (int j = 0; j < K; ++j) { ex[j] = expf(sv[j] - sv[0]); sum += ex[j]; }
  sort_ids_with_weights<K>(si, ex);
  if (sub == 0) {
#pragma unroll
    for (int j = 0; j < K; ++j) {
      ids_out[j] = (unsigned)si[j] < (unsigned)E ? si[j] : 0;  // a NaN row selects nothing: expert 0
      w_out[j] = ex[j] / sum;
    }
  }
}

}  // namespace flyai
