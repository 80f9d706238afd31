// Ragged GQA attention with learned sinks and an optional sliding window, for decode, spec-verify
// and prefill-chunk rows over per-sequence KV slabs.
//
// KV slab of sequence b at element offset kv_base[b] (caller-owned pools, kv_cap[b] % 64 == 0):
//   K  [Hkv][cap][64]   (row per key)
//   Vt [Hkv][64][cap]   (V transposed: row per head dim)
// Work item = (sequence, kv head, <= 4 query tokens, key split).  Its 32 query rows (4 tokens x 8
// heads of the GQA group) are processed by one wave with 16x16x32 bf16 MFMAs:
//   S^T[16 keys][16 qrows] = K_tile . Q^T       (K as A operand, Q^T as B, head dim reduced)
//   O^T[16 dims][16 qrows] += Vt_tile . P^T     (Vt as A operand, P^T as B, keys reduced)
// The key order inside a 64-key block is permuted so that the S^T accumulator registers of a lane
// are exactly the P^T operand the second MFMA needs (no shuffles): S^T tile kt, row m holds key
// 16*(m/4) + 4*kt + m%4, so lane (qrow n, group g) holds keys 16g .. 16g+15 across the 4 tiles,
// which is the contiguous 32-byte run of the Vt row it loads.
// Each item writes (m, l, O[64]) per query row; a merge kernel folds the splits and the sink.
#include <math.h>
#include <vector>

#include "common.h"

namespace flyai {

constexpr int kAttnRows = 32;     // query rows per item (4 tokens x 8 heads)
constexpr int kPartFloats = 66;   // m, l, O[64]

__device__ __forceinline__ uint4 mask_keys(uint4 v, int key0, int lo, int hi) {
  // zero the bf16 elements whose key (key0 + element index) lies outside [lo, hi)
  uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int key = key0 + i;
    if (key < lo || key >= hi) w[i >> 1] &= (i & 1) ? 0x0000ffffu : 0xffff0000u;
  }
  return make_uint4(w[0], w[1], w[2], w[3]);
}

__global__ __launch_bounds__(64) void attn_partial_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k_pool,
    const uint16_t* __restrict__ v_pool, const int64_t* __restrict__ kv_base,
    const int32_t* __restrict__ kv_cap, int window, int Hq,
    const flyai_attn_item* __restrict__ items, float* __restrict__ partials) {
  const flyai_attn_item it = items[blockIdx.x];
  const int lane = threadIdx.x;
  const int n = lane & 15, g = lane >> 4;
  const int cap = kv_cap[it.seq];
  const int64_t base = kv_base[it.seq] + (int64_t)it.kv_head * cap * 64;
  const uint16_t* K = k_pool + base;
  const uint16_t* Vt = v_pool + base;
  const float scale = 0.125f;  // 64 ** -0.5

  // Q^T operand: qrow rq = 16*qt + n -> token rq/8, head kv_head*8 + rq%8; dims 16g .. 16g+15
  bf16x8_t qf[2][2];
  int qpos[2];
  bool qval[2];
#pragma unroll
  for (int qt = 0; qt < 2; ++qt) {
    const int rq = 16 * qt + n;
    const int ti = rq >> 3;
    qval[qt] = ti < it.ntok;
    qpos[qt] = it.pos0 + ti;
    uint4 a = make_uint4(0, 0, 0, 0), b2 = make_uint4(0, 0, 0, 0);
    if (qval[qt]) {
      const uint4* qp = reinterpret_cast<const uint4*>(
          q + ((size_t)(it.tok + ti) * Hq + it.kv_head * 8 + (rq & 7)) * 64 + 16 * g);
      a = qp[0];
      b2 = qp[1];
    }
    qf[qt][0] = as_bf16x8(a);
    qf[qt][1] = as_bf16x8(b2);
  }
  float m_run[2] = {-1e30f, -1e30f}, l_run[2] = {0.f, 0.f};
  f32x4_t O[2][4];
#pragma unroll
  for (int qt = 0; qt < 2; ++qt)
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) O[qt][dt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  const bool two_tiles = it.ntok > 2;

  for (int kb = it.key_lo & ~63; kb < it.key_hi; kb += 64) {
    // K tiles (A operand): lane row n of tile kt is key kb + 16*(n/4) + 4*kt + n%4
    uint4 ka[4][2];
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) {
      const int key = kb + 16 * (n >> 2) + 4 * kt + (n & 3);
      if (key < it.key_hi) {
        const uint4* kp = reinterpret_cast<const uint4*>(K + (size_t)key * 64 + 16 * g);
        ka[kt][0] = kp[0];
        ka[kt][1] = kp[1];
      } else {
        ka[kt][0] = make_uint4(0, 0, 0, 0);
        ka[kt][1] = make_uint4(0, 0, 0, 0);
      }
    }
    // Vt tiles (A operand of the PV product): lane row n = dim 16*dt + n, keys kb + 16g .. +15
    uint4 va[4][2];
    const int vkey0 = kb + 16 * g;
    const bool vfull = vkey0 >= it.key_lo && vkey0 + 16 <= it.key_hi;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {
      if (vkey0 < it.key_hi) {
        const uint4* vp = reinterpret_cast<const uint4*>(Vt + (size_t)(16 * dt + n) * cap + vkey0);
        va[dt][0] = vp[0];
        va[dt][1] = vp[1];
        if (!vfull) {
          va[dt][0] = mask_keys(va[dt][0], vkey0, it.key_lo, it.key_hi);
          va[dt][1] = mask_keys(va[dt][1], vkey0 + 8, it.key_lo, it.key_hi);
        }
      } else {
        va[dt][0] = make_uint4(0, 0, 0, 0);
        va[dt][1] = make_uint4(0, 0, 0, 0);
      }
    }
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) {
      if (qt == 1 && !two_tiles) break;
      f32x4_t s[4];
#pragma unroll
      for (int kt = 0; kt < 4; ++kt) {
        s[kt] = mfma16x16x32(as_bf16x8(ka[kt][0]), qf[qt][0], f32x4_t{0.f, 0.f, 0.f, 0.f});
        s[kt] = mfma16x16x32(as_bf16x8(ka[kt][1]), qf[qt][1], s[kt]);
      }
      // lane holds S^T[key kb + 16g + 4kt + v][qrow n]
      const int p = qpos[qt];
      const int lo = window > 0 ? max(0, p - window + 1) : 0;
      float bmax = -INFINITY;
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int key = kb + 16 * g + 4 * kt + v;
          const bool ok = qval[qt] && key >= lo && key <= p && key >= it.key_lo && key < it.key_hi;
          s[kt][v] = ok ? s[kt][v] * scale : -INFINITY;
          bmax = fmaxf(bmax, s[kt][v]);
        }
      bmax = fmaxf(bmax, __shfl_xor(bmax, 16, 64));
      bmax = fmaxf(bmax, __shfl_xor(bmax, 32, 64));
      const float m_new = fmaxf(m_run[qt], bmax);
      const float alpha = __expf(m_run[qt] - m_new);
      m_run[qt] = m_new;
      float lsum = 0.f;
      bf16x8_t pt[2];
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const float pv = __expf(s[kt][v] - m_new);
          const uint16_t pb = f2bf(pv);
          lsum += bf2f(pb);
          pt[kt >> 1][(kt & 1) * 4 + v] = __builtin_bit_cast(__bf16, pb);
        }
      l_run[qt] = l_run[qt] * alpha + lsum;
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) {
        O[qt][dt] *= alpha;
        O[qt][dt] = mfma16x16x32(as_bf16x8(va[dt][0]), pt[0], O[qt][dt]);
        O[qt][dt] = mfma16x16x32(as_bf16x8(va[dt][1]), pt[1], O[qt][dt]);
      }
    }
  }
  // partial record per query row: [m, l, O[64]]; O^T layout: lane holds dims 16dt + 4g + v of qrow n
#pragma unroll
  for (int qt = 0; qt < 2; ++qt) {
    float l = l_run[qt];
    l += __shfl_xor(l, 16, 64);
    l += __shfl_xor(l, 32, 64);
    const int rq = 16 * qt + n;
    if (!qval[qt]) continue;
    float* rec = partials + ((size_t)blockIdx.x * kAttnRows + rq) * kPartFloats;
    if (g == 0) {
      rec[0] = m_run[qt];
      rec[1] = l;
    }
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int v = 0; v < 4; ++v) rec[2 + 16 * dt + 4 * g + v] = O[qt][dt][v];
  }
}

// Merge: per query row, M = max(sink, max_s m_s), L = e^(sink-M) + sum_s l_s e^(m_s-M),
// out = bf16(sum_s O_s e^(m_s-M) / L).  Thread (row = tid/8, part = tid%8) writes 8 dims.
__global__ __launch_bounds__(256) void attn_merge_kernel(const float* __restrict__ partials,
                                                         const flyai_attn_group* __restrict__ groups,
                                                         const float* __restrict__ sinks, int Hq,
                                                         uint16_t* __restrict__ out) {
  const flyai_attn_group gr = groups[blockIdx.x];
  const int rq = threadIdx.x >> 3, part = threadIdx.x & 7;
  const int ti = rq >> 3;
  if (ti >= gr.ntok) return;
  const int h = gr.kv_head * 8 + (rq & 7);
  const float sink = sinks[h];
  float M = sink;
  for (int s = 0; s < gr.n_splits; ++s)
    M = fmaxf(M, partials[((size_t)(gr.first_item + s) * kAttnRows + rq) * kPartFloats]);
  float L = __expf(sink - M);
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  for (int s = 0; s < gr.n_splits; ++s) {
    const float* rec = partials + ((size_t)(gr.first_item + s) * kAttnRows + rq) * kPartFloats;
    const float wgt = __expf(rec[0] - M);
    L += rec[1] * wgt;
#pragma unroll
    for (int d = 0; d < 8; ++d) acc[d] += rec[2 + part * 8 + d] * wgt;
  }
  const float inv = 1.0f / L;
  uint16_t* o = out + ((size_t)(gr.tok + ti) * Hq + h) * 64 + part * 8;
  uint32_t wv[4];
#pragma unroll
  for (int d = 0; d < 4; ++d)
    wv[d] = (uint32_t)f2bf(acc[2 * d] * inv) | ((uint32_t)f2bf(acc[2 * d + 1] * inv) << 16);
  *reinterpret_cast<uint4*>(o) = make_uint4(wv[0], wv[1], wv[2], wv[3]);
}

int launch_attn(const uint16_t* q, const uint16_t* k_pool, const uint16_t* v_pool,
                const int64_t* kv_base, const int32_t* kv_cap, const float* sinks, int window,
                int Hq, const flyai_attn_item* items, int n_items, const flyai_attn_group* groups,
                int n_groups, float* partials, uint16_t* out, hipStream_t s) {
  if (n_items == 0) return FLYAI_OK;
  hipLaunchKernelGGL(attn_partial_kernel, dim3(n_items), dim3(64), 0, s, q, k_pool, v_pool,
                     kv_base, kv_cap, window, Hq, items, partials);
  int rc = check_launch("attn_partial");
  if (rc) return rc;
  hipLaunchKernelGGL(attn_merge_kernel, dim3(n_groups), dim3(256), 0, s, partials, groups, sinks,
                     Hq, out);
  return check_launch("attn_merge");
}

int attn_plan(const int32_t* q_lens, const int32_t* starts, int S, int Hkv, int window,
              int split_keys, flyai_attn_item* items, int max_items, flyai_attn_group* groups,
              int max_groups, int* n_items, int* n_groups) {
  int ni = 0, ng = 0, tok = 0;
  for (int b = 0; b < S; ++b) {
    const int ql = q_lens[b], st = starts[b];
    for (int i0 = 0; i0 < ql; i0 += 4) {
      const int nt = ql - i0 < 4 ? ql - i0 : 4;
      const int p_first = st + i0, p_last = st + i0 + nt - 1;
      const int key_hi = p_last + 1;
      const int key_lo = window > 0 ? (p_first - window + 1 > 0 ? p_first - window + 1 : 0) : 0;
      const int kb0 = key_lo & ~63;
      const int nsplit = (key_hi - kb0 + split_keys - 1) / split_keys;
      for (int g = 0; g < Hkv; ++g) {
        if (ng >= max_groups || ni + nsplit > max_items)
          return set_error(FLYAI_ERANGE, "attention plan exceeds capacity (%d items, %d groups)",
                           max_items, max_groups);
        flyai_attn_group& gr = groups[ng];
        gr.first_item = ni;
        gr.n_splits = nsplit;
        gr.tok = tok + i0;
        gr.ntok = nt;
        gr.kv_head = g;
        gr.pad[0] = gr.pad[1] = gr.pad[2] = 0;
        for (int sp = 0; sp < nsplit; ++sp) {
          flyai_attn_item& it = items[ni++];
          it.seq = b;
          it.kv_head = g;
          it.tok = tok + i0;
          it.ntok = nt;
          it.pos0 = p_first;
          const int lo = kb0 + sp * split_keys;
          it.key_lo = lo > key_lo ? lo : key_lo;
          const int hi = kb0 + (sp + 1) * split_keys;
          it.key_hi = hi < key_hi ? hi : key_hi;
          it.group = ng;
        }
        ++ng;
      }
    }
    tok += ql;
  }
  *n_items = ni;
  *n_groups = ng;
  return FLYAI_OK;
}

}  // namespace flyai

using namespace flyai;

extern "C" int flyai_attn_plan(const int32_t* q_lens_host, const int32_t* starts_host,
                               int32_t n_seqs, int32_t Hkv, int32_t window, int32_t split_keys,
                               flyai_attn_item* items_host, int32_t max_items,
                               flyai_attn_group* groups_host, int32_t max_groups, int32_t* n_items,
                               int32_t* n_groups) {
  FLYAI_REQUIRE(n_seqs >= 0 && Hkv > 0 && window >= 0 && split_keys >= 64 && split_keys % 64 == 0,
                "attn_plan: split_keys must be a positive multiple of 64");
  FLYAI_REQUIRE(q_lens_host && starts_host && items_host && groups_host && n_items && n_groups,
                "attn_plan: null pointer");
  for (int b = 0; b < n_seqs; ++b)
    FLYAI_REQUIRE(q_lens_host[b] >= 1 && starts_host[b] >= 0, "attn_plan: bad q_len/start at %d", b);
  return attn_plan(q_lens_host, starts_host, n_seqs, Hkv, window, split_keys, items_host, max_items,
                   groups_host, max_groups, n_items, n_groups);
}

extern "C" size_t flyai_attn_partials_bytes(int32_t n_items) {
  return (size_t)(n_items > 0 ? n_items : 0) * kAttnRows * kPartFloats * sizeof(float);
}

extern "C" int flyai_attn_ragged(const uint16_t* q, const uint16_t* k_pool, const uint16_t* v_pool,
                                 const int64_t* kv_base, const int32_t* kv_cap, const float* sinks,
                                 int32_t window, int32_t Hq, int32_t Hkv, int32_t D,
                                 const flyai_attn_item* items_dev, int32_t n_items,
                                 const flyai_attn_group* groups_dev, int32_t n_groups,
                                 float* partials, uint16_t* out, flyai_stream_t stream) {
  FLYAI_REQUIRE(D == 64 && Hkv > 0 && Hq == 8 * Hkv, "attn: needs head_dim 64 and 8 query heads per kv head");
  FLYAI_REQUIRE(n_items >= 0 && n_groups >= 0 && window >= 0, "attn: bad counts");
  FLYAI_REQUIRE(q && k_pool && v_pool && kv_base && kv_cap && sinks && out &&
                    (n_items == 0 || (items_dev && groups_dev && partials)),
                "attn: null pointer");
  return launch_attn(q, k_pool, v_pool, kv_base, kv_cap, sinks, window, Hq, items_dev, n_items,
                     groups_dev, n_groups, partials, out, as_stream(stream));
}
