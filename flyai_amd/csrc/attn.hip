// Ragged GQA attention with learned sinks and an optional sliding window, for decode, spec-verify
// and prefill-chunk rows over per-sequence KV slabs.
//
// KV slab of sequence b at element offset kv_base[b] (caller-owned pools, kv_cap[b] % 64 == 0): per
// kv head a region of cap x 64 elements, tiled in 64-key blocks in the fragment order below
// (kv_k_off / kv_v_off in common.h), so every K or V load instruction of a wave reads one KiB.
// Work item = (sequence, kv head, <= 4 query tokens, key split).  Its query rows (tokens x the 8
// heads of the GQA group, in tiles of 16) are processed by one wave with 16x16x32 bf16 MFMAs:
//   S^T[16 keys][16 qrows] = K_tile . Q^T       (K as A operand, Q^T as B, head dim reduced)
//   O^T[16 dims][16 qrows] += Vt_tile . P^T     (Vt as A operand, P^T as B, keys reduced)
// Operand orders are permuted (any order consistent between the two operands of a product is
// valid), and the slab stores each block in exactly the order the lanes consume it:
//   head dims: lane group g supplies dims 8g..8g+7 (step 0) and 32+8g..32+8g+7 (step 1);
//   keys of a 64-key block: S^T tile kt, row m is key 32*(kt/2) + 8*(m/4) + 4*(kt%2) + m%4, so the
//   C-layout registers of lane (qrow n, group g) hold keys 8g..8g+7 (tiles 0,1) and 32+8g..+7
//   (tiles 2,3) -- exactly the P^T operand of the two PV steps and the two 16-byte Vt loads.
// K and V of the next block are loaded while the current block computes.  Each item writes (m, l, O[64])
// per query row; a merge kernel folds the splits and the sink.
#include <limits.h>
#include <math.h>
#include <type_traits>
#include <vector>

#include "common.h"

namespace flyai {

constexpr int kAttnRows = 32;     // query rows per item (4 tokens x 8 heads)
constexpr int kPartFloats = 66;   // m (base-2 units), l, O[64]
constexpr float kLog2e = 1.4426950408889634f;

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

__device__ __forceinline__ int tile_key(int kt, int m) {
  return 32 * (kt >> 1) + 8 * (m >> 2) + 4 * (kt & 1) + (m & 3);
}

// Every 64-key block starts at a multiple of 64 below key_hi <= cap (cap % 64 == 0), so all 64 keys
// are inside the slab: the loads below are unconditional (no branch between loads).  The slab is
// tiled (kv_k_off / kv_v_off in common.h): a 64-key block is 4096 contiguous elements, and each of
// these 16-byte-per-lane loads reads one contiguous KiB of it.
// KV is read once per step, so the loads are nontemporal (streamed, as the expert weights are).
typedef unsigned int attn_u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint4 ld_kv(const uint16_t* p) {
  const attn_u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const attn_u32x4*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ void load_k_tile(uint4 (&k)[4][2], const uint16_t* __restrict__ K, int kb,
                                            int lane) {
  const uint16_t* blk = K + (size_t)kb * 64 + lane * 8;
#pragma unroll
  for (int kt = 0; kt < 4; ++kt) {
    k[kt][0] = ld_kv(blk + kt * 1024);
    k[kt][1] = ld_kv(blk + kt * 1024 + 512);
  }
}

__device__ __forceinline__ void load_v_tile(uint4 (&v)[4][2], const uint16_t* __restrict__ Vt, int kb,
                                            int lane) {
  const uint16_t* blk = Vt + (size_t)kb * 64 + lane * 8;
#pragma unroll
  for (int h = 0; h < 2; ++h)
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) v[dt][h] = ld_kv(blk + h * 2048 + dt * 512);
}

// A tree-verify launch's view of its flyai_attn_tree: the node depths and the visibility mask of the
// launch's layer kind (bit j of row i: node i sees tree slot start + j).  Empty outside trees.
struct TreeView {
  int start = 0, n = 0, words = 0;
  const int32_t* depth = nullptr;
  const uint64_t* mask = nullptr;
};

// Per-wave state of QT query-row tiles of 16 (QT = 1: up to 2 tokens; QT = 2: up to 4 tokens): the
// Q^T operand, each row's position (and, in a tree, its depth and node), and the running
// softmax (max, sum, O^T accumulators).  Query row rq = 16*qt + n is token rq/8, head kv_head*8 + rq%8.
// The row sums are accumulated like O^T, by an MFMA with an all-ones A operand: every element of
// lane (n, g)'s L[qt] is row n's complete sum over the keys so far.
template <int QT>
struct QRows {
  bf16x8_t qf[QT][2];
  int qpos[QT], qdep[QT], qnode[QT];
  bool qval[QT];
  float m_run[QT];
  f32x4_t O[QT][4], L[QT];
};

// Load the rows of tokens tok .. tok+ntok-1 (positions pos0 + ti, or tree positions) and reset the
// running softmax.
template <int QT, bool TREE>
__device__ __forceinline__ void rows_init(QRows<QT>& R, const uint16_t* __restrict__ q, int tok, int ntok,
                                          int pos0, int kv_head, int Hq, const TreeView& tv) {
  const int lane = threadIdx.x & 63;
  const int n = lane & 15, g = lane >> 4;
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    const int rq = 16 * qt + n;
    const int ti = rq >> 3;
    R.qval[qt] = ti < ntok;
    if (TREE) {
      R.qnode[qt] = R.qval[qt] ? tok + ti : 0;  // tok + ti < n_nodes for every valid row
      R.qdep[qt] = R.qval[qt] ? tv.depth[tok + ti] : 0;
      R.qpos[qt] = tv.start + R.qdep[qt];
    } else {
      R.qnode[qt] = 0;
      R.qdep[qt] = 0;
      R.qpos[qt] = pos0 + ti;
    }
    uint4 a = make_uint4(0, 0, 0, 0), b2 = make_uint4(0, 0, 0, 0);
    if (R.qval[qt]) {
      const uint16_t* qp = q + ((size_t)(tok + ti) * Hq + kv_head * 8 + (rq & 7)) * 64 + 8 * g;
      a = *reinterpret_cast<const uint4*>(qp);
      b2 = *reinterpret_cast<const uint4*>(qp + 32);
    }
    R.qf[qt][0] = as_bf16x8(a);
    R.qf[qt][1] = as_bf16x8(b2);
    R.m_run[qt] = -1e30f;
    R.L[qt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) R.O[qt][dt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  }
}

// Max over the four lanes n, n+16, n+32, n+48 (one query row's lane groups), with gfx950's
// v_permlane32_swap / v_permlane16_swap (VALU lane swaps, no LDS round trip).  Swapping a register
// with a copy of itself leaves lane i's value and its partner's in the two results.  (A compare and
// select: fmaxf on the swapped values is three instructions, since the compiler quiets possible
// signalling NaNs in both operands first.)
__device__ __forceinline__ float max_lane_groups(float v) {
  const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  const float x0 = __uint_as_float(a[0]), x1 = __uint_as_float(a[1]);
  v = x0 > x1 ? x0 : x1;
  const auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  const float y0 = __uint_as_float(b[0]), y1 = __uint_as_float(b[1]);
  return y0 > y1 ? y0 : y1;
}

// One 64-key block kb (K fragments kc, V fragments vv of this lane) against the rows: scores
// S^T = K . Q^T, the mask (positions in [key_lo, key_hi) within each row's causal / window range, or
// the tree rule), the online softmax update and O^T += V^T . P^T, L += 1 . P^T.  interior: every key of
// the block is visible to every valid row (no mask).  Values of keys at or past key_hi are zeroed (they
// may be unwritten, even non-finite; P is 0 there).
// Scores are kept raw and scaled inside the exponent, P = 2^(s * scale - m) with scale = head_dim^-0.5
// log2(e) (one FMA and one v_exp_f32; the max commutes with the positive scale).  The running max m
// (base-2 units) moves only when a block's max exceeds it by more than kMaxSlack, so P <= 2^kMaxSlack
// between moves; a wave rescales O and L only when one of its rows moved (alpha = 1 exactly for the
// others, so skipping is exact and a row's result does not depend on its wave mates).
constexpr float kMaxSlack = 8.f;
constexpr float kMaxSentinel = -1e29f;  // a running max at or below this is the initial -1e30 (no key yet)

template <int QT, bool TREE>
__device__ __forceinline__ void rows_block(QRows<QT>& R, const uint4 (&kc)[4][2], uint4 (&vv)[4][2], int kb,
                                           bool interior, int key_lo, int key_hi, int window,
                                           const TreeView& tv) {
  const int g = (threadIdx.x & 63) >> 4;
  const float scale = 0.125f * kLog2e;
  const int tstart = TREE ? tv.start : 0;
  const bf16x8_t ones = as_bf16x8(make_uint4(0x3f803f80u, 0x3f803f80u, 0x3f803f80u, 0x3f803f80u));
  if (kb + 64 > key_hi) {
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) vv[dt][h] = mask_keys(vv[dt][h], kb + 32 * h + 8 * g, INT_MIN, key_hi);
  }
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    f32x4_t s[4];
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) {
      s[kt] = mfma16x16x32(as_bf16x8(kc[kt][0]), R.qf[qt][0], f32x4_t{0.f, 0.f, 0.f, 0.f});
      s[kt] = mfma16x16x32(as_bf16x8(kc[kt][1]), R.qf[qt][1], s[kt]);
    }
    // lane holds S^T[key kb + tile_key(kt, 4g + v)][qrow n]
    float bmax = -INFINITY;
    if (interior && R.qval[qt]) {
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
#pragma unroll
        for (int v = 0; v < 4; ++v) bmax = fmaxf(bmax, s[kt][v]);
    } else {
      const int p = R.qpos[qt];
      const int lo = max(key_lo, window > 0 ? p - window + 1 : 0);
      const int hi = min(p, key_hi - 1);
      // tree: bits [kb - start, kb - start + 64) of the row's mask (key kb + t is bit t)
      uint64_t tbits = 0;
      if (TREE) {
        const int j0 = kb - tstart;
        if (R.qval[qt] && j0 > -64 && j0 < tv.n) {
          const int wq = j0 >> 6, sh = j0 & 63;  // floor division (j0 may be negative)
          const uint64_t* mrow = tv.mask + (size_t)R.qnode[qt] * tv.words;
          const uint64_t w0 = wq >= 0 ? mrow[wq] : 0ull;
          const uint64_t w1 = wq + 1 < tv.words ? mrow[wq + 1] : 0ull;
          tbits = sh == 0 ? w0 : (w0 >> sh) | (w1 << (64 - sh));
        }
      }
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int key = kb + tile_key(kt, 4 * g + v);
          bool ok;
          if (TREE) {
            if (key < tstart)
              ok = key >= lo && key < key_hi;  // committed prefix (window on positions)
            else  // tree slot: the mask (its window already applied for sliding layers)
              ok = key >= key_lo && key < key_hi && ((tbits >> tile_key(kt, 4 * g + v)) & 1ull);
            ok = ok && R.qval[qt];
          } else {
            ok = R.qval[qt] && key >= lo && key <= hi;
          }
          s[kt][v] = ok ? s[kt][v] : -INFINITY;
          bmax = fmaxf(bmax, s[kt][v]);
        }
    }
    bmax = max_lane_groups(bmax);
    // (a fully masked row keeps m = -1e30: -1e30 + kMaxSlack rounds to -1e30 and -inf never exceeds it)
    const float m_blk = bmax * scale;
    const bool move = m_blk > R.m_run[qt] + kMaxSlack;
    if (__ballot(move)) {
      const float m_new = move ? m_blk : R.m_run[qt];
      // v_exp_f32 directly (results below 2^-126 may flush to zero: immaterial for a probability)
      const float alpha = __builtin_amdgcn_exp2f(R.m_run[qt] - m_new);
      R.m_run[qt] = m_new;
      R.L[qt] *= alpha;
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) R.O[qt][dt] *= alpha;
    }
    const float neg_m = -R.m_run[qt];
    // P rounded to bf16 (the PV operand; the row sum uses the same rounded values).  The cast is
    // gfx950's v_cvt_pk_bf16_f32: round to nearest even, two values per instruction.
    bf16x8_t pt[2];
#pragma unroll
    for (int kt = 0; kt < 4; ++kt)
#pragma unroll
      for (int v = 0; v < 4; ++v)
        pt[kt >> 1][(kt & 1) * 4 + v] = (__bf16)__builtin_amdgcn_exp2f(fmaf(s[kt][v], scale, neg_m));
    R.L[qt] = mfma16x16x32(ones, pt[0], R.L[qt]);
    R.L[qt] = mfma16x16x32(ones, pt[1], R.L[qt]);
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {
      R.O[qt][dt] = mfma16x16x32(as_bf16x8(vv[dt][0]), pt[0], R.O[qt][dt]);
      R.O[qt][dt] = mfma16x16x32(as_bf16x8(vv[dt][1]), pt[1], R.O[qt][dt]);
    }
  }
}

// The chunked-prefill rows' block step: rows_block's math for the two row tiles of a prefill wave,
// with the block's K and V fragments read from its LDS copy as they are used -- the scores of both
// row tiles per K tile, then the softmax, then O per V tile -- so K and V are never live at once
// (about 40 fewer registers than rows_block over fragments loaded beforehand).  MASKED = false is an
// interior block, unmasked for every row of the wave, the rows past the wave's tokens included (their
// scores come from zero queries, they never move another row's max and are never written); it has no
// masking code at all, so the block loop over interior blocks stays free of it.
template <bool MASKED>
__device__ __forceinline__ void prefill_rows_block(QRows<2>& R, const uint4* __restrict__ kbuf,
                                                   const uint4* __restrict__ vbuf, int kb, int key_lo,
                                                   int key_hi, int window) {
  const int lane = threadIdx.x & 63;
  const int g = lane >> 4;
  const bf16x8_t ones = as_bf16x8(make_uint4(0x3f803f80u, 0x3f803f80u, 0x3f803f80u, 0x3f803f80u));
  // The queries are pre-scaled by head_dim^-0.5 log2(e) (attn_prefill_body), and each row's score
  // MFMAs start from -m (its running max), so they produce s * scale - m directly and P = 2^(score)
  // needs no FMA.  A row still at the sentinel max (no key seen yet) starts from 0 instead.
  f32x4_t s[2][4];
  float c0[2];
#pragma unroll
  for (int qt = 0; qt < 2; ++qt) c0[qt] = R.m_run[qt] > kMaxSentinel ? -R.m_run[qt] : 0.f;
#pragma unroll
  for (int kt = 0; kt < 4; ++kt) {
    const uint4 k0 = kbuf[kt * 128 + lane], k1 = kbuf[kt * 128 + 64 + lane];
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) {
      s[qt][kt] = mfma16x16x32(as_bf16x8(k0), R.qf[qt][0], f32x4_t{c0[qt], c0[qt], c0[qt], c0[qt]});
      s[qt][kt] = mfma16x16x32(as_bf16x8(k1), R.qf[qt][1], s[qt][kt]);
    }
  }
  bf16x8_t pt[2][2];
#pragma unroll
  for (int qt = 0; qt < 2; ++qt) {
    // lane holds S^T[key kb + tile_key(kt, 4g + v)][qrow n], relative to the row's running max
    float bmax = -INFINITY;
    if constexpr (!MASKED) {
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
#pragma unroll
        for (int v = 0; v < 4; ++v) bmax = fmaxf(bmax, s[qt][kt][v]);
    } else {
      const int p = R.qpos[qt];
      const int lo = max(key_lo, window > 0 ? p - window + 1 : 0);
      const int hi = min(p, key_hi - 1);
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int key = kb + tile_key(kt, 4 * g + v);
          const bool ok = R.qval[qt] && key >= lo && key <= hi;
          s[qt][kt][v] = ok ? s[qt][kt][v] : -INFINITY;
          bmax = fmaxf(bmax, s[qt][kt][v]);
        }
    }
    bmax = max_lane_groups(bmax);
    // the max moves when the block's exceeds it by more than kMaxSlack; a row at the sentinel takes
    // the block's max as soon as it sees a key (a block fully masked for it leaves it at the sentinel)
    const bool fresh = R.m_run[qt] <= kMaxSentinel;
    const bool move = bmax > (fresh ? -INFINITY : kMaxSlack);
    if (__ballot(move)) {
      const float delta = move ? bmax : 0.f;  // scores are relative to the old max: shift by delta
      const float m_new = (fresh ? 0.f : R.m_run[qt]) + delta;
      const float alpha = move ? __builtin_amdgcn_exp2f(R.m_run[qt] - m_new) : 1.f;
      R.m_run[qt] = move ? m_new : R.m_run[qt];
      R.L[qt] *= alpha;
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) R.O[qt][dt] *= alpha;
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
#pragma unroll
        for (int v = 0; v < 4; ++v) s[qt][kt][v] -= delta;
    }
    // P rounded to bf16 (the PV operand; the row sum uses the same rounded values)
#pragma unroll
    for (int kt = 0; kt < 4; ++kt)
#pragma unroll
      for (int v = 0; v < 4; ++v) pt[qt][kt >> 1][(kt & 1) * 4 + v] = (__bf16)__builtin_amdgcn_exp2f(s[qt][kt][v]);
    R.L[qt] = mfma16x16x32(ones, pt[qt][0], R.L[qt]);
    R.L[qt] = mfma16x16x32(ones, pt[qt][1], R.L[qt]);
  }
  const bool tail = MASKED && kb + 64 > key_hi;  // values of keys at or past key_hi are zeroed (maybe unwritten)
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) {
    uint4 v0 = vbuf[dt * 64 + lane], v1 = vbuf[256 + dt * 64 + lane];
    if (tail) {
      v0 = mask_keys(v0, kb + 8 * g, INT_MIN, key_hi);
      v1 = mask_keys(v1, kb + 32 + 8 * g, INT_MIN, key_hi);
    }
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) {
      R.O[qt][dt] = mfma16x16x32(as_bf16x8(v0), pt[qt][0], R.O[qt][dt]);
      R.O[qt][dt] = mfma16x16x32(as_bf16x8(v1), pt[qt][1], R.O[qt][dt]);
    }
  }
}

// One work item (<= 4 tokens x the 8 heads of a kv head, one key split) by one wave, K and V
// streamed from the slab; writes a partial record (m, l, O[64]) per query row.
// TREE: the batch is one tree-verify sequence; token (= node) i sits at position
// tv.start + depth[i] and sees the committed keys below tv.start plus the tree slots its mask row
// sets (FastVerify._tset masks).
// LEAN: only K is loaded a block ahead; a block's V is loaded at the block's start and is first
// read by its PV products, after the scores and the softmax.  Three K/V tiles live instead of four
// (32 fewer registers): the step kernel that fits three waves per SIMD, where the other waves of the
// SIMD hide what the shorter V lead leaves exposed.
template <int QT, bool TREE, bool LEAN = false>
__device__ __forceinline__ void attn_item(const flyai_attn_item& it, int item_idx,
                                          const uint16_t* __restrict__ q,
                                          const uint16_t* __restrict__ k_pool,
                                          const uint16_t* __restrict__ v_pool,
                                          const int64_t* __restrict__ kv_base,
                                          const int32_t* __restrict__ kv_cap, int window, int Hq,
                                          float* __restrict__ partials,
                                          const flyai_attn_group* __restrict__ groups, int n_groups,
                                          const float* __restrict__ sinks, uint16_t* __restrict__ out,
                                          const TreeView& tv) {
  const int lane = threadIdx.x & 63;
  const int n = lane & 15, g = lane >> 4;
  // the item is its rows' whole key range (a group index outside the plan reads as "not single")
  const bool single = it.group >= 0 && it.group < n_groups && groups[it.group].n_splits == 1;
  const int cap = kv_cap[it.seq];
  const int64_t base = kv_base[it.seq] + (int64_t)it.kv_head * cap * 64;
  const uint16_t* K = k_pool + base;
  const uint16_t* Vt = v_pool + base;
  QRows<QT> R;
  rows_init<QT, TREE>(R, q, it.tok, it.ntok, it.pos0, it.kv_head, Hq, tv);

  const int kb_first = it.key_lo & ~63;
  // Blocks fully inside every valid query row's key range need no score mask (wave-uniform test).
  // In a tree only committed keys (below tree->start) can be unmasked for every row.
  int pos_last, int_hi;
  if (TREE) {
    int dmax = 0;
    for (int i = 0; i < it.ntok; ++i) dmax = max(dmax, tv.depth[it.tok + i]);
    pos_last = tv.start + dmax;
    int_hi = min(it.key_hi - 1, tv.start - 1);
  } else {
    pos_last = it.pos0 + it.ntok - 1;
    int_hi = min(it.key_hi - 1, it.pos0);
  }
  const int int_lo = max(it.key_lo, window > 0 ? pos_last - window + 1 : 0);
  // K and V of the next block are loaded while the current block computes
  uint4 kc[4][2], kn[4][2], vv[4][2], vn[4][2];
  load_k_tile(kc, K, kb_first, lane);
  if (!LEAN) load_v_tile(vv, Vt, kb_first, lane);
  for (int kb = kb_first; kb < it.key_hi; kb += 64) {
    const bool more = kb + 64 < it.key_hi;
    if (LEAN) load_v_tile(vv, Vt, kb, lane);
    if (more) {
      load_k_tile(kn, K, kb + 64, lane);
      if (!LEAN) load_v_tile(vn, Vt, kb + 64, lane);
    }
    const bool interior = kb >= int_lo && kb + 63 <= int_hi;
    rows_block<QT, TREE>(R, kc, vv, kb, interior, it.key_lo, it.key_hi, window, tv);
    if (more) {
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        kc[t][0] = kn[t][0];
        kc[t][1] = kn[t][1];
        if (!LEAN) {
          vv[t][0] = vn[t][0];
          vv[t][1] = vn[t][1];
        }
      }
    }
  }
  // partial record per query row: [m, l, O[64]]; O^T layout: lane holds dims 16dt + 4g + v of qrow n.
  // A row whose whole key range is this item is finished here with the merge's arithmetic for one
  // split (the same operations in the same order, so the same bits), and the merge skips its group.
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    const float l = R.L[qt][0];
    const int rq = 16 * qt + n;
    if (!R.qval[qt]) continue;
    if (single) {
      const int h = it.kv_head * 8 + (rq & 7);
      const float sink = sinks[h] * kLog2e;
      const float M = fmaxf(sink, R.m_run[qt]);
      float L = exp2f(sink - M);
      const float wgt = exp2f(R.m_run[qt] - M);
      L += l * wgt;
      const float inv = 1.0f / L;
      uint16_t* o = out + ((size_t)(it.tok + (rq >> 3)) * Hq + h) * 64;
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) {
        float a[4];
#pragma unroll
        for (int v = 0; v < 4; ++v) a[v] = 0.f + R.O[qt][dt][v] * wgt;
        const uint32_t lo = (uint32_t)f2bf(a[0] * inv) | ((uint32_t)f2bf(a[1] * inv) << 16);
        const uint32_t hi = (uint32_t)f2bf(a[2] * inv) | ((uint32_t)f2bf(a[3] * inv) << 16);
        *reinterpret_cast<uint2*>(o + 16 * dt + 4 * g) = make_uint2(lo, hi);
      }
      continue;
    }
    float* rec = partials + ((size_t)item_idx * kAttnRows + rq) * kPartFloats;
    if (g == 0) {
      rec[0] = R.m_run[qt];
      rec[1] = l;
    }
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int v = 0; v < 4; ++v) rec[2 + 16 * dt + 4 * g + v] = R.O[qt][dt][v];
  }
}

// One launch for every item; the body is chosen per item (uniform across the wave).
__global__ __launch_bounds__(64, 2) void attn_partial_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k_pool,
    const uint16_t* __restrict__ v_pool, const int64_t* __restrict__ kv_base,
    const int32_t* __restrict__ kv_cap, int window, int Hq,
    const flyai_attn_item* __restrict__ items, const int32_t* __restrict__ n_live,
    float* __restrict__ partials, const flyai_attn_group* __restrict__ groups, int n_groups,
    const float* __restrict__ sinks, uint16_t* __restrict__ out) {
  // a graph-replayed step launches the plan's capacity; items past this step's count exit
  if (n_live && (int)blockIdx.x >= *n_live) return;
  const flyai_attn_item it = items[blockIdx.x];
  if (it.ntok <= 2)
    attn_item<1, false>(it, blockIdx.x, q, k_pool, v_pool, kv_base, kv_cap, window, Hq, partials, groups, n_groups, sinks, out,
                        TreeView{});
  else
    attn_item<2, false>(it, blockIdx.x, q, k_pool, v_pool, kv_base, kv_cap, window, Hq, partials, groups, n_groups, sinks, out,
                        TreeView{});
}

// The items of one tree-verify sequence (flyai_stage_forward_tree).  Its own kernel: the mask words
// of the tree rows take registers the decode kernel's two waves per SIMD do not have to spare.
__global__ __launch_bounds__(64, 1) void attn_tree_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k_pool,
    const uint16_t* __restrict__ v_pool, const int64_t* __restrict__ kv_base,
    const int32_t* __restrict__ kv_cap, int window, int Hq,
    const flyai_attn_item* __restrict__ items, float* __restrict__ partials,
    const flyai_attn_group* __restrict__ groups, int n_groups, const float* __restrict__ sinks,
    uint16_t* __restrict__ out, const flyai_attn_tree* __restrict__ tree) {
  const flyai_attn_item it = items[blockIdx.x];
  const char* tb = reinterpret_cast<const char*>(tree);
  TreeView tv;
  tv.start = tree->start;
  tv.n = tree->n_nodes;
  tv.words = tree->words;
  tv.depth = reinterpret_cast<const int32_t*>(tb + tree->depth_off);
  tv.mask = reinterpret_cast<const uint64_t*>(tb + tree->mask_off[window > 0 ? 1 : 0]);
  if (it.ntok <= 2)
    attn_item<1, true>(it, blockIdx.x, q, k_pool, v_pool, kv_base, kv_cap, window, Hq, partials, groups, n_groups, sinks, out,
                       tv);
  else
    attn_item<2, true>(it, blockIdx.x, q, k_pool, v_pool, kv_base, kv_cap, window, Hq, partials, groups, n_groups, sinks, out,
                       tv);
}

// ---- chunked-prefill rows -------------------------------------------------------------------------
// Work item = (sequence, kv head, up to kPrefillTokens consecutive query tokens): a workgroup of
// kPrefillWaves waves, wave w owning tokens 4w .. 4w+3 of the item (32 query rows, the same math as a
// decode item).  The item's 64-key blocks are staged once in LDS for all waves -- the tiled slab
// block is copied as it is, global -> LDS directly (global_load_lds, no register staging), so each
// wave reads its K and V fragments as contiguous KiBs -- through two buffers with one barrier per
// block, the next block's loads in flight while the current one computes.  Block kb sits in buffer
// (kb / 64) % 2; the buffers are separate LDS arrays picked at compile time (the block loop is
// unrolled by parity), so the compiler can tell the reads of one from the DMA writes into the other
// and a block's reads do not wait for the next block's loads.  No key splits: each wave ends with
// the sink and the normalisation and writes its rows.
constexpr int kPrefillWaves = kPrefillTokens / 4;

__device__ __forceinline__ void attn_prefill_body(
    int bid, const uint16_t* __restrict__ q, const uint16_t* __restrict__ k_pool,
    const uint16_t* __restrict__ v_pool, const int64_t* __restrict__ kv_base,
    const int32_t* __restrict__ kv_cap, const float* __restrict__ sinks, int window, int Hq,
    const flyai_attn_item* __restrict__ items, uint16_t* __restrict__ out) {
  typedef __attribute__((address_space(3))) void* lds_ptr;
  __shared__ uint4 kvs0[2][512], kvs1[2][512];  // the two buffers: [K, V][one 64-key block: 4096 bf16]
  const flyai_attn_item it = items[bid];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int n = lane & 15, g = lane >> 4;
  const int cap = kv_cap[it.seq];
  const int64_t base = kv_base[it.seq] + (int64_t)it.kv_head * cap * 64;
  const uint4* Kb = reinterpret_cast<const uint4*>(k_pool + base);
  const uint4* Vb = reinterpret_cast<const uint4*>(v_pool + base);
  // this wave's tokens and the keys they see
  const int ntw = max(0, min(4, it.ntok - 4 * wave));
  const int tok_w = it.tok + 4 * wave, pos_w = it.pos0 + 4 * wave;
  QRows<2> R;
  rows_init<2, false>(R, q, tok_w, ntw, pos_w, it.kv_head, Hq, TreeView{});
  // the queries pre-scaled by head_dim^-0.5 log2(e), rounded to bf16 (prefill_rows_block's scores)
#pragma unroll
  for (int qt = 0; qt < 2; ++qt)
#pragma unroll
    for (int hh = 0; hh < 2; ++hh)
#pragma unroll
      for (int i = 0; i < 8; ++i) R.qf[qt][hh][i] = (__bf16)((float)R.qf[qt][hh][i] * (0.125f * kLog2e));
  const int pos_last = pos_w + max(ntw, 1) - 1;
  const int lo_w = max(it.key_lo, window > 0 ? pos_w - window + 1 : 0);  // the wave's first visible key
  const int int_lo = max(it.key_lo, window > 0 ? pos_last - window + 1 : 0);
  const int int_hi = min(it.key_hi - 1, pos_w);

  // staging: load instruction j (j < 4) of wave w copies uint4s s0 .. s0 + 63, s0 = 256 j + 64 w, of
  // the block (K: s < 512, V: s >= 512), lane L the one at s0 + L (the DMA's lane order).  The
  // source is a wave-uniform block address plus the lane's fixed 16 L bytes, and the wave index is
  // read into a scalar, so a block's loads cost scalar adds only (no per-lane 64-bit address math).
  constexpr int kPer = 1024 / (64 * kPrefillWaves);
  const int kb_first = it.key_lo & ~63;
  const int wave_s = __builtin_amdgcn_readfirstlane(wave);
  const uint32_t lane_off = (uint32_t)lane * 16u;
  auto issue = [&](uint4 (&dst)[2][512], int kb) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const int s0 = 64 * kPrefillWaves * j + 64 * wave_s;  // wave-uniform
      const char* blk = reinterpret_cast<const char*>(s0 < 512 ? Kb : Vb) + ((size_t)kb * 8 + (s0 & 511)) * 16;
      __builtin_amdgcn_global_load_lds((const void*)(blk + lane_off), (lds_ptr)(&dst[0][0] + s0), 16, 0, 0);
    }
  };
  // the wave's own loads have landed (vector memory loads complete in issue order; the DMA counts
  // as a load), then the barrier: every wave's have
  auto landed = [&]() __attribute__((always_inline)) {
    __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
    lds_barrier();
  };
  if ((kb_first >> 6) & 1) issue(kvs1, kb_first); else issue(kvs0, kb_first);
  landed();
  // One block: the next one's loads go out into the other buffer (every wave finished reading it
  // before the last barrier), this wave's rows take the block (if any of their keys is in it), the
  // loads land, one barrier.  Every wave steps through the same blocks, so the workgroup's barriers
  // match; each wave's blocks split into a masked run before its interior blocks (window start), the
  // interior run, and a masked run after (causal diagonal, the item's end), each its own loop, so the
  // interior loop carries no masking code.
  auto step = [&](int kb, auto masked, auto parity) __attribute__((always_inline)) {
    uint4 (&cur)[2][512] = decltype(parity)::value ? kvs1 : kvs0;
    uint4 (&nxt)[2][512] = decltype(parity)::value ? kvs0 : kvs1;
    if (kb + 64 < it.key_hi) issue(nxt, kb + 64);
    // (an interior block is seen by the wave's rows: no test)
    if (!decltype(masked)::value || (ntw > 0 && kb <= pos_last && kb + 63 >= lo_w))
      prefill_rows_block<decltype(masked)::value>(R, cur[0], cur[1], kb, it.key_lo, it.key_hi, window);
    landed();
  };
  int kb = kb_first;
  auto run = [&](auto more, auto masked) __attribute__((always_inline)) {
    while (more(kb)) {
      if (((kb >> 6) & 1) == 0) {
        step(kb, masked, std::false_type{});
        kb += 64;
        if (!more(kb)) break;
      }
      step(kb, masked, std::true_type{});
      kb += 64;
    }
  };
  run([&](int k) { return k < it.key_hi && k < int_lo; }, std::true_type{});
  run([&](int k) { return k < it.key_hi && k >= int_lo && k + 63 <= int_hi; }, std::false_type{});
  run([&](int k) { return k < it.key_hi; }, std::true_type{});
  // out = O 2^(m-M) / (l 2^(m-M) + 2^(sink-M)), M = max(m, sink), all in base-2 units: the merge of a
  // single split
#pragma unroll
  for (int qt = 0; qt < 2; ++qt) {
    const float l = R.L[qt][0];
    const int rq = 16 * qt + n;
    if (!R.qval[qt]) continue;
    const int h = it.kv_head * 8 + (rq & 7);
    const float sink = sinks[h] * kLog2e;  // base-2 units, as the running max
    const float M = fmaxf(R.m_run[qt], sink);
    const float w = exp2f(R.m_run[qt] - M);
    const float inv = 1.0f / (l * w + exp2f(sink - M));
    uint16_t* o = out + ((size_t)(tok_w + (rq >> 3)) * Hq + h) * 64;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {
      const uint32_t lo = (uint32_t)f2bf(R.O[qt][dt][0] * w * inv) | ((uint32_t)f2bf(R.O[qt][dt][1] * w * inv) << 16);
      const uint32_t hi = (uint32_t)f2bf(R.O[qt][dt][2] * w * inv) | ((uint32_t)f2bf(R.O[qt][dt][3] * w * inv) << 16);
      *reinterpret_cast<uint2*>(o + 16 * dt + 4 * g) = make_uint2(lo, hi);
    }
  }
}

__global__ __launch_bounds__(64 * kPrefillWaves, 2) void attn_prefill_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k_pool,
    const uint16_t* __restrict__ v_pool, const int64_t* __restrict__ kv_base,
    const int32_t* __restrict__ kv_cap, const float* __restrict__ sinks, int window, int Hq,
    const flyai_attn_item* __restrict__ items, uint16_t* __restrict__ out) {
  attn_prefill_body(blockIdx.x, q, k_pool, v_pool, kv_base, kv_cap, sinks, window, Hq, items, out);
}

// A step with prefill items and split items in one launch: prefill workgroups and workgroups of
// kPrefillWaves split items (one per wave; the split body has no workgroup barrier, so a wave past the
// item count leaves alone).
// LEAN (every split item has <= 2 tokens, one row tile): the split body is the lean one and the
// kernel fits three waves per SIMD, as the prefill body alone does; the split workgroups are spread
// evenly through the grid, so the bandwidth-bound split items stream KV from HBM while the prefill
// items (VALU- and MFMA-bound, their keys L2-resident) compute.  Otherwise (row tiles of up to 4
// tokens) both bodies fit two waves per SIMD, the prefill workgroups come first and the split items
// fill the slots the prefill workgroups free towards their end.
template <bool LEAN>
__global__ __launch_bounds__(64 * kPrefillWaves, LEAN ? 3 : 2) void attn_step_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k_pool,
    const uint16_t* __restrict__ v_pool, const int64_t* __restrict__ kv_base,
    const int32_t* __restrict__ kv_cap, int window, int Hq,
    const flyai_attn_item* __restrict__ items, int n_items, const int32_t* __restrict__ n_live,
    float* __restrict__ partials, const flyai_attn_group* __restrict__ groups, int n_groups,
    const float* __restrict__ sinks, uint16_t* __restrict__ out, const flyai_attn_item* __restrict__ pitems,
    int n_pitems) {
  const int b = blockIdx.x;
  int split_wg;  // this workgroup's index among the split workgroups, or -1 (a prefill item)
  int pidx = b;
  if (LEAN) {
    // Bresenham spread over groups of 8 blocks: group gi is split group d0 when
    // floor((gi+1) DG/TG) > floor(gi DG/TG) = d0 (exactly DG of the TG groups); otherwise it is
    // prefill group gi - d0.  Whole groups of 8 keep prefill item i on block i mod 8, i.e. on
    // XCD i mod 8 (workgroups are dealt round-robin over the 8 XCDs) as in the prefill-only
    // launch: the plan lists a chunk's kv heads consecutively, so each XCD's L2 holds the K/V of
    // one kv head (with 8) instead of all of them.
    const int P = n_pitems, D = (n_items + kPrefillWaves - 1) / kPrefillWaves;
    const int64_t PG = (P + 7) / 8, DG = (D + 7) / 8, TG = PG + DG;
    const int gi = b >> 3, l8 = b & 7;
    const int d0 = (int)(gi * DG / TG), d1 = (int)((gi + 1) * DG / TG);
    if (d1 > d0) {
      split_wg = 8 * d0 + l8;
      if (split_wg >= D) return;
    } else {
      split_wg = -1;
      pidx = 8 * (gi - d0) + l8;
      if (pidx >= P) return;
    }
  } else {
    split_wg = b < n_pitems ? -1 : b - n_pitems;
  }
  if (split_wg < 0) {
    attn_prefill_body(pidx, q, k_pool, v_pool, kv_base, kv_cap, sinks, window, Hq, pitems, out);
    return;
  }
  const int idx = split_wg * kPrefillWaves + (int)(threadIdx.x >> 6);
  if (idx >= n_items || (n_live && idx >= *n_live)) return;
  const flyai_attn_item it = items[idx];
  if (LEAN || it.ntok <= 2)
    attn_item<1, false, LEAN>(it, idx, q, k_pool, v_pool, kv_base, kv_cap, window, Hq, partials, groups, n_groups,
                              sinks, out, TreeView{});
  else
    attn_item<2, false>(it, idx, q, k_pool, v_pool, kv_base, kv_cap, window, Hq, partials, groups, n_groups, sinks,
                        out, TreeView{});
}

int launch_attn_prefill(const uint16_t* q, const uint16_t* k_pool, const uint16_t* v_pool,
                        const int64_t* kv_base, const int32_t* kv_cap, const float* sinks, int window, int Hq,
                        const flyai_attn_item* pitems, int n_pitems, uint16_t* out, hipStream_t s) {
  if (n_pitems == 0) return FLYAI_OK;
  hipLaunchKernelGGL(attn_prefill_kernel, dim3(n_pitems), dim3(64 * kPrefillWaves), 0, s, q, k_pool, v_pool,
                     kv_base, kv_cap, sinks, window, Hq, pitems, out);
  return check_launch("attn_prefill");
}

// Merge: per query row, in base-2 units (s' = s log2(e), sink' = sink log2(e)): M = max(sink',
// max_s m_s), L = 2^(sink'-M) + sum_s l_s 2^(m_s-M), out = bf16(sum_s O_s 2^(m_s-M) / L) -- the
// softmax with the sink column, e^(s - m) = 2^(s' - m').  Thread (row = tid/8, part = tid%8) writes 8 dims.
constexpr int kMergeM = 16, kMergeChunk = 4;

__global__ __launch_bounds__(256) void attn_merge_kernel(const float* __restrict__ partials,
                                                         const flyai_attn_group* __restrict__ groups,
                                                         const float* __restrict__ sinks, int Hq,
                                                         const int32_t* __restrict__ n_live,
                                                         uint16_t* __restrict__ out) {
  if (n_live && (int)blockIdx.x >= *n_live) return;  // as in attn_partial_kernel
  const flyai_attn_group gr = groups[blockIdx.x];
  if (gr.n_splits == 1) return;  // finished by its only item (attn_item)
  const int rq = threadIdx.x >> 3, part = threadIdx.x & 7;
  const int ti = rq >> 3;
  if (ti >= gr.ntok) return;
  const int h = gr.kv_head * 8 + (rq & 7);
  const float sink = sinks[h] * kLog2e;  // the partial maxima are in base-2 units
  const int n = gr.n_splits;
  auto rec_of = [&](int s) {
    return partials + ((size_t)(gr.first_item + min(s, n - 1)) * kAttnRows + rq) * kPartFloats;
  };
  // The split maxima are read kMergeM at a time and the split records kMergeChunk at a time, every
  // load of a batch issued before its first use (a round trip per batch, not per split); indices past
  // the last split are clamped for the loads and left out.  The sums run in split order as before.
  float M = sink;
  for (int s0 = 0; s0 < n; s0 += kMergeM) {
    float mv[kMergeM];
#pragma unroll
    for (int j = 0; j < kMergeM; ++j) mv[j] = rec_of(s0 + j)[0];
#pragma unroll
    for (int j = 0; j < kMergeM; ++j)
      if (s0 + j < n) M = fmaxf(M, mv[j]);
  }
  float L = exp2f(sink - M);
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  for (int s0 = 0; s0 < n; s0 += kMergeChunk) {
    float rm[kMergeChunk], rl[kMergeChunk], rd[kMergeChunk][8];
#pragma unroll
    for (int j = 0; j < kMergeChunk; ++j) {
      const float* rec = rec_of(s0 + j);
      rm[j] = rec[0];
      rl[j] = rec[1];
#pragma unroll
      for (int d = 0; d < 8; ++d) rd[j][d] = rec[2 + part * 8 + d];
    }
#pragma unroll
    for (int j = 0; j < kMergeChunk; ++j)
      if (s0 + j < n) {
        const float wgt = exp2f(rm[j] - M);
        L += rl[j] * wgt;
#pragma unroll
        for (int d = 0; d < 8; ++d) acc[d] += rd[j][d] * wgt;
      }
  }
  const float inv = 1.0f / L;
  uint16_t* o = out + ((size_t)(gr.tok + ti) * Hq + h) * 64 + part * 8;
  uint32_t wv[4];
#pragma unroll
  for (int d = 0; d < 4; ++d)
    wv[d] = (uint32_t)f2bf(acc[2 * d] * inv) | ((uint32_t)f2bf(acc[2 * d + 1] * inv) << 16);
  *reinterpret_cast<uint4*>(o) = make_uint4(wv[0], wv[1], wv[2], wv[3]);
}

// n_items / n_groups size the grids; counts (nullable) holds this step's live item and group
// counts on the device, for launches sized by a plan capacity (graph replay)
int launch_attn(const uint16_t* q, const uint16_t* k_pool, const uint16_t* v_pool,
                const int64_t* kv_base, const int32_t* kv_cap, const float* sinks, int window,
                int Hq, const flyai_attn_item* items, int n_items, int n_small,
                const flyai_attn_group* groups, int n_groups, const int32_t* counts, float* partials,
                uint16_t* out, const flyai_attn_tree* tree, bool merge, hipStream_t s) {
  if (n_items == 0) return FLYAI_OK;
  (void)n_small;  // the plan's two ranges share one launch
  if (tree)  // launched directly with exact counts (never from a graph)
    hipLaunchKernelGGL(attn_tree_kernel, dim3(n_items), dim3(64), 0, s, q, k_pool, v_pool, kv_base, kv_cap, window,
                       Hq, items, partials, groups, n_groups, sinks, out, tree);
  else
    hipLaunchKernelGGL(attn_partial_kernel, dim3(n_items), dim3(64), 0, s, q, k_pool, v_pool, kv_base,
                       kv_cap, window, Hq, items, counts, partials, groups, n_groups, sinks, out);
  int rc = check_launch(tree ? "attn_tree" : "attn_partial");
  if (rc) return rc;
  if (!merge) return FLYAI_OK;  // every group has one split: the items wrote the output
  hipLaunchKernelGGL(attn_merge_kernel, dim3(n_groups), dim3(256), 0, s, partials, groups, sinks,
                     Hq, counts ? counts + 1 : nullptr, out);
  return check_launch("attn_merge");
}

// One launch of attn_step_kernel for a step with both item kinds, then the merge as in launch_attn.
// lean: every split item has <= 2 tokens (the planner's n_small covers all of them).
int launch_attn_step(const uint16_t* q, const uint16_t* k_pool, const uint16_t* v_pool, const int64_t* kv_base,
                     const int32_t* kv_cap, const float* sinks, int window, int Hq, const flyai_attn_item* items,
                     int n_items, const flyai_attn_group* groups, int n_groups, const int32_t* counts, float* partials,
                     const flyai_attn_item* pitems, int n_pitems, uint16_t* out, bool merge, bool lean,
                     hipStream_t s) {
  const int n_split_wg = (n_items + kPrefillWaves - 1) / kPrefillWaves;
  // the lean kernel deals whole groups of 8 blocks (see attn_step_kernel)
  const int grid = lean ? 8 * ((n_pitems + 7) / 8 + (n_split_wg + 7) / 8) : n_pitems + n_split_wg;
  if (grid == 0) return FLYAI_OK;
  hipLaunchKernelGGL(lean ? attn_step_kernel<true> : attn_step_kernel<false>, dim3(grid), dim3(64 * kPrefillWaves),
                     0, s, q, k_pool, v_pool, kv_base, kv_cap, window, Hq, items, n_items, counts, partials, groups,
                     n_groups, sinks, out, pitems, n_pitems);
  int rc = check_launch("attn_step");
  if (rc) return rc;
  if (!merge || n_items == 0) return FLYAI_OK;
  hipLaunchKernelGGL(attn_merge_kernel, dim3(n_groups), dim3(256), 0, s, partials, groups, sinks,
                     Hq, counts ? counts + 1 : nullptr, out);
  return check_launch("attn_merge");
}

// Groups of <= 2 query tokens (one 16-row tile) are emitted first, then the larger ones, so the two
// kernel variants each take one contiguous item range; a group's splits stay consecutive.
// Sequences with q_len >= prefill_min (0: none) become prefill items instead (attn_prefill_kernel):
// kPrefillTokens tokens x one kv head each, the chunk's last tiles first (they see the most keys).
int attn_plan(const int32_t* q_lens, const int32_t* starts, int S, int Hkv, int window,
              int split_keys, flyai_attn_item* items, int max_items, flyai_attn_group* groups,
              int max_groups, int* n_items, int* n_groups, int* n_small, int prefill_min,
              flyai_attn_item* pitems, int max_pitems, int* n_pitems) {
  int ni = 0, ng = 0, np = 0;
  {
    int tok = 0;
    for (int b = 0; b < S; ++b) {
      const int ql = q_lens[b], st = starts[b];
      if (prefill_min > 0 && ql >= prefill_min) {
        for (int i0 = (ql - 1) / kPrefillTokens * kPrefillTokens; i0 >= 0; i0 -= kPrefillTokens) {
          const int nt = ql - i0 < kPrefillTokens ? ql - i0 : kPrefillTokens;
          const int p_first = st + i0;
          for (int g = 0; g < Hkv; ++g) {
            if (np >= max_pitems)
              return set_error(FLYAI_ERANGE, "prefill attention plan exceeds capacity (%d items)", max_pitems);
            flyai_attn_item& it = pitems[np++];
            it.seq = b;
            it.kv_head = g;
            it.tok = tok + i0;
            it.ntok = nt;
            it.pos0 = p_first;
            it.key_lo = window > 0 ? (p_first - window + 1 > 0 ? p_first - window + 1 : 0) : 0;
            it.key_hi = p_first + nt;
            it.group = -1;
          }
        }
      }
      tok += ql;
    }
  }
  *n_pitems = np;
  for (int pass = 0; pass < 2; ++pass) {
    if (pass == 1) *n_small = ni;
    int tok = 0;
    for (int b = 0; b < S; ++b) {
      const int ql = q_lens[b], st = starts[b];
      if (prefill_min > 0 && ql >= prefill_min) {
        tok += ql;
        continue;
      }
      for (int i0 = 0; i0 < ql; i0 += 4) {
        const int nt = ql - i0 < 4 ? ql - i0 : 4;
        if ((nt <= 2) != (pass == 0)) continue;
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
  }
  *n_items = ni;
  *n_groups = ng;
  return FLYAI_OK;
}

// Tree-verify plan: the n nodes of one sequence (seq 0, tokens 0..n-1) at committed length st, in
// groups of <= 4 consecutive nodes; every group's keys run to st + n (the mask picks the tree slots),
// and from the window start of its shallowest node on sliding layers.
int attn_plan_tree(int st, int n, const int32_t* depth, int Hkv, int window, int split_keys,
                   flyai_attn_item* items, int max_items, flyai_attn_group* groups, int max_groups,
                   int* n_items, int* n_groups, int* n_small) {
  int ni = 0, ng = 0;
  for (int i0 = 0; i0 < n; i0 += 4) {
    const int nt = n - i0 < 4 ? n - i0 : 4;
    int dmin = depth[i0];
    for (int i = 1; i < nt; ++i) dmin = depth[i0 + i] < dmin ? depth[i0 + i] : dmin;
    const int p_first = st + dmin;
    const int key_hi = st + n;
    const int key_lo = window > 0 ? (p_first - window + 1 > 0 ? p_first - window + 1 : 0) : 0;
    const int kb0 = key_lo & ~63;
    const int nsplit = (key_hi - kb0 + split_keys - 1) / split_keys;
    for (int g = 0; g < Hkv; ++g) {
      if (ng >= max_groups || ni + nsplit > max_items)
        return set_error(FLYAI_ERANGE, "tree attention plan exceeds capacity (%d items, %d groups)",
                         max_items, max_groups);
      flyai_attn_group& gr = groups[ng];
      gr.first_item = ni;
      gr.n_splits = nsplit;
      gr.tok = i0;
      gr.ntok = nt;
      gr.kv_head = g;
      gr.pad[0] = gr.pad[1] = gr.pad[2] = 0;
      for (int sp = 0; sp < nsplit; ++sp) {
        flyai_attn_item& it = items[ni++];
        it.seq = 0;
        it.kv_head = g;
        it.tok = i0;
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
  *n_items = ni;
  *n_groups = ng;
  *n_small = 0;
  return FLYAI_OK;
}

}  // namespace flyai

using namespace flyai;

extern "C" int flyai_attn_plan(const int32_t* q_lens_host, const int32_t* starts_host,
                               int32_t n_seqs, int32_t Hkv, int32_t window, int32_t split_keys,
                               flyai_attn_item* items_host, int32_t max_items,
                               flyai_attn_group* groups_host, int32_t max_groups, int32_t* n_items,
                               int32_t* n_groups, int32_t* n_items_small) {
  FLYAI_REQUIRE(n_seqs >= 0 && Hkv > 0 && window >= 0 && split_keys >= 64 && split_keys % 64 == 0,
                "attn_plan: split_keys must be a positive multiple of 64");
  FLYAI_REQUIRE(q_lens_host && starts_host && items_host && groups_host && n_items && n_groups &&
                    n_items_small,
                "attn_plan: null pointer");
  for (int b = 0; b < n_seqs; ++b)
    FLYAI_REQUIRE(q_lens_host[b] >= 1 && starts_host[b] >= 0, "attn_plan: bad q_len/start at %d", b);
  int np = 0;
  return attn_plan(q_lens_host, starts_host, n_seqs, Hkv, window, split_keys, items_host, max_items,
                   groups_host, max_groups, n_items, n_groups, n_items_small, 0, nullptr, 0, &np);
}

extern "C" int flyai_attn_plan_prefill(const int32_t* q_lens_host, const int32_t* starts_host,
                                       int32_t n_seqs, int32_t Hkv, int32_t window, int32_t split_keys,
                                       int32_t prefill_min, flyai_attn_item* items_host, int32_t max_items,
                                       flyai_attn_group* groups_host, int32_t max_groups,
                                       flyai_attn_item* pitems_host, int32_t max_pitems, int32_t* n_items,
                                       int32_t* n_groups, int32_t* n_items_small, int32_t* n_pitems) {
  FLYAI_REQUIRE(n_seqs >= 0 && Hkv > 0 && window >= 0 && split_keys >= 64 && split_keys % 64 == 0 &&
                    prefill_min >= 0,
                "attn_plan_prefill: split_keys must be a positive multiple of 64");
  FLYAI_REQUIRE(q_lens_host && starts_host && items_host && groups_host && pitems_host && n_items &&
                    n_groups && n_items_small && n_pitems,
                "attn_plan_prefill: null pointer");
  for (int b = 0; b < n_seqs; ++b)
    FLYAI_REQUIRE(q_lens_host[b] >= 1 && starts_host[b] >= 0, "attn_plan_prefill: bad q_len/start at %d", b);
  return attn_plan(q_lens_host, starts_host, n_seqs, Hkv, window, split_keys, items_host, max_items,
                   groups_host, max_groups, n_items, n_groups, n_items_small, prefill_min, pitems_host,
                   max_pitems, n_pitems);
}

extern "C" int flyai_attn_prefill(const uint16_t* q, const uint16_t* k_pool, const uint16_t* v_pool,
                                  const int64_t* kv_base, const int32_t* kv_cap, const float* sinks,
                                  int32_t window, int32_t Hq, int32_t Hkv, int32_t D,
                                  const flyai_attn_item* pitems_dev, int32_t n_pitems, uint16_t* out,
                                  flyai_stream_t stream) {
  FLYAI_REQUIRE(D == 64 && Hkv > 0 && Hq == 8 * Hkv, "attn_prefill: needs head_dim 64 and 8 query heads per kv head");
  FLYAI_REQUIRE(n_pitems >= 0 && window >= 0, "attn_prefill: bad counts");
  FLYAI_REQUIRE(q && k_pool && v_pool && kv_base && kv_cap && sinks && out && (n_pitems == 0 || pitems_dev),
                "attn_prefill: null pointer");
  return launch_attn_prefill(q, k_pool, v_pool, kv_base, kv_cap, sinks, window, Hq, pitems_dev, n_pitems, out,
                             as_stream(stream));
}

extern "C" size_t flyai_attn_partials_bytes(int32_t n_items) {
  return (size_t)(n_items > 0 ? n_items : 0) * kAttnRows * kPartFloats * sizeof(float);
}

extern "C" int flyai_attn_ragged(const uint16_t* q, const uint16_t* k_pool, const uint16_t* v_pool,
                                 const int64_t* kv_base, const int32_t* kv_cap, const float* sinks,
                                 int32_t window, int32_t Hq, int32_t Hkv, int32_t D,
                                 const flyai_attn_item* items_dev, int32_t n_items,
                                 int32_t n_items_small, const flyai_attn_group* groups_dev,
                                 int32_t n_groups, float* partials, uint16_t* out,
                                 flyai_stream_t stream) {
  FLYAI_REQUIRE(D == 64 && Hkv > 0 && Hq == 8 * Hkv, "attn: needs head_dim 64 and 8 query heads per kv head");
  FLYAI_REQUIRE(n_items >= 0 && n_groups >= 0 && window >= 0 && n_items_small >= 0 &&
                    n_items_small <= n_items,
                "attn: bad counts");
  FLYAI_REQUIRE(q && k_pool && v_pool && kv_base && kv_cap && sinks && out &&
                    (n_items == 0 || (items_dev && groups_dev && partials)),
                "attn: null pointer");
  return launch_attn(q, k_pool, v_pool, kv_base, kv_cap, sinks, window, Hq, items_dev, n_items,
                     n_items_small, groups_dev, n_groups, nullptr, partials, out, nullptr, true,
                     as_stream(stream));
}
