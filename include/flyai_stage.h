/*
 * flyai_stage.h -- C ABI of the MI355X (gfx950) stage-step library libflyai_stage.so.
 *
 * One pipeline stage's continuous-batch forward step for a GPT-OSS-120B-shaped MXFP4 MoE model:
 * ragged packing, router top-k + histogram + permute + combine, MXFP4 expert GEMMs, ragged GQA
 * attention with sinks and a sliding window, and the layer glue around them.
 *
 * Conventions
 *   - Every pointer named *_dev / every tensor argument is DEVICE memory unless the name ends in
 *     _host.  bf16 tensors are passed as uint16_t bit patterns, row-major, densely packed.
 *   - Every launch takes an explicit stream (a hipStream_t, passed as void*; NULL = null stream).
 *   - Return value: 0 on success, a negative FLYAI_E* code on error; flyai_last_error() gives a
 *     message.  Shapes are validated on the host before any launch; nothing aborts the process.
 *   - The library allocates no device memory: scratch comes from caller-provided workspaces whose
 *     sizes the *_bytes functions report.  A stage handle is not thread-safe (one per worker thread,
 *     matching the reference's one ContinuousRingWorker thread per ring,
 *     shard/continuous_batch.py:98-156).
 */
#ifndef FLYAI_STAGE_H
#define FLYAI_STAGE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* flyai_stream_t;

#define FLYAI_OK 0
#define FLYAI_EINVAL -1   /* bad shape / argument */
#define FLYAI_ERANGE -2   /* context or capacity overflow (reference: ContextOverflow,
                             phase0/fastverify.py:23-26), raised before any write */
#define FLYAI_EHIP -3     /* a HIP runtime call failed */

#define FLYAI_ABI_VERSION 2

/* Last error message of the calling thread ("" when none). */
const char* flyai_last_error(void);
int flyai_abi_version(void);

/* ---- a1: ragged packing ----------------------------------------------------------------------
 * Replaces the per-stream position/mask construction of BatchedFastVerify._set
 * (phase0/batchverify.py:149-158, :51-61) and FastVerify._set (phase0/fastverify.py:170-183) with a
 * flat token axis.  Inputs per sequence b (device): q_lens[b] >= 1, starts[b] (committed length =
 * position of its first query token), kv_base[b] (element offset of the sequence's K/V slab in a
 * pool), kv_cap[b] (slab capacity in positions).  Outputs: cu_seqlens[S+1], positions[T],
 * seq_id[T], kv_len[S] = starts+q_lens, kv_slot[T] = kv_base + position*head_dim.
 * *status_dev gets bit 0 set if any kv_len > kv_cap (those tokens get kv_slot = -1) and bit 1 if
 * T > max_tokens (nothing past max_tokens is written). */
int flyai_pack_ragged(const int32_t* q_lens, const int32_t* starts, const int64_t* kv_base,
                      const int32_t* kv_cap, int32_t n_seqs, int32_t head_dim, int32_t max_tokens,
                      int32_t* cu_seqlens, int32_t* positions, int32_t* seq_id, int32_t* kv_len,
                      int64_t* kv_slot, int32_t* status_dev, flyai_stream_t stream);

/* ---- a2: router --------------------------------------------------------------------------------
 * GPT-OSS top-k softmax router; replaces GptOssTopKRouter.forward
 * (transformers/models/gpt_oss/modeling_gpt_oss.py:126-130) and the native path's bf16 router
 * Linear + hub `routing` (transformers/integrations/mxfp4.py:484-487, torch restatement
 * routing_torch_dist :435-444).  x bf16 [T,H], w bf16 [E,H], b bf16 [E].  Logits are the bf16
 * rounding of an fp32 dot product in a fixed order (64 lane partials, lane l summing
 * k = 512j + 8l + i in order, then a xor butterfly 32..1) plus bias; top-k by (value desc, id asc);
 * softmax over the k selected values in fp32; each row's ids sorted ascending with their weights
 * (a row of NaN logits selects nothing by value; its slots get id 0).
 * H % 8 == 0, H <= 7168, E % 4 == 0, E <= 256, k in {2, 4, 8}.  logits_out (fp32 [T,E], required) receives the
 * bf16-valued logits and is the scratch between the logits and top-k kernels. */
int flyai_router_topk_softmax(const uint16_t* x, const uint16_t* w, const uint16_t* b, int32_t T,
                              int32_t H, int32_t E, int32_t k, int32_t* topk_ids, float* topk_w,
                              float* logits_out, flyai_stream_t stream);

/* ---- a3: expert histogram + stable permute -----------------------------------------------------
 * Replaces routing_torch_dist's histc / stable argsort / inverse argsort
 * (transformers/integrations/mxfp4.py:449-457) and the one_hot/where expert loop of
 * GptOssExperts.forward (modeling_gpt_oss.py:93-107).  topk_ids int32 [T*k] in [0,E).
 * hist[E], offsets[E+1] (exclusive scan), perm[T*k] (experts ascending, flat index ascending
 * within an expert), inv[T*k] (inverse).  T*k <= 65536, E <= 256.  An id outside [0,E) (a router row
 * of NaN) is counted as expert 0, so hist sums to T*k and perm / inv stay a permutation and its
 * inverse whatever the ids hold (the expert and combine kernels index with them). */
int flyai_moe_permute(const int32_t* topk_ids, int32_t T, int32_t k, int32_t E, int32_t* hist,
                      int32_t* offsets, int32_t* perm, int32_t* inv, flyai_stream_t stream);

/* a2 + a3 in one call (the stage's path): router logits, then -- for T*k <= 4096 -- top-k of every
 * token and the histogram / permute in a single one-workgroup kernel (separate kernels above that).
 * Same outputs and bit-exact indices as flyai_router_topk_softmax followed by flyai_moe_permute. */
int flyai_moe_route_permute(const uint16_t* x, const uint16_t* w, const uint16_t* b, int32_t T,
                            int32_t H, int32_t E, int32_t k, int32_t* topk_ids, float* topk_w,
                            float* logits, int32_t* hist, int32_t* offsets, int32_t* perm,
                            int32_t* inv, flyai_stream_t stream);

/* ---- a4: unpermute / combine -------------------------------------------------------------------
 * Replaces the weighted index_add_ of GptOssExperts.forward (modeling_gpt_oss.py:108-113) / the
 * gammas scatter of matmul_ogs (transformers/integrations/mxfp4.py:394-403) and the residual add
 * (modeling_gpt_oss.py:375).  out[t] = bf16(sum_s topk_w[t,s] * y_perm[inv[t*k+s]]) in fp32, slot
 * order; when residual is non-NULL, out[t] = bf16(residual[t] + that) (residual may equal out). */
int flyai_moe_combine(const float* y_perm, const int32_t* inv, const float* topk_w, int32_t T,
                      int32_t k, int32_t H, const uint16_t* residual, uint16_t* out,
                      flyai_stream_t stream);

/* ---- a5: MXFP4 weight format -------------------------------------------------------------------
 * The HF/GPT-OSS checkpoint layout (Mxfp4GptOssExperts, transformers/integrations/mxfp4.py:349-365;
 * checked by phase0/mxfp4_guard.py:223-276): blocks u8 [E, N, K/32, 16] (E2M1 pairs, low nibble =
 * even element), scales u8 [E, N, K/32] (E8M0).  The expert kernels read a one-time re-packed
 * tile layout with identical values: flyai_mxfp4_repack converts on the device (N % 16 == 0,
 * K % 32 == 0).  flyai_mxfp4_packed_bytes gives the packed size for all E experts. */
size_t flyai_mxfp4_packed_bytes(int32_t E, int32_t N, int32_t K);
int flyai_mxfp4_repack(const uint8_t* blocks, const uint8_t* scales, int32_t E, int32_t N,
                       int32_t K, uint8_t* packed, flyai_stream_t stream);

/* ---- a6: MXFP4 expert FFN (GPT-OSS SwiGLU) -------------------------------------------------------
 * Replaces Mxfp4GptOssExperts.forward's two matmul_ogs calls (transformers/integrations/
 * mxfp4.py:372-403) and GptOssExperts.forward/_apply_gate (modeling_gpt_oss.py:82-88, :108-111).
 * gate_up: for permuted row p of expert e (offsets[e] <= p < offsets[e+1]), token t = perm[p]/k:
 *   gu = x[t] . W13[e]^T + b13[e] (fp32), rows 2j/2j+1 = gate/up of unit j,
 *   h[p, j] = bf16((clamp(up,-7,7)+1) * min(gate,7) * sigmoid(1.702*min(gate,7))).
 * down: y_perm[p] = h[p] . W2[e]^T + b2[e] (fp32).
 * x bf16 [T,H]; w13_packed/w2_packed from flyai_mxfp4_repack; b13 fp32 [E,2I]; b2 fp32 [E,H];
 * h bf16 [T*k, I]; y_perm fp32 [T*k, H] (rows = T*k).  Groups of any row count are handled, with
 * MFMA on tiles dequantised in registers: decode-sized groups stream the expert's weights once per
 * 8 rows; when the batch averages at least 8 rows per expert, groups of more than 8 rows take the
 * dense kernel (96 rows per weight pass). */
int flyai_moe_gate_up_mxfp4(const uint16_t* x, const int32_t* perm, const int32_t* offsets,
                            int32_t T, int32_t k, const uint8_t* w13_packed, const float* b13,
                            int32_t E, int32_t H, int32_t I, uint16_t* h, flyai_stream_t stream);
int flyai_moe_down_mxfp4(const uint16_t* h, const int32_t* offsets, int32_t rows,
                         const uint8_t* w2_packed, const float* b2, int32_t E, int32_t H, int32_t I,
                         float* y_perm, flyai_stream_t stream);

/* ---- a6, dense groups on the scaled MFMA (fp8 activations x MXFP4 weights) -----------------------
 * The dense-group path of flyai_moe_gate_up_mxfp4 / flyai_moe_down_mxfp4 with the activation operand in
 * fp8: groups the bf16 entry points give the dense tiled GEMM run v_mfma_scale_f32_16x16x128_f8f6f4 on
 * fp8 e4m3 activations and the packed E2M1 weights, each with its E8M0 per-32 scales applied inside the
 * MFMA (the reference's fp8-activation x fp4-weight GEMM, vendor/deepseek_v4_ref/inference/kernel.py:
 * 441-449, with the activations on 32-blocks); decode-sized groups take the bf16 row-pass kernel on x
 * (h) as before.  Each activation row is carried as two e4m3 terms, so the products keep the bf16
 * operand's 8 significant bits: flyai_mx_act_quant quantises bf16 rows x [M, K] (K % 32 == 0) into
 * q [2M, K] and scale rows s_e8m0 [2M] (flyai_mx_act_scale_bytes(2M, K) bytes).  Row r is the high term:
 * per 32-block s1 = 2^ceil(log2(max(amax, 1e-4) / 448)), q1 = e4m3 RNE of clamp(x / s1, -448, 448);
 * row M + r is the low term, the same rule on the exact residual x - s1 q1.  Scale bytes are stored per
 * row as 16 * ceil(ceil(K/128)/4) bytes in MFMA order: byte 4 * (4 * kg4 + g) + i holds the scale of
 * block 4 * (4 * kg4 + i) + g, 127 past K.  gate_up reads x (bf16) and xq/xs = flyai_mx_act_quant(x)
 * for the same T rows (2T rows of xq and xs); down reads h and hq/hs = flyai_mx_act_quant(h) (2 * rows).
 * Each dense product is the sum of the two terms' products in fp32, so results match the bf16 path to
 * fp32 accumulation order, not bit for bit. */
size_t flyai_mx_act_scale_bytes(int32_t M, int32_t K);
int flyai_mx_act_quant(const uint16_t* x, int32_t M, int32_t K, uint8_t* q, uint8_t* s_e8m0,
                       flyai_stream_t stream);
int flyai_moe_gate_up_mxfp4_fp8act(const uint16_t* x, const uint8_t* xq, const uint8_t* xs,
                                   const int32_t* perm, const int32_t* offsets, int32_t T, int32_t k,
                                   const uint8_t* w13_packed, const float* b13, int32_t E, int32_t H,
                                   int32_t I, uint16_t* h, flyai_stream_t stream);
int flyai_moe_down_mxfp4_fp8act(const uint16_t* h, const uint8_t* hq, const uint8_t* hs,
                                const int32_t* offsets, int32_t rows, const uint8_t* w2_packed,
                                const float* b2, int32_t E, int32_t H, int32_t I, float* y_perm,
                                flyai_stream_t stream);

/* ---- a2 (DeepSeek-V3 shape): grouped sigmoid router ---------------------------------------------
 * Replaces KimiMoEGate.forward (vendor/kimi_k3_ref/modeling_kimi_linear.py:703-759) / the V4 Gate
 * (vendor/deepseek_v4_ref/inference/model.py:560-589) for score_func sigmoid with group limits.
 * logits (fp32 [T,E], written) = the fixed-order fp32 dot of x and w (no bias); scores =
 * sigmoid(logits); choice = scores + e_bias (e_bias fp32 [E], may be NULL); the topk_group groups
 * with the largest top-2 sums stay (ties -> lower group); the k largest choices among them are
 * selected (ties -> lower id); topk_ids ascending; topk_w = score / (sum + 1e-20) * route_scale.
 * Indices are bit-exact against the oracle (deterministic sigmoid, fixed summation orders).
 * E % 4 == 0, E <= 256, E / n_group = 4 * 2^j, k in {4, 6, 8}, H % 8 == 0, H <= 7168. */
int flyai_router_grouped_sigmoid(const uint16_t* x, const uint16_t* w, const float* e_bias,
                                 int32_t T, int32_t H, int32_t E, int32_t n_group,
                                 int32_t topk_group, int32_t k, float route_scale, float* logits,
                                 int32_t* topk_ids, float* topk_w, flyai_stream_t stream);

/* ---- a7: FP8 e4m3 128x128 block-scaled experts (DeepSeek-V3 shape) ------------------------------
 * act_quant replaces act_quant (vendor/deepseek_v4_ref/inference/kernel.py:42-80 with power-of-two
 * scales; engines/deepseek_v4/v4_kernels_cpu.py:89-104): per row per 128-K block,
 * s = 2^ceil(log2(max(amax, 1e-4) / 448)) stored as its E8M0 byte (s_e8m0 u8 [M, K/128]) and
 * q = e4m3 RNE of clamp(x / s, -448, 448) (q u8 [M, K]).
 * Weights: e4m3 bytes w [E][N][K] with E8M0 block scales [E][ceil(N/128)][K/128]
 * (model.py:143-149).  flyai_fp8_repack converts them once into the kernels' tile layout; with
 * w3/s3 given (gate_up), the packed N is 2N with w1/w3 rows interleaved.  K % 1024 == 0, K <= 8192.
 * gate_up replaces Expert.forward up to w2 (model.py:601-610) for every routed row of every expert:
 *   row p of expert e takes token perm[p] / k (perm NULL: token p); gate = bf16(x . W1[e]),
 *   up = bf16(x . W3[e]) (fp8_gemm semantics, kernel.py:241-254); h[p] = bf16(silu(gate) * up *
 *   topk_w[perm[p]]) (topk_w NULL: weight 1) -- h bf16 [P, I].
 * down: y[p] = bf16(hq[p] . W2[e]) with hq/hs = act_quant(h) -- y bf16 [P, H].
 * Shared expert (model.py:632, :648): with n_shared > 0 the packed buffers hold E+1 experts, the
 * last being the shared one; its rows P .. P+n_shared-1 (P = offsets[E]) take tokens 0 ..
 * n_shared-1 with weight 1, so h and y have P + n_shared rows and one launch serves both.
 * combine_sum replaces MoE.forward's accumulation (model.py:640-650): out[t] = bf16(sum over slots
 * in order of y[inv[t*k+s]] + shared[t]) in fp32, then out = bf16(residual + out) when residual is
 * given (shared and residual may be NULL; residual may equal out). */
int flyai_fp8_act_quant(const uint16_t* x, int32_t M, int32_t K, uint8_t* q, uint8_t* s_e8m0,
                        flyai_stream_t stream);
size_t flyai_fp8_packed_bytes(int32_t E, int32_t N, int32_t K);
int flyai_fp8_repack(const uint8_t* w1, const uint8_t* s1, const uint8_t* w3, const uint8_t* s3,
                     int32_t E, int32_t N, int32_t K, uint8_t* packed, flyai_stream_t stream);
int flyai_moe_gate_up_fp8(const uint8_t* xq, const uint8_t* xs, const int32_t* perm,
                          const int32_t* offsets, int32_t k, const float* topk_w,
                          const uint8_t* w13_packed, int32_t E, int32_t H, int32_t I,
                          int32_t n_shared, uint16_t* h, flyai_stream_t stream);
int flyai_moe_down_fp8(const uint8_t* hq, const uint8_t* hs, const int32_t* offsets,
                       const uint8_t* w2_packed, int32_t E, int32_t H, int32_t I, int32_t n_shared,
                       uint16_t* y, flyai_stream_t stream);
int flyai_moe_combine_sum(const uint16_t* y_perm, const int32_t* inv, int32_t T, int32_t k,
                          int32_t H, const uint16_t* shared, const uint16_t* residual,
                          uint16_t* out, flyai_stream_t stream);

/* ---- a9: layer glue ------------------------------------------------------------------------------
 * RMSNorm: GptOssRMSNorm.forward (modeling_gpt_oss.py:57-62): y = bf16(w * (x * rsqrt(mean(x^2)+eps)))
 * with fp32 weight.  Linear: q/k/v/o projections (modeling_gpt_oss.py:280-291): y = bf16(x W^T + b),
 * W bf16 [N,K]; with residual non-NULL the result is bf16(residual + y) written to residual
 * (the residual add of modeling_gpt_oss.py:369); the product is a split-K GEMM whose fp32 partial
 * sums (flyai_linear_workspace_bytes) are added in a fixed order by a finalize kernel.  RoPE + KV append: GPT-OSS half-split rotary
 * (modeling_gpt_oss.py:215-232) with per-op bf16 rounding, then the K/V write at each token's
 * position (StaticKV.update, phase0/fastverify.py:71-77; BatchedStaticKV.update,
 * phase0/batchverify.py:42-48).  KV pool layout per sequence slab (element offset kv_base[b]):
 * per kv head a region of kv_cap[b] x 64 elements (D must be 64) in 64-key blocks of 4096 elements in
 * the attention kernel's MFMA-fragment order: K block [kt 4][step 2][lane 64][8], lane 16gd+n holding
 * key 32(kt/2) + 8(n/4) + 4(kt%2) + n%4 and dims 32step+8gd..+7; V block [h 2][dt 4][lane 64][8], lane
 * 16gk+n holding dim 16dt+n and keys 32h+8gk..+7 (flyai_amd/kvlayout.py restates it).  cos_tab/sin_tab bf16
 * [rope_positions][D/2]; a token whose position is outside the table or its slab is skipped.  kv_base and
 * kv_cap are device arrays here, so these standalone kernels cannot check a slab against its pool: the
 * caller keeps every slab inside its pools (flyai_stage_forward checks this on the host). */
int flyai_rmsnorm(const uint16_t* x, const float* w, int32_t T, int32_t H, float eps, uint16_t* y,
                  flyai_stream_t stream);
size_t flyai_linear_workspace_bytes(int32_t M, int32_t N, int32_t K);
int flyai_linear_bf16(const uint16_t* x, const uint16_t* w, const uint16_t* b, int32_t M, int32_t N,
                      int32_t K, uint16_t* y, uint16_t* residual, float* workspace,
                      flyai_stream_t stream);
/* flyai_linear_bf16 without allocation.  No counterpart in the reference: it is for callers that cannot
 * allocate device memory or pass a workspace (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  Same arguments and results minus the workspace, same kernels and
 * bits: the fp32 partials live in a static device array of flyai_linear_noalloc_max_bytes() = 16 MiB
 * that every GPU the library runs on holds until the process ends.  A shape whose partials exceed it
 * -> FLYAI_EINVAL before any launch (partials = 4*M*N bytes, times ceil(ceil(K/128)/4) planes below 256
 * rows; one plane from 256 rows).  The first call on a device resolves the array's address there.
 * Every call on one GPU shares that array and it keeps the last call's contents: calls that overlap on
 * one GPU (other streams or threads) race, so the caller serialises them. */
size_t flyai_linear_noalloc_max_bytes(void);
int flyai_linear_bf16_noalloc(const uint16_t* x, const uint16_t* w, const uint16_t* b, int32_t M, int32_t N,
                              int32_t K, uint16_t* y, uint16_t* residual, flyai_stream_t stream);
int flyai_rope_kv_append(const uint16_t* qkv, const int32_t* positions, const int32_t* seq_id,
                         const uint16_t* cos_tab, const uint16_t* sin_tab, int32_t rope_positions,
                         int32_t T, int32_t Hq, int32_t Hkv, int32_t D, const int64_t* kv_base,
                         const int32_t* kv_cap, uint16_t* q_out, uint16_t* k_pool,
                         uint16_t* v_pool, flyai_stream_t stream);

/* ---- a8: ragged GQA attention with sinks and sliding window -------------------------------------
 * Replaces eager_attention_forward (modeling_gpt_oss.py:235-263) over the additive masks of
 * phase0/pipeline.py:38-48 / phase0/batchverify.py:51-61 and the bucketed StaticKV reads
 * (phase0/fastverify.py:52-77).  Query token i of sequence b (position p = starts[b]+i) attends
 * keys j in [lo, p], lo = 0 or max(0, p-window+1); logits scaled by D^-0.5; the per-head sink
 * logit joins the softmax denominator only.  q bf16 [T,Hq,D] (rotated); out bf16 [T,Hq,D].
 * KV slabs in the tiled layout above (flyai_rope_kv_append); every K or V load instruction of a wave
 * reads one contiguous KiB.
 * Work is split over (sequence, kv head, group of <= 4 query tokens, key split); the host-side
 * plan (flyai_attn_plan) is copied to the device by the caller.  The plan lists groups of <= 2
 * tokens first (n_items_small items, run by a one-tile kernel variant), then the rest.  D == 64,
 * Hq/Hkv == 8, kv_cap[b] % 64 == 0, kv_base[b] % 8 == 0, starts[b] + q_lens[b] <= kv_cap[b], and every
 * slab inside its pools (device arrays: not checked here; flyai_stage_forward checks them).
 * Partials scratch: flyai_attn_partials_bytes(n_items). */
typedef struct {
  int32_t seq;      /* sequence index b */
  int32_t kv_head;  /* g */
  int32_t tok;      /* flat token index of the item's first query token */
  int32_t ntok;     /* query tokens in the item (1..4) */
  int32_t pos0;     /* position of the first query token */
  int32_t key_lo;   /* key range [key_lo, key_hi) of this split */
  int32_t key_hi;
  int32_t group;    /* query group index (items of one group are consecutive) */
} flyai_attn_item;

typedef struct {
  int32_t first_item; /* index of the group's first split item */
  int32_t n_splits;
  int32_t tok;        /* flat token index of the first query token */
  int32_t ntok;
  int32_t kv_head;
  int32_t pad[3];
} flyai_attn_group;

int flyai_attn_plan(const int32_t* q_lens_host, const int32_t* starts_host, int32_t n_seqs,
                    int32_t Hkv, int32_t window, int32_t split_keys, flyai_attn_item* items_host,
                    int32_t max_items, flyai_attn_group* groups_host, int32_t max_groups,
                    int32_t* n_items, int32_t* n_groups, int32_t* n_items_small);
size_t flyai_attn_partials_bytes(int32_t n_items);
int flyai_attn_ragged(const uint16_t* q, const uint16_t* k_pool, const uint16_t* v_pool,
                      const int64_t* kv_base, const int32_t* kv_cap, const float* sinks,
                      int32_t window, int32_t Hq, int32_t Hkv, int32_t D,
                      const flyai_attn_item* items_dev, int32_t n_items, int32_t n_items_small,
                      const flyai_attn_group* groups_dev, int32_t n_groups, float* partials,
                      uint16_t* out, flyai_stream_t stream);

/* Chunked-prefill rows (chunked-prefill attention on device, replacing the flex prefill of
 * phase0/fastverify.py:138-155).  flyai_attn_plan_prefill is flyai_attn_plan with every
 * sequence of q_len >= prefill_min (0: none) moved to prefill items instead: 16 consecutive query tokens
 * x one kv head per item (ntok <= 16, key range [key_lo, key_hi) = the tiles' window start .. last
 * position + 1, group -1), the chunk's last tiles first.  flyai_attn_prefill runs them: a workgroup of
 * 4 waves per item shares each 64-key K/V block through LDS and writes the final rows of `out` (sink
 * and normalisation included; no partials).  Same math, masks and layout as flyai_attn_ragged. */
int flyai_attn_plan_prefill(const int32_t* q_lens_host, const int32_t* starts_host, int32_t n_seqs,
                            int32_t Hkv, int32_t window, int32_t split_keys, int32_t prefill_min,
                            flyai_attn_item* items_host, int32_t max_items, flyai_attn_group* groups_host,
                            int32_t max_groups, flyai_attn_item* pitems_host, int32_t max_pitems,
                            int32_t* n_items, int32_t* n_groups, int32_t* n_items_small, int32_t* n_pitems);
int flyai_attn_prefill(const uint16_t* q, const uint16_t* k_pool, const uint16_t* v_pool,
                       const int64_t* kv_base, const int32_t* kv_cap, const float* sinks, int32_t window,
                       int32_t Hq, int32_t Hkv, int32_t D, const flyai_attn_item* pitems_dev, int32_t n_pitems,
                       uint16_t* out, flyai_stream_t stream);

/* ---- head and tail of a served model (the continuous-batch backend's token step) --------------
 * Embedding: replaces parts["embed"](token_ids) (phase0/specpipe.py:595-596, :779): out[t] =
 * table[ids[t]] (bf16 [V, H] table; an id outside [0, V) gives a zero row).  H % 8 == 0.
 * lm_head + greedy pick: replaces lm_head(norm(h)).argmax(-1) (phase0/specpipe.py:796-800; the
 * greedy branches of Sampler.sample_logits / accept, phase0/specsample.py:78-100).  x holds the
 * final-normed hidden rows (flyai_rmsnorm); rows (device, nullable) selects n_rows <= 64 of them
 * (NULL: rows 0..n_rows-1), e.g. only the last token of a prefill chunk (specpipe.py:794-795).
 * logits[r][v] = bf16(fp32 dot(x[rows[r]], W[v])) (MFMA accumulation); ids[r] = the first v of
 * maximal logit (torch.argmax semantics).  logits_out (nullable, bf16 [n_rows, V]) receives the
 * logits.  W is re-packed once by flyai_bf16_tile_repack from the nn.Linear layout [V, H]
 * (V % 16 == 0, H % 32 == 0; flyai_bf16_tile_packed_bytes(V, H) bytes).  workspace:
 * flyai_lm_head_workspace_bytes(n_rows, V). */
size_t flyai_bf16_tile_packed_bytes(int32_t N, int32_t K);
int flyai_bf16_tile_repack(const uint16_t* w, int32_t N, int32_t K, uint8_t* packed, flyai_stream_t stream);
int flyai_embed_gather(const uint16_t* table, const int32_t* ids, int32_t T, int32_t H, int32_t V,
                       uint16_t* out, flyai_stream_t stream);
size_t flyai_lm_head_workspace_bytes(int32_t n_rows, int32_t V);
int flyai_lm_head_argmax(const uint16_t* x, const int32_t* rows, int32_t n_rows, int32_t H,
                         const uint8_t* w_packed, int32_t V, int32_t* ids, uint16_t* logits_out,
                         void* workspace, flyai_stream_t stream);

/* ---- measurement -------------------------------------------------------------------------------
 * HBM read-streaming probe (no counterpart in the reference: it measures the bandwidth ceiling the
 * weight-streaming kernels are held against).  Reads every byte of src once, 16 bytes per lane per
 * load: `grid` workgroups of 256 take contiguous 32 KiB chunks round-robin, 8 loads in flight per
 * thread; nontemporal selects nontemporal loads.  sink (device, 4 bytes) is written only in a 1-in-2^32 case.  bytes % 16
 * == 0, src 16-byte aligned, grid in [1, 65536]. */
int flyai_hbm_read_probe(const void* src, size_t bytes, int32_t nontemporal, int32_t grid, uint32_t* sink,
                         flyai_stream_t stream);

/* ---- token sampling (the tail's Sampler: phase0/specsample.py:36-107) -------------------------------
 * Per logits row x[V] (bf16, R rows, one workgroup each): z = x / max(temp, 1e-6) in fp32; top-k
 * (0 < top_k < V) keeps z >= the k-th largest z; weights w = floor(2^40 e^(z - max z)) as exact integers
 * (a fixed fp64 exp); top-p (0 < top_p < 1) keeps, in (z desc, id asc) order, each token whose preceding
 * weight is <= floor(top_p * W); the distribution is w / W over what is kept.  Outputs (each nullable):
 * p_draft[r] = the kept probability of token draft[r] (draft nullable; each in [-1, V), -1 = none: an id
 * outside that range is read as none); probs [R, V] fp32 the
 * distribution; draw[r] = the first id (ascending) whose inclusive prefix of w exceeds floor(u[r] * W'')
 * where w has the drafted token removed (the speculative-sampling residual) -- the first id of maximal w
 * when nothing is left, and id 0 when every weight is 0 (a row with a NaN or infinite logit); a sampled
 * draw needs u (fp64 in [0, 1); a u below 0 draws as 0 and one at or above 1 as just below 1).  temp <= 0
 * is greedy: draw is the first id of maximal x (u unused) and p_draft is 1 for that id, else 0.  Logits
 * should be finite.  Sums are integer, so results do not depend on the launch. */
int flyai_sample_rows(const uint16_t* logits, int32_t R, int32_t V, float temp, int32_t top_k, float top_p,
                      const int32_t* draft, const double* u, float* p_draft, int32_t* draw, float* probs,
                      flyai_stream_t stream);
/* A draw from a probability vector p[V] (fp32, device; Sampler.sample): weights floor(p * 2^40), then the
 * same inverse-CDF rule with uniform u in [0, 1); out (device int32) gets the id (0 when all are 0). */
int flyai_sample_probs(const float* probs, int32_t V, double u, int32_t* out, flyai_stream_t stream);

/* ---- a10: stage step driver ----------------------------------------------------------------------
 * The per-layer loop of FastVerify._layers / BatchedFastVerify._layers (phase0/fastverify.py:116-122,
 * phase0/batchverify.py:132-138) over GptOssDecoderLayer.forward (modeling_gpt_oss.py:347-376), for
 * a ragged batch of decode / verify / prefill-chunk rows.  Weights and KV pools are caller-owned
 * device memory bound once per layer; the step itself only launches kernels on `stream`. */
typedef struct {
  int32_t n_layers, hidden, n_q_heads, n_kv_heads, head_dim;
  int32_t n_experts, top_k, intermediate, window;
  int32_t max_tokens, max_seqs, max_attn_items, rope_positions, attn_split_keys;
  float rms_eps;
  int32_t attn_prefill_min;   /* sequences with q_len >= this take the prefill attention items (0: never) */
  int32_t moe_dense_fp8;      /* 1: dense expert groups take the fp8-activation scaled-MFMA path
                                 (flyai_moe_gate_up_mxfp4_fp8act); 0: the bf16 dense kernel */
} flyai_stage_config;

typedef struct {
  const float* ln1;           /* fp32 [H] */
  const float* ln2;           /* fp32 [H] */
  const uint16_t* wqkv;       /* bf16 [(Hq+2Hkv)*D, H]: q_proj, k_proj, v_proj stacked */
  const uint16_t* bqkv;       /* bf16 [(Hq+2Hkv)*D] */
  const uint16_t* wo;         /* bf16 [H, Hq*D] */
  const uint16_t* bo;         /* bf16 [H] */
  const float* sinks;         /* fp32 [Hq] (bf16-valued) */
  const uint16_t* router_w;   /* bf16 [E, H] */
  const uint16_t* router_b;   /* bf16 [E] */
  const uint8_t* w13_packed;  /* flyai_mxfp4_repack of gate_up blocks/scales */
  const float* b13;           /* fp32 [E, 2I] */
  const uint8_t* w2_packed;   /* flyai_mxfp4_repack of down blocks/scales */
  const float* b2;            /* fp32 [E, H] */
  uint16_t* k_pool;           /* this layer's K pool */
  uint16_t* v_pool;           /* this layer's V pool (tiled slabs, same size as k_pool) */
  int32_t sliding;            /* 1: sliding-window layer */
  int32_t pad;
  int64_t kv_pool_elems;      /* bf16 elements of k_pool and of v_pool (each); > 0 */
} flyai_layer_desc;

typedef struct flyai_stage flyai_stage;

/* Rebinding rule: flyai_stage_set_layer, flyai_stage_set_rope and flyai_stage_set_workspace drop every
 * captured step graph (see flyai_stage_set_graphs), because a graph keeps the pointers bound when it was
 * captured; the next step with graphs enabled captures again from the new bindings. */
int flyai_stage_create(const flyai_stage_config* cfg, flyai_stage** out);
void flyai_stage_destroy(flyai_stage* st);
int flyai_stage_set_layer(flyai_stage* st, int32_t layer, const flyai_layer_desc* desc);
int flyai_stage_set_rope(flyai_stage* st, const uint16_t* cos_tab, const uint16_t* sin_tab);
size_t flyai_stage_workspace_bytes(const flyai_stage* st);
size_t flyai_stage_host_staging_bytes(const flyai_stage* st);
/* device workspace (>= workspace_bytes) and pinned host staging (>= host_staging_bytes).  Each step's
 * batch blob goes through one half of the staging; when the staging is mapped into the device's
 * address space (hipHostMalloc / pinned torch memory) a kernel reads it there, otherwise an H2D copy
 * moves it. */
int flyai_stage_set_workspace(flyai_stage* st, void* dev_ws, size_t dev_bytes, void* host_pinned,
                              size_t host_bytes);
/* One step.  Batch description on the host (validated here; ContextOverflow -> FLYAI_ERANGE before
 * any launch): per sequence q_lens, starts, kv_base (element offset of its slab in every layer's
 * pools), kv_cap.  hidden: device bf16 [T, H] in packed token order, updated in place.
 * Slab bounds: sequence b's slab is [kv_base[b], kv_base[b] + n_kv_heads*kv_cap[b]*head_dim) in every
 * layer's pools.  A slab that ends past the smallest bound kv_pool_elems -> FLYAI_ERANGE; two
 * sequences whose slabs overlap (their K/V writes would race) -> FLYAI_EINVAL; both before any launch. */
int flyai_stage_forward(flyai_stage* st, const int32_t* q_lens_host, const int32_t* starts_host,
                        const int64_t* kv_base_host, const int32_t* kv_cap_host, int32_t n_seqs,
                        uint16_t* hidden, flyai_stream_t stream);
/* Tree verify (replaces FastVerify.tree_decode, phase0/fastverify.py:233-299, with the masks of
 * FastVerify._tset, :250-272, and phase0/tree.py:26-46).  One sequence at committed length `start`
 * feeds n_nodes tree nodes (hidden bf16 [n_nodes, H], updated in place).  Node i is rotated at
 * position start + depth[i] and its K/V is written to slot start + i; it attends every committed
 * key j < start (sliding layers: start + depth[i] - j < window) and the slots of its ancestors and
 * itself (sliding layers: depth[i] - depth[a] < window).  parent_host/depth_host follow
 * validate_tree (fastverify.py:29-49): parent[i] in [-1, n), parent[i] != i, depth[i] == 0 for a
 * root and depth[parent[i]] + 1 otherwise (which rules out cycles); FLYAI_EINVAL otherwise, and for
 * n_nodes outside [1, min(max_tokens, FLYAI_TREE_MAX_NODES)].  start + n_nodes past kv_cap or the
 * rope table, or a slab past the pools -> FLYAI_ERANGE before any launch.  Always launched directly
 * (no graph). */
#define FLYAI_TREE_MAX_NODES 2048
/* The tree as the attention kernel reads it (built by flyai_stage_forward_tree in the step's batch
 * blob): this header, then int32 depth[n_nodes] and two visibility masks uint64 [n_nodes][words],
 * one per layer kind; bit j of row i (word j / 64, bit j % 64) lets node i see tree slot start + j.
 * Offsets are in bytes from the header. */
typedef struct {
  int32_t start;       /* committed length: node i's K/V sits at slot start + i */
  int32_t n_nodes;     /* 1 .. min(max_tokens, FLYAI_TREE_MAX_NODES) */
  int32_t words;       /* 64-bit words per mask row: (n_nodes + 63) / 64 */
  int32_t depth_off;   /* int32 depth[n_nodes]: node i is rotated at position start + depth[i] */
  int64_t mask_off[2]; /* [0] full-attention layers (ancestors and self), [1] sliding layers (those
                          of them less than window levels above the node) */
} flyai_attn_tree;

int flyai_stage_forward_tree(flyai_stage* st, int32_t start, int32_t n_nodes,
                             const int32_t* parent_host, const int32_t* depth_host, int64_t kv_base,
                             int32_t kv_cap, uint16_t* hidden, flyai_stream_t stream);
/* HIP-graph replay of flyai_stage_forward (the CUDA-graph capture of FastVerify.decode /
 * BatchedFastVerify.decode, phase0/fastverify.py:221-231, phase0/batchverify.py:180-190).  When
 * enabled, each step's kernels are one graph per (tokens, sequences, attention-plan capacity) key:
 * captured on first use, replayed after, least recently used evicted beyond 16.  The plan
 * capacities round the step's attention item and group counts up to multiples of 64, so steps whose
 * KV grows within that bucket replay the same graph (kernels past the live count exit).  The
 * caller's hidden rows are copied into a stage-owned buffer around the replay.  Off by default. */
int flyai_stage_set_graphs(flyai_stage* st, int32_t enable);
/* Number of graphs captured so far (tests: rebuilt only on a key change). */
int32_t flyai_stage_graphs_captured(const flyai_stage* st);
/* Device pointer of an internal buffer of the last step (for tests): 0 xn, 1 gemm partials, 2 q_rot,
 * 3 attn_out, 4 topk_ids, 5 topk_w, 6 offsets, 7 perm, 8 inv, 9 h_moe, 10 y_perm, 11 positions,
 * 12 seq_id, 13 cu_seqlens. */
void* flyai_stage_debug_buffer(flyai_stage* st, int32_t which);

#ifdef __cplusplus
}
#endif

#endif /* FLYAI_STAGE_H */
