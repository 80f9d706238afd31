// C ABI: error reporting and the stage step driver (per-layer kernel sequence on one stream).
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <new>
#include <string>
#include <vector>

#include "common.h"

namespace flyai {

static thread_local char g_last_error[512] = "";

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(FLYAI_EHIP, "%s: %s", what, hipGetErrorString(e));
  return FLYAI_OK;
}

// launchers defined in the kernel files
int launch_router(const uint16_t*, const uint16_t*, const uint16_t*, int, int, int, int, int32_t*,
                  float*, float*, hipStream_t);
int launch_permute(const int32_t*, int, int, int, int32_t*, int32_t*, int32_t*, int32_t*, hipStream_t);
int launch_route_permute(const uint16_t*, const uint16_t*, const uint16_t*, int, int, int, int, int32_t*,
                         float*, float*, int32_t*, int32_t*, int32_t*, int32_t*, hipStream_t);
int launch_combine(const float*, const int32_t*, const float*, int, int, int, const uint16_t*,
                   uint16_t*, const float*, float, uint16_t*, hipStream_t);
int launch_moe_gate_up(const uint16_t*, const int32_t*, const int32_t*, int, const uint8_t*,
                       const float*, int, int, int, int, uint16_t*, hipStream_t);
int launch_moe_down(const uint16_t*, const int32_t*, const uint8_t*, const float*, int, int, int, int,
                    float*, hipStream_t);
int launch_mx_act_quant(const uint16_t*, int, int, uint8_t*, uint8_t*, hipStream_t);
int launch_moe_gate_up_fp8act(const uint16_t*, const uint8_t*, const uint8_t*, const int32_t*, const int32_t*, int,
                              const uint8_t*, const float*, int, int, int, int, uint16_t*, hipStream_t);
int launch_moe_down_fp8act(const uint16_t*, const uint8_t*, const uint8_t*, const int32_t*, const uint8_t*,
                           const float*, int, int, int, int, float*, hipStream_t);
bool moe_batch_is_dense(int rows_total, int E, int K);
int launch_rmsnorm(const uint16_t*, const float*, int, int, float, uint16_t*, hipStream_t);
int launch_linear_residual_rmsnorm(const uint16_t*, const uint16_t*, const uint16_t*, int, int, int,
                                   uint16_t*, const float*, float, uint16_t*, float*, hipStream_t);
int launch_linear_residual_rmsnorm_logits(const uint16_t*, const uint16_t*, const uint16_t*, int, int,
                                          int, const uint16_t*, uint16_t*, const float*, float, uint16_t*,
                                          float*, const uint16_t*, const uint16_t*, int, float*, hipStream_t);
int launch_topk_permute(const float*, int, int, int, int32_t*, float*, int32_t*, int32_t*, int32_t*,
                        int32_t*, hipStream_t);
int launch_qkv_rope_kv(const uint16_t*, const uint16_t*, const uint16_t*, float*, const int32_t*,
                       const int32_t*, const uint16_t*, const uint16_t*, int, int, int, int, int, int,
                       const int64_t*, const int32_t*, uint16_t*, uint16_t*, uint16_t*, const int32_t*,
                       hipStream_t);
size_t linear_partials_bytes(int M, int N, int K);
int launch_attn(const uint16_t*, const uint16_t*, const uint16_t*, const int64_t*, const int32_t*,
                const float*, int, int, const flyai_attn_item*, int, int, const flyai_attn_group*, int,
                const int32_t*, float*, uint16_t*, const flyai_attn_tree*, bool, hipStream_t);
int attn_plan(const int32_t*, const int32_t*, int, int, int, int, flyai_attn_item*, int,
              flyai_attn_group*, int, int*, int*, int*, int, flyai_attn_item*, int, int*);
int launch_attn_prefill(const uint16_t*, const uint16_t*, const uint16_t*, const int64_t*, const int32_t*,
                        const float*, int, int, const flyai_attn_item*, int, uint16_t*, hipStream_t);
int launch_attn_step(const uint16_t*, const uint16_t*, const uint16_t*, const int64_t*, const int32_t*,
                     const float*, int, int, const flyai_attn_item*, int, const flyai_attn_group*, int,
                     const int32_t*, float*, const flyai_attn_item*, int, uint16_t*, bool, bool, hipStream_t);
int attn_plan_tree(int, int, const int32_t*, int, int, int, flyai_attn_item*, int, flyai_attn_group*, int,
                   int*, int*, int*);
int launch_pack(const int32_t*, const int32_t*, const int64_t*, const int32_t*, int, int, int, int32_t*,
                int32_t*, int32_t*, int32_t*, int64_t*, int32_t*, const int32_t*, int32_t*, hipStream_t, int,
                const uint16_t*, const float*, int, float, uint16_t*);
int launch_blob_fetch(const char*, char*, size_t, hipStream_t);

}  // namespace flyai

using namespace flyai;

namespace {

size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

struct Carve {
  size_t off = 0;
  size_t take(size_t bytes) {
    const size_t o = off;
    off = align256(off + bytes);
    return o;
  }
};

}  // namespace

struct flyai_stage {
  flyai_stage_config cfg;
  int qkv_width, max_groups, max_pitems, P;
  flyai_layer_desc* layers = nullptr;
  const uint16_t* cos_tab = nullptr;
  const uint16_t* sin_tab = nullptr;
  // device workspace offsets; o_blob holds the per-step batch blob moved from the host staging
  size_t o_blob, blob_max, o_cu, o_pos, o_sid, o_kvlen, o_slot, o_status, o_kvpos;
  size_t o_xn, o_gemm, o_qrot, o_attn, o_parts;
  size_t o_ids, o_w, o_logits, o_hist, o_off, o_perm, o_inv, o_hmoe, o_y;
  size_t o_h2;  // the post-attention residual stream of the decode-sized path
  size_t o_xq, o_xs, o_hq, o_hs;  // fp8 activation operands of the dense groups (moe_dense_fp8)
  size_t o_hidden;  // stage-owned hidden rows the replayed graphs read and update
  size_t dev_bytes = 0;
  size_t host_half = 0;  // bytes of one pinned staging half (== blob_max)
  std::vector<flyai_attn_item> plan_items[2];
  std::vector<flyai_attn_group> plan_groups[2];
  std::vector<flyai_attn_item> plan_pitems[2];
  char* dev = nullptr;
  char* host = nullptr;
  // the staging's address in the device's address space (mapped pinned memory): the blob is then
  // fetched by a kernel; null: the staging is not mapped, and an H2D copy moves it
  const char* host_dev = nullptr;
  hipEvent_t staged[2] = {nullptr, nullptr};
  int half = 0;
  bool events_ready = false;
  // HIP-graph replay of the step (off by default).  One executable graph per key (tokens,
  // sequences, attention plan capacities), captured on first use on a stream of the stage's own
  // (the null stream cannot be captured) and replayed on the caller's stream.
  bool graphs = false;
  hipStream_t capture_stream = nullptr;
  struct Graph {
    int64_t key[12];
    hipGraphExec_t exec;
    uint64_t last_use;
  };
  std::vector<Graph> graph_cache;
  uint64_t use_clock = 0;
  int graphs_captured = 0;
  std::vector<int> slab_order;  // host scratch of the slab-overlap check (max_seqs entries)
  int tree_cap = 0;             // largest tree: min(max_tokens, FLYAI_TREE_MAX_NODES) nodes
  std::vector<char> tree_img;   // host image of a tree step's flyai_attn_tree (header, depths, masks)
  std::vector<int> tree_order;  // host scratch: the nodes in order of depth
};
static constexpr int kGraphCacheMax = 16;
static constexpr int kPlanBucket = 64;  // attention plan capacities round up to this

// Byte layout of a tree of n nodes as flyai_attn_tree describes it: the header, int32 depths, then the
// two masks of n rows of (n + 63) / 64 words, each part at a 64-byte boundary.
static size_t align64(size_t x) { return (x + 63) & ~(size_t)63; }
static void tree_layout(int n, flyai_attn_tree* h) {
  h->n_nodes = n;
  h->words = (n + 63) / 64;
  h->depth_off = (int32_t)align64(sizeof(flyai_attn_tree));
  h->mask_off[0] = (int64_t)align64((size_t)h->depth_off + (size_t)n * 4);
  h->mask_off[1] = h->mask_off[0] + (int64_t)align64((size_t)n * h->words * 8);
}
static size_t tree_bytes(int n) {
  flyai_attn_tree h;
  tree_layout(n, &h);
  return (size_t)h.mask_off[1] + align64((size_t)n * h.words * 8);
}

static size_t blob_bytes(int S, int n_items0, int n_items1, int n_groups0, int n_groups1, int n_pitems,
                         int tree_nodes) {
  return align256(4 * sizeof(int32_t)) + align256((size_t)S * 4) * 3 + align256((size_t)S * 8) +
         align256((size_t)n_items0 * sizeof(flyai_attn_item)) + align256((size_t)n_items1 * sizeof(flyai_attn_item)) +
         align256((size_t)n_groups0 * sizeof(flyai_attn_group)) + align256((size_t)n_groups1 * sizeof(flyai_attn_group)) +
         2 * align256((size_t)n_pitems * sizeof(flyai_attn_item)) + align256(tree_bytes(tree_nodes));
}

static void layout(flyai_stage* st) {
  const flyai_stage_config& c = st->cfg;
  const size_t S = c.max_seqs, T = c.max_tokens, P = (size_t)T * c.top_k;
  st->blob_max = blob_bytes(c.max_seqs, c.max_attn_items, c.max_attn_items, st->max_groups, st->max_groups,
                            st->max_pitems, st->tree_cap);
  Carve d;
  st->o_blob = d.take(st->blob_max);
  st->o_cu = d.take((S + 1) * 4);
  st->o_pos = d.take(T * 4);
  st->o_sid = d.take(T * 4);
  st->o_kvlen = d.take(S * 4);
  st->o_slot = d.take(T * 8);
  st->o_status = d.take(4);
  st->o_kvpos = d.take(T * 4);
  st->o_xn = d.take(T * c.hidden * 2);
  {
    const size_t a = linear_partials_bytes(c.max_tokens, st->qkv_width, c.hidden);
    const size_t b = linear_partials_bytes(c.max_tokens, c.hidden, c.n_q_heads * c.head_dim);
    st->o_gemm = d.take(a > b ? a : b);
  }
  st->o_qrot = d.take(T * c.n_q_heads * c.head_dim * 2);
  st->o_attn = d.take(T * c.n_q_heads * c.head_dim * 2);
  st->o_parts = d.take(flyai_attn_partials_bytes(c.max_attn_items));
  st->o_ids = d.take(P * 4);
  st->o_w = d.take(P * 4);
  st->o_logits = d.take(T * (size_t)c.n_experts * 4);
  st->o_hist = d.take((size_t)c.n_experts * 4);
  st->o_off = d.take(((size_t)c.n_experts + 1) * 4);
  st->o_perm = d.take(P * 4);
  st->o_inv = d.take(P * 4);
  st->o_hmoe = d.take(P * c.intermediate * 2);
  st->o_y = d.take(P * c.hidden * 4);
  st->o_h2 = d.take(T * c.hidden * 2);
  st->o_hidden = d.take(T * c.hidden * 2);
  if (c.moe_dense_fp8) {
    // two e4m3 terms per row (high, then low): 2 rows of bytes and scales per activation row
    st->o_xq = d.take(2 * T * c.hidden);
    st->o_xs = d.take(flyai_mx_act_scale_bytes(2 * c.max_tokens, c.hidden));
    st->o_hq = d.take(2 * P * c.intermediate);
    st->o_hs = d.take(flyai_mx_act_scale_bytes((int32_t)(2 * P), c.intermediate));
  }
  st->dev_bytes = d.off;
  st->host_half = st->blob_max;
}

extern "C" const char* flyai_last_error(void) { return g_last_error; }
extern "C" int flyai_abi_version(void) { return FLYAI_ABI_VERSION; }

extern "C" int flyai_stage_create(const flyai_stage_config* cfg, flyai_stage** out) {
  FLYAI_REQUIRE(cfg && out, "stage_create: null pointer");
  const flyai_stage_config& c = *cfg;
  FLYAI_REQUIRE(c.n_layers > 0 && c.hidden > 0 && c.hidden % 64 == 0 && c.hidden <= 7168,
                "stage: hidden must be a multiple of 64, at most 7168");
  FLYAI_REQUIRE(c.head_dim == 64 && c.n_kv_heads > 0 && c.n_q_heads == 8 * c.n_kv_heads,
                "stage: attention kernel needs head_dim 64 and 8 query heads per kv head");
  FLYAI_REQUIRE(c.n_experts >= 4 && c.n_experts <= 256 && c.n_experts % 4 == 0 &&
                    (c.top_k == 2 || c.top_k == 4 || c.top_k == 8),
                "stage: need n_experts %% 4 == 0 in [4, 256] and top_k in {2, 4, 8}");
  FLYAI_REQUIRE(c.intermediate > 0 && c.intermediate % 32 == 0 && c.hidden % 32 == 0,
                "stage: MXFP4 needs hidden and intermediate multiples of 32");
  FLYAI_REQUIRE(c.max_tokens > 0 && (int64_t)c.max_tokens * c.top_k <= 65536, "stage: max_tokens*top_k <= 65536");
  FLYAI_REQUIRE(c.max_seqs > 0 && c.max_seqs <= 8192, "stage: max_seqs in [1, 8192]");
  FLYAI_REQUIRE(c.max_attn_items > 0 && c.rope_positions > 0, "stage: bad capacities");
  FLYAI_REQUIRE(c.attn_split_keys >= 64 && c.attn_split_keys % 64 == 0, "stage: attn_split_keys % 64");
  FLYAI_REQUIRE(c.attn_prefill_min >= 0, "stage: attn_prefill_min must be >= 0");
  FLYAI_REQUIRE(c.moe_dense_fp8 == 0 || c.moe_dense_fp8 == 1, "stage: moe_dense_fp8 must be 0 or 1");
  flyai_stage* st = new (std::nothrow) flyai_stage();
  if (!st) return set_error(FLYAI_EINVAL, "stage_create: out of host memory");
  st->cfg = c;
  st->qkv_width = (c.n_q_heads + 2 * c.n_kv_heads) * c.head_dim;
  st->max_groups = (c.max_seqs + (c.max_tokens + 3) / 4) * c.n_kv_heads;
  st->max_pitems = c.attn_prefill_min > 0 ? (c.max_seqs + (c.max_tokens + kPrefillTokens - 1) / kPrefillTokens) * c.n_kv_heads : 0;
  st->tree_cap = std::min(c.max_tokens, FLYAI_TREE_MAX_NODES);
  st->layers = new (std::nothrow) flyai_layer_desc[c.n_layers];
  if (!st->layers) { delete st; return set_error(FLYAI_EINVAL, "stage_create: out of host memory"); }
  memset(st->layers, 0, sizeof(flyai_layer_desc) * c.n_layers);
  try {
    st->slab_order.resize(c.max_seqs);
    st->tree_order.resize(2 * (size_t)st->tree_cap + 1);
    for (int i = 0; i < 2; ++i) {
      st->plan_items[i].resize(c.max_attn_items);
      st->plan_groups[i].resize(st->max_groups);
      st->plan_pitems[i].resize(st->max_pitems > 0 ? st->max_pitems : 1);
    }
  } catch (...) {
    delete[] st->layers;
    delete st;
    return set_error(FLYAI_EINVAL, "stage_create: out of host memory for the attention plan");
  }
  layout(st);
  *out = st;
  return FLYAI_OK;
}

// A captured graph keeps the workspace, weight, pool and rope pointers bound when it was captured:
// every setter that rebinds one of them drops the cache, and the next step captures again.
static void drop_graphs(flyai_stage* st) {
  for (auto& g : st->graph_cache) hipGraphExecDestroy(g.exec);
  st->graph_cache.clear();
}

extern "C" void flyai_stage_destroy(flyai_stage* st) {
  if (!st) return;
  drop_graphs(st);
  if (st->capture_stream) hipStreamDestroy(st->capture_stream);
  for (int i = 0; i < 2; ++i)
    if (st->staged[i]) hipEventDestroy(st->staged[i]);
  delete[] st->layers;
  delete st;
}

extern "C" int flyai_stage_set_layer(flyai_stage* st, int32_t layer, const flyai_layer_desc* d) {
  FLYAI_REQUIRE(st && d, "set_layer: null pointer");
  FLYAI_REQUIRE(layer >= 0 && layer < st->cfg.n_layers, "set_layer: layer %d out of range", layer);
  FLYAI_REQUIRE(d->ln1 && d->ln2 && d->wqkv && d->wo && d->sinks && d->router_w && d->router_b &&
                    d->w13_packed && d->b13 && d->w2_packed && d->b2 && d->k_pool && d->v_pool,
                "set_layer: null weight pointer");
  FLYAI_REQUIRE(d->kv_pool_elems > 0, "set_layer: kv_pool_elems must be > 0");
  drop_graphs(st);
  st->layers[layer] = *d;
  return FLYAI_OK;
}

extern "C" int flyai_stage_set_rope(flyai_stage* st, const uint16_t* cos_tab, const uint16_t* sin_tab) {
  FLYAI_REQUIRE(st && cos_tab && sin_tab, "set_rope: null pointer");
  drop_graphs(st);
  st->cos_tab = cos_tab;
  st->sin_tab = sin_tab;
  return FLYAI_OK;
}

extern "C" size_t flyai_stage_workspace_bytes(const flyai_stage* st) { return st ? st->dev_bytes : 0; }
extern "C" size_t flyai_stage_host_staging_bytes(const flyai_stage* st) {
  return st ? 2 * st->host_half : 0;
}

extern "C" int flyai_stage_set_workspace(flyai_stage* st, void* dev_ws, size_t dev_bytes,
                                         void* host_pinned, size_t host_bytes) {
  FLYAI_REQUIRE(st && dev_ws && host_pinned, "set_workspace: null pointer");
  FLYAI_REQUIRE(dev_bytes >= st->dev_bytes && host_bytes >= 2 * st->host_half,
                "set_workspace: need %zu device and %zu pinned host bytes", st->dev_bytes,
                2 * st->host_half);
  FLYAI_REQUIRE(((uintptr_t)dev_ws & 255) == 0, "set_workspace: device workspace must be 256-byte aligned");
  drop_graphs(st);
  st->dev = static_cast<char*>(dev_ws);
  st->host = static_cast<char*>(host_pinned);
  void* mapped = nullptr;
  if (hipHostGetDevicePointer(&mapped, host_pinned, 0) == hipSuccess && mapped) {
    st->host_dev = static_cast<const char*>(mapped);
  } else {
    st->host_dev = nullptr;
    (void)hipGetLastError();  // not mapped: the H2D copy path, and no error left behind
  }
  if (!st->events_ready) {
    for (int i = 0; i < 2; ++i) {
      const hipError_t e = hipEventCreateWithFlags(&st->staged[i], hipEventDisableTiming);
      if (e != hipSuccess) return set_error(FLYAI_EHIP, "hipEventCreate: %s", hipGetErrorString(e));
    }
    st->events_ready = true;
  }
  return FLYAI_OK;
}

extern "C" void* flyai_stage_debug_buffer(flyai_stage* st, int32_t which) {
  if (!st || !st->dev) return nullptr;
  const size_t offs[] = {st->o_xn, st->o_gemm, st->o_qrot, st->o_attn, st->o_ids, st->o_w,
                         st->o_off, st->o_perm, st->o_inv, st->o_hmoe, st->o_y, st->o_pos,
                         st->o_sid, st->o_cu};
  if (which < 0 || which >= (int)(sizeof(offs) / sizeof(offs[0]))) return nullptr;
  return st->dev + offs[which];
}

#define RUN(x)              \
  do {                      \
    const int rc__ = (x);   \
    if (rc__) return rc__;  \
  } while (0)

static int copy_h2d(char* dst, const char* src, size_t bytes, hipStream_t s) {
  if (bytes == 0) return FLYAI_OK;
  const hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, s);
  if (e != hipSuccess) return set_error(FLYAI_EHIP, "hipMemcpyAsync: %s", hipGetErrorString(e));
  return FLYAI_OK;
}

// Where this step's batch sits in the device blob, and how the kernels are sized.
namespace {
struct StepPlan {
  int Tn, S;
  int grid_items[2], grid_groups[2];  // launch sizes: exact counts, or the plan capacities (graphs)
  int n_small[2];
  int n_pitems[2];  // chunked-prefill attention items (exact counts, part of the graph key)
  int merge[2];     // some group has more than one split: the merge kernel runs (part of the graph key)
  int lean[2];      // every split item has <= 2 tokens: the three-wave step kernel (part of the graph key)
  size_t off_counts, off_q, off_st, off_cap, off_base, off_items[2], off_groups[2], off_pitems[2];
  bool tree = false;  // a tree-verify step: the blob carries the flyai_attn_tree at off_tree
  size_t off_tree = 0, off_tree_depth = 0;
};
}  // namespace

// The step's kernel sequence: ragged packing, then every layer.  Runs eagerly or under capture.
// counts != nullptr: the attention grids are capacities and the kernels read the live counts there.
static int record_step(flyai_stage* st, const StepPlan& sp, const int32_t* counts, uint16_t* hidden,
                       hipStream_t s) {
  const flyai_stage_config& c = st->cfg;
  char* d = st->dev;
  char* blob = d + st->o_blob;
  auto I32 = [&](size_t o) { return reinterpret_cast<int32_t*>(d + o); };
  auto F32 = [&](size_t o) { return reinterpret_cast<float*>(d + o); };
  auto B16 = [&](size_t o) { return reinterpret_cast<uint16_t*>(d + o); };
  const int64_t* base_d = reinterpret_cast<const int64_t*>(blob + sp.off_base);
  const int32_t* cap_d = reinterpret_cast<const int32_t*>(blob + sp.off_cap);
  const flyai_attn_tree* tree_d = sp.tree ? reinterpret_cast<const flyai_attn_tree*>(blob + sp.off_tree) : nullptr;
  const int32_t* kv_pos = sp.tree ? I32(st->o_kvpos) : nullptr;

  const int Tn = sp.Tn;
  const int H = c.hidden, E = c.n_experts, k = c.top_k, I = c.intermediate;
  const bool fused_route = Tn <= 256 && Tn * k <= 4096;
  // the batch packing and the first layer's input RMSNorm in one launch (independent of each other)
  RUN(launch_pack(reinterpret_cast<const int32_t*>(blob + sp.off_q),
                  reinterpret_cast<const int32_t*>(blob + sp.off_st), base_d, cap_d, sp.S, c.head_dim,
                  c.max_tokens, I32(st->o_cu), I32(st->o_pos), I32(st->o_sid), I32(st->o_kvlen),
                  reinterpret_cast<int64_t*>(d + st->o_slot), I32(st->o_status),
                  sp.tree ? reinterpret_cast<const int32_t*>(blob + sp.off_tree_depth) : nullptr,
                  I32(st->o_kvpos), s, Tn, hidden, st->layers[0].ln1, H, c.rms_eps, B16(st->o_xn)));
  for (int l = 0; l < c.n_layers; ++l) {
    const flyai_layer_desc& L = st->layers[l];
    const int p = L.sliding ? 1 : 0;
    // xn holds this layer's input RMSNorm (written by the previous layer's combine)
    RUN(launch_qkv_rope_kv(B16(st->o_xn), L.wqkv, L.bqkv, F32(st->o_gemm), I32(st->o_pos),
                           I32(st->o_sid), st->cos_tab, st->sin_tab, c.rope_positions, Tn, H,
                           c.n_q_heads, c.n_kv_heads, c.head_dim, base_d, cap_d, B16(st->o_qrot),
                           L.k_pool, L.v_pool, kv_pos, s));
    if (sp.n_pitems[p] > 0 && !tree_d) {
      // prefill and split items share one launch (attn_step_kernel)
      RUN(launch_attn_step(B16(st->o_qrot), L.k_pool, L.v_pool, base_d, cap_d, L.sinks, L.sliding ? c.window : 0,
                           c.n_q_heads, reinterpret_cast<const flyai_attn_item*>(blob + sp.off_items[p]),
                           sp.grid_items[p], reinterpret_cast<const flyai_attn_group*>(blob + sp.off_groups[p]),
                           sp.grid_groups[p], counts ? counts + 2 * p : nullptr, F32(st->o_parts),
                           reinterpret_cast<const flyai_attn_item*>(blob + sp.off_pitems[p]), sp.n_pitems[p],
                           B16(st->o_attn), sp.merge[p] != 0, sp.lean[p] != 0, s));
    } else {
      RUN(launch_attn(B16(st->o_qrot), L.k_pool, L.v_pool, base_d, cap_d, L.sinks,
                      L.sliding ? c.window : 0, c.n_q_heads,
                      reinterpret_cast<const flyai_attn_item*>(blob + sp.off_items[p]), sp.grid_items[p],
                      sp.n_small[p], reinterpret_cast<const flyai_attn_group*>(blob + sp.off_groups[p]),
                      sp.grid_groups[p], counts ? counts + 2 * p : nullptr, F32(st->o_parts),
                      B16(st->o_attn), tree_d, sp.merge[p] != 0, s));
      RUN(launch_attn_prefill(B16(st->o_qrot), L.k_pool, L.v_pool, base_d, cap_d, L.sinks,
                              L.sliding ? c.window : 0, c.n_q_heads,
                              reinterpret_cast<const flyai_attn_item*>(blob + sp.off_pitems[p]), sp.n_pitems[p],
                              B16(st->o_attn), s));
    }
    if (fused_route) {
      // decode-sized: o-proj finalize + residual + RMSNorm + router logits, then top-k + permute
      RUN(launch_linear_residual_rmsnorm_logits(B16(st->o_attn), L.wo, L.bo, Tn, H, c.n_q_heads * c.head_dim,
                                                hidden, B16(st->o_h2), L.ln2, c.rms_eps, B16(st->o_xn),
                                                F32(st->o_gemm), L.router_w, L.router_b, E,
                                                F32(st->o_logits), s));
      RUN(launch_topk_permute(F32(st->o_logits), Tn, E, k, I32(st->o_ids), F32(st->o_w), I32(st->o_hist),
                              I32(st->o_off), I32(st->o_perm), I32(st->o_inv), s));
    } else {
      RUN(launch_linear_residual_rmsnorm(B16(st->o_attn), L.wo, L.bo, Tn, H, c.n_q_heads * c.head_dim,
                                         hidden, L.ln2, c.rms_eps, B16(st->o_xn), F32(st->o_gemm), s));
      RUN(launch_route_permute(B16(st->o_xn), L.router_w, L.router_b, Tn, H, E, k, I32(st->o_ids),
                               F32(st->o_w), F32(st->o_logits), I32(st->o_hist), I32(st->o_off),
                               I32(st->o_perm), I32(st->o_inv), s));
    }
    if (c.moe_dense_fp8 && moe_batch_is_dense(Tn * k, E, H < I ? H : I)) {
      // dense groups on the scaled MFMA: the activation operands quantised to fp8 first
      uint8_t* xq = reinterpret_cast<uint8_t*>(d + st->o_xq);
      uint8_t* xs = reinterpret_cast<uint8_t*>(d + st->o_xs);
      uint8_t* hq = reinterpret_cast<uint8_t*>(d + st->o_hq);
      uint8_t* hs = reinterpret_cast<uint8_t*>(d + st->o_hs);
      RUN(launch_mx_act_quant(B16(st->o_xn), Tn, H, xq, xs, s));
      RUN(launch_moe_gate_up_fp8act(B16(st->o_xn), xq, xs, I32(st->o_perm), I32(st->o_off), k, L.w13_packed, L.b13,
                                    Tn, E, H, I, B16(st->o_hmoe), s));
      RUN(launch_mx_act_quant(B16(st->o_hmoe), Tn * k, I, hq, hs, s));
      RUN(launch_moe_down_fp8act(B16(st->o_hmoe), hq, hs, I32(st->o_off), L.w2_packed, L.b2, Tn * k, E, H, I,
                                 F32(st->o_y), s));
    } else {
      RUN(launch_moe_gate_up(B16(st->o_xn), I32(st->o_perm), I32(st->o_off), k, L.w13_packed, L.b13,
                             Tn, E, H, I, B16(st->o_hmoe), s));
      RUN(launch_moe_down(B16(st->o_hmoe), I32(st->o_off), L.w2_packed, L.b2, Tn * k, E, H, I,
                          F32(st->o_y), s));
    }
    const float* next_ln1 = (l + 1 < c.n_layers) ? st->layers[l + 1].ln1 : nullptr;
    // the fused path left the post-attention residual in o_h2; the other path updated hidden in place
    const uint16_t* resid = fused_route ? B16(st->o_h2) : hidden;
    RUN(launch_combine(F32(st->o_y), I32(st->o_inv), F32(st->o_w), Tn, k, H, resid, hidden, next_ln1,
                       c.rms_eps, B16(st->o_xn), s));
  }
  return FLYAI_OK;
}

static int hip_fail(const char* what, hipError_t e) {
  return set_error(FLYAI_EHIP, "%s: %s", what, hipGetErrorString(e));
}

// The executable graph for this step's key, captured on first use (least recently used evicted).
static int step_graph(flyai_stage* st, const StepPlan& sp, hipGraphExec_t* out) {
  const int64_t key[12] = {sp.Tn, sp.S, sp.grid_items[0], sp.grid_items[1], sp.grid_groups[0], sp.grid_groups[1],
                           sp.n_pitems[0], sp.n_pitems[1], sp.merge[0], sp.merge[1], sp.lean[0], sp.lean[1]};
  ++st->use_clock;
  for (auto& g : st->graph_cache)
    if (memcmp(g.key, key, sizeof(key)) == 0) {
      g.last_use = st->use_clock;
      *out = g.exec;
      return FLYAI_OK;
    }
  if (!st->capture_stream) {
    const hipError_t e = hipStreamCreateWithFlags(&st->capture_stream, hipStreamNonBlocking);
    if (e != hipSuccess) return hip_fail("hipStreamCreate", e);
  }
  hipStream_t cs = st->capture_stream;
  hipError_t e = hipStreamBeginCapture(cs, hipStreamCaptureModeThreadLocal);
  if (e != hipSuccess) return hip_fail("hipStreamBeginCapture", e);
  const int rc = record_step(st, sp, reinterpret_cast<const int32_t*>(st->dev + st->o_blob + sp.off_counts),
                             reinterpret_cast<uint16_t*>(st->dev + st->o_hidden), cs);
  hipGraph_t graph = nullptr;
  e = hipStreamEndCapture(cs, &graph);
  if (rc) {
    if (graph) hipGraphDestroy(graph);
    return rc;
  }
  if (e != hipSuccess) return hip_fail("hipStreamEndCapture", e);
  hipGraphExec_t exec = nullptr;
  e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
  hipGraphDestroy(graph);
  if (e != hipSuccess) return hip_fail("hipGraphInstantiate", e);
  if ((int)st->graph_cache.size() >= kGraphCacheMax) {
    size_t lru = 0;
    for (size_t i = 1; i < st->graph_cache.size(); ++i)
      if (st->graph_cache[i].last_use < st->graph_cache[lru].last_use) lru = i;
    hipGraphExecDestroy(st->graph_cache[lru].exec);
    st->graph_cache.erase(st->graph_cache.begin() + lru);
  }
  flyai_stage::Graph g;
  memcpy(g.key, key, sizeof(key));
  g.exec = exec;
  g.last_use = st->use_clock;
  st->graph_cache.push_back(g);
  ++st->graphs_captured;
  *out = exec;
  return FLYAI_OK;
}

extern "C" int flyai_stage_set_graphs(flyai_stage* st, int32_t enable) {
  FLYAI_REQUIRE(st, "set_graphs: null stage");
  st->graphs = enable != 0;
  return FLYAI_OK;
}

extern "C" int32_t flyai_stage_graphs_captured(const flyai_stage* st) { return st ? st->graphs_captured : 0; }

// A group of one split is finished by its item; the merge kernel is needed only past that.
static int plan_needs_merge(const flyai_attn_group* groups, int n) {
  for (int i = 0; i < n; ++i)
    if (groups[i].n_splits > 1) return 1;
  return 0;
}

// One compact blob per step: live counts | q_lens | starts | kv_cap | kv_base | items x2 | groups x2
// [| tree], staged through the double-buffered pinned halves and moved to the device by one
// launch (blob_fetch_kernel; an H2D copy if the staging is not mapped).
static int stage_blob(flyai_stage* st, StepPlan& sp, const int32_t* q_lens, const int32_t* starts,
                      const int64_t* kv_base, const int32_t* kv_cap, const int* n_items,
                      const int* n_groups, const std::vector<char>* tree, hipStream_t s) {
  const int S = sp.S;
  Carve b;
  sp.off_counts = b.take(4 * sizeof(int32_t));
  sp.off_q = b.take((size_t)S * 4);
  sp.off_st = b.take((size_t)S * 4);
  sp.off_cap = b.take((size_t)S * 4);
  sp.off_base = b.take((size_t)S * 8);
  for (int p = 0; p < 2; ++p) sp.off_items[p] = b.take((size_t)sp.grid_items[p] * sizeof(flyai_attn_item));
  for (int p = 0; p < 2; ++p) sp.off_groups[p] = b.take((size_t)sp.grid_groups[p] * sizeof(flyai_attn_group));
  for (int p = 0; p < 2; ++p) sp.off_pitems[p] = b.take((size_t)sp.n_pitems[p] * sizeof(flyai_attn_item));
  sp.tree = tree != nullptr;
  if (tree) {
    sp.off_tree = b.take(tree->size());
    sp.off_tree_depth = sp.off_tree + reinterpret_cast<const flyai_attn_tree*>(tree->data())->depth_off;
  }
  if (b.off > st->blob_max) return set_error(FLYAI_ERANGE, "batch blob exceeds its reservation");
  // wait until the GPU consumed this staging half's previous contents, then fill it
  const int h = st->half;
  st->half ^= 1;
  const hipError_t ew = hipEventSynchronize(st->staged[h]);
  if (ew != hipSuccess) return hip_fail("hipEventSynchronize", ew);
  char* hb = st->host + h * st->host_half;
  const int32_t counts[4] = {n_items[0], n_groups[0], n_items[1], n_groups[1]};
  memcpy(hb + sp.off_counts, counts, sizeof(counts));
  memcpy(hb + sp.off_q, q_lens, S * 4);
  memcpy(hb + sp.off_st, starts, S * 4);
  memcpy(hb + sp.off_cap, kv_cap, S * 4);
  memcpy(hb + sp.off_base, kv_base, S * 8);
  for (int p = 0; p < 2; ++p) {
    memcpy(hb + sp.off_items[p], st->plan_items[p].data(), n_items[p] * sizeof(flyai_attn_item));
    memcpy(hb + sp.off_groups[p], st->plan_groups[p].data(), n_groups[p] * sizeof(flyai_attn_group));
    memcpy(hb + sp.off_pitems[p], st->plan_pitems[p].data(), sp.n_pitems[p] * sizeof(flyai_attn_item));
  }
  if (tree) memcpy(hb + sp.off_tree, tree->data(), tree->size());
  if (st->host_dev)
    RUN(launch_blob_fetch(st->host_dev + h * st->host_half, st->dev + st->o_blob, b.off, s));
  else
    RUN(copy_h2d(st->dev + st->o_blob, hb, b.off, s));
  const hipError_t er = hipEventRecord(st->staged[h], s);
  if (er != hipSuccess) return hip_fail("hipEventRecord", er);
  return FLYAI_OK;
}

// Every sequence's slab [kv_base, kv_base + Hkv * kv_cap * D) must end inside the smallest bound pool,
// and no two sequences' slabs may overlap: their K/V appends would race and each would read the other's
// keys.  Host-side, before any launch (the reference raises ContextOverflow before any write,
// phase0/fastverify.py:23-26).
static int check_slabs(flyai_stage* st, const int64_t* kv_base, const int32_t* kv_cap, int S) {
  const flyai_stage_config& c = st->cfg;
  int64_t pool = INT64_MAX;
  for (int l = 0; l < c.n_layers; ++l) pool = std::min(pool, st->layers[l].kv_pool_elems);
  const int64_t per_pos = (int64_t)c.n_kv_heads * c.head_dim;
  for (int b = 0; b < S; ++b) {
    const int64_t end = kv_base[b] + (int64_t)kv_cap[b] * per_pos;
    if (end > pool)
      return set_error(FLYAI_ERANGE, "sequence %d: KV slab [%lld, %lld) ends past the pools (%lld elements)", b,
                       (long long)kv_base[b], (long long)end, (long long)pool);
  }
  if (S < 2) return FLYAI_OK;
  int* order = st->slab_order.data();
  for (int b = 0; b < S; ++b) order[b] = b;
  std::sort(order, order + S, [&](int a, int b) { return kv_base[a] < kv_base[b]; });
  for (int i = 0; i + 1 < S; ++i) {
    const int a = order[i], b = order[i + 1];
    if (kv_base[a] + (int64_t)kv_cap[a] * per_pos > kv_base[b])
      return set_error(FLYAI_EINVAL, "sequences %d and %d have overlapping KV slabs (bases %lld and %lld)", a, b,
                       (long long)kv_base[a], (long long)kv_base[b]);
  }
  return FLYAI_OK;
}

extern "C" int flyai_stage_forward(flyai_stage* st, const int32_t* q_lens, const int32_t* starts,
                                   const int64_t* kv_base, const int32_t* kv_cap, int32_t S,
                                   uint16_t* hidden, flyai_stream_t stream) {
  FLYAI_REQUIRE(st && q_lens && starts && kv_base && kv_cap && hidden, "forward: null pointer");
  const flyai_stage_config& c = st->cfg;
  FLYAI_REQUIRE(S >= 1 && S <= c.max_seqs, "forward: n_seqs %d out of [1, %d]", S, c.max_seqs);
  int64_t T = 0;
  for (int b = 0; b < S; ++b) {
    FLYAI_REQUIRE(q_lens[b] >= 1 && starts[b] >= 0, "forward: sequence %d has q_len %d start %d", b,
                  q_lens[b], starts[b]);
    FLYAI_REQUIRE(kv_cap[b] > 0 && kv_cap[b] % 64 == 0 && kv_base[b] >= 0 && kv_base[b] % 8 == 0,
                  "forward: sequence %d needs kv_cap %% 64 == 0 and kv_base %% 8 == 0", b);
    const int64_t need = (int64_t)starts[b] + q_lens[b];
    if (need > kv_cap[b])
      return set_error(FLYAI_ERANGE, "sequence %d needs %lld positions > KV capacity %d", b,
                       (long long)need, kv_cap[b]);
    if (need > c.rope_positions)
      return set_error(FLYAI_ERANGE, "sequence %d needs %lld positions > rope table %d", b,
                       (long long)need, c.rope_positions);
    T += q_lens[b];
  }
  if (T > c.max_tokens)
    return set_error(FLYAI_ERANGE, "batch has %lld tokens > max_tokens %d", (long long)T, c.max_tokens);
  for (int l = 0; l < c.n_layers; ++l)
    FLYAI_REQUIRE(st->layers[l].wqkv, "forward: layer %d not bound", l);
  RUN(check_slabs(st, kv_base, kv_cap, S));
  FLYAI_REQUIRE(st->dev && st->host, "forward: workspace not set");
  FLYAI_REQUIRE(st->cos_tab && st->sin_tab, "forward: rope tables not set");
  hipStream_t s = as_stream(stream);

  StepPlan sp;
  sp.Tn = (int)T;
  sp.S = S;
  int n_items[2], n_groups[2];
  for (int p = 0; p < 2; ++p) {
    RUN(attn_plan(q_lens, starts, S, c.n_kv_heads, p == 0 ? 0 : c.window, c.attn_split_keys,
                  st->plan_items[p].data(), c.max_attn_items, st->plan_groups[p].data(), st->max_groups,
                  &n_items[p], &n_groups[p], &sp.n_small[p], c.attn_prefill_min, st->plan_pitems[p].data(),
                  st->max_pitems, &sp.n_pitems[p]));
    // replayed graphs are sized by capacities, so that a step with a few more items (longer KV)
    // reuses the graph; the kernels read the live counts from the blob
    auto bucket = [](int n, int cap) { const int b = (n + kPlanBucket - 1) / kPlanBucket * kPlanBucket; return b < cap ? b : cap; };
    sp.grid_items[p] = st->graphs ? bucket(n_items[p], c.max_attn_items) : n_items[p];
    sp.grid_groups[p] = st->graphs ? bucket(n_groups[p], st->max_groups) : n_groups[p];
    sp.merge[p] = plan_needs_merge(st->plan_groups[p].data(), n_groups[p]);
    sp.lean[p] = sp.n_small[p] == n_items[p];
  }
  RUN(stage_blob(st, sp, q_lens, starts, kv_base, kv_cap, n_items, n_groups, nullptr, s));
  if (!st->graphs) return record_step(st, sp, nullptr, hidden, s);

  hipGraphExec_t exec = nullptr;
  RUN(step_graph(st, sp, &exec));
  // the graph reads and updates the stage-owned rows; the caller's rows are copied in and out
  uint16_t* hs = reinterpret_cast<uint16_t*>(st->dev + st->o_hidden);
  const size_t hb = (size_t)sp.Tn * c.hidden * 2;
  hipError_t e = hipMemcpyAsync(hs, hidden, hb, hipMemcpyDeviceToDevice, s);
  if (e != hipSuccess) return hip_fail("hipMemcpyAsync", e);
  e = hipGraphLaunch(exec, s);
  if (e != hipSuccess) return hip_fail("hipGraphLaunch", e);
  e = hipMemcpyAsync(hidden, hs, hb, hipMemcpyDeviceToDevice, s);
  if (e != hipSuccess) return hip_fail("hipMemcpyAsync", e);
  return FLYAI_OK;
}


extern "C" int flyai_stage_forward_tree(flyai_stage* st, int32_t start, int32_t n, const int32_t* parent,
                                        const int32_t* depth, int64_t kv_base, int32_t kv_cap,
                                        uint16_t* hidden, flyai_stream_t stream) {
  FLYAI_REQUIRE(st && parent && depth && hidden, "forward_tree: null pointer");
  const flyai_stage_config& c = st->cfg;
  FLYAI_REQUIRE(n >= 1 && n <= st->tree_cap, "forward_tree: tree size %d outside [1, %d] (min(max_tokens, %d))", n,
                st->tree_cap, FLYAI_TREE_MAX_NODES);
  FLYAI_REQUIRE(start >= 0 && kv_cap > 0 && kv_cap % 64 == 0 && kv_base >= 0 && kv_base % 8 == 0,
                "forward_tree: needs start >= 0, kv_cap %% 64 == 0 and kv_base %% 8 == 0");
  // validate_tree (phase0/fastverify.py:29-49): parents in range and not self, depths consistent,
  // which forces acyclicity -- checked before any parent walk
  for (int i = 0; i < n; ++i) {
    FLYAI_REQUIRE(parent[i] >= -1 && parent[i] < n && parent[i] != i,
                  "forward_tree: tree node %d: parent %d out of range [-1, %d)", i, parent[i], n);
    FLYAI_REQUIRE(depth[i] >= 0, "forward_tree: tree node %d: depth %d invalid", i, depth[i]);
  }
  for (int i = 0; i < n; ++i) {
    const int want = parent[i] == -1 ? 0 : depth[parent[i]] + 1;
    FLYAI_REQUIRE(depth[i] == want, "forward_tree: tree node %d: depth %d != %d (parent %d; cycle or bad depth)",
                  i, depth[i], want, parent[i]);
  }
  const int64_t need = (int64_t)start + n;
  if (need > kv_cap)
    return set_error(FLYAI_ERANGE, "tree decode needs %lld positions > KV capacity %d", (long long)need, kv_cap);
  if (need > c.rope_positions)
    return set_error(FLYAI_ERANGE, "tree decode needs %lld positions > rope table %d", (long long)need,
                     c.rope_positions);
  for (int l = 0; l < c.n_layers; ++l)
    FLYAI_REQUIRE(st->layers[l].wqkv, "forward_tree: layer %d not bound", l);
  RUN(check_slabs(st, &kv_base, &kv_cap, 1));
  FLYAI_REQUIRE(st->dev && st->host, "forward_tree: workspace not set");
  FLYAI_REQUIRE(st->cos_tab && st->sin_tab, "forward_tree: rope tables not set");
  // The two visibility masks (FastVerify._tset, phase0/fastverify.py:250-272): row i of mask 0 holds
  // node i and its ancestors, row i of mask 1 those of them fewer than `window` levels above node i.
  // Nodes are visited in order of depth (a counting sort), so a parent's rows are complete before
  // its children copy them: row(i) = row(parent) + node i, and on sliding layers minus the one
  // ancestor exactly `window` levels up.
  try {
    st->tree_img.assign(tree_bytes(n), 0);
  } catch (...) {
    return set_error(FLYAI_EINVAL, "forward_tree: out of host memory for the tree masks");
  }
  char* img = st->tree_img.data();
  flyai_attn_tree* tr = reinterpret_cast<flyai_attn_tree*>(img);
  tree_layout(n, tr);
  tr->start = start;
  const int W = tr->words;
  memcpy(img + tr->depth_off, depth, (size_t)n * 4);
  uint64_t* m0 = reinterpret_cast<uint64_t*>(img + tr->mask_off[0]);
  uint64_t* m1 = reinterpret_cast<uint64_t*>(img + tr->mask_off[1]);
  int* cnt = st->tree_order.data();  // n + 1 depth counters (depths are below n), then the order
  int* order = cnt + n + 1;
  std::fill(cnt, cnt + n + 1, 0);
  for (int i = 0; i < n; ++i) ++cnt[depth[i] + 1];
  for (int d = 0; d < n; ++d) cnt[d + 1] += cnt[d];
  for (int i = 0; i < n; ++i) order[cnt[depth[i]]++] = i;
  for (int k = 0; k < n; ++k) {
    const int i = order[k], p = parent[i];
    uint64_t* r0 = m0 + (size_t)i * W;
    uint64_t* r1 = m1 + (size_t)i * W;
    if (p >= 0) {
      memcpy(r0, m0 + (size_t)p * W, (size_t)W * 8);
      memcpy(r1, m1 + (size_t)p * W, (size_t)W * 8);
    }
    r0[i >> 6] |= 1ull << (i & 63);
    r1[i >> 6] |= 1ull << (i & 63);
    if (c.window > 0 && depth[i] >= c.window) {
      int a = i;
      for (int up = 0; up < c.window; ++up) a = parent[a];
      r1[a >> 6] &= ~(1ull << (a & 63));
    }
  }
  hipStream_t s = as_stream(stream);
  StepPlan sp;
  sp.Tn = n;
  sp.S = 1;
  int n_items[2], n_groups[2];
  for (int p = 0; p < 2; ++p) {
    RUN(attn_plan_tree(start, n, depth, c.n_kv_heads, p == 0 ? 0 : c.window, c.attn_split_keys, st->plan_items[p].data(),
                       c.max_attn_items, st->plan_groups[p].data(), st->max_groups, &n_items[p],
                       &n_groups[p], &sp.n_small[p]));
    sp.grid_items[p] = n_items[p];
    sp.grid_groups[p] = n_groups[p];
    sp.n_pitems[p] = 0;
    sp.merge[p] = plan_needs_merge(st->plan_groups[p].data(), n_groups[p]);
    sp.lean[p] = 0;
  }
  const int32_t q_len = n, st0 = start;
  RUN(stage_blob(st, sp, &q_len, &st0, &kv_base, &kv_cap, n_items, n_groups, &st->tree_img, s));
  return record_step(st, sp, nullptr, hidden, s);
}
