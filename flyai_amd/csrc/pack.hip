// Ragged batch packing (decode, spec-verify and chunked-prefill rows -> one flat token axis).
#include "common.h"

namespace flyai {

constexpr int kPackThreads = 1024;
constexpr int kPackMaxSeqs = 8192;

// One workgroup: block-wide exclusive scan of q_lens into cu_seqlens (LDS), then every thread
// walks tokens with a binary search over the scanned offsets.
// Tree verify (tree_depth != NULL, one sequence): token i is rotated at position
// starts[0] + tree_depth[i] but its K/V goes to slot starts[0] + i; kv_pos receives the slot
// positions (it is only written in that mode).
__device__ __forceinline__ void pack_ragged_body(
    const int32_t* __restrict__ q_lens, const int32_t* __restrict__ starts,
    const int64_t* __restrict__ kv_base, const int32_t* __restrict__ kv_cap, int S, int head_dim,
    int max_tokens, int32_t* __restrict__ cu_out, int32_t* __restrict__ positions,
    int32_t* __restrict__ seq_id, int32_t* __restrict__ kv_len, int64_t* __restrict__ kv_slot,
    int32_t* __restrict__ status, const int32_t* __restrict__ tree_depth,
    int32_t* __restrict__ kv_pos) {
  __shared__ int32_t cu[kPackMaxSeqs + 1];
  __shared__ int32_t wave_tot[kPackThreads / 64];
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  if (tid == 0) *status = 0;
  // each thread owns a contiguous run of sequences
  const int per = (S + kPackThreads - 1) / kPackThreads;
  const int s0 = min(S, tid * per), s1 = min(S, s0 + per);
  int local = 0;
  for (int s = s0; s < s1; ++s) local += q_lens[s];
  // inclusive wave scan
  int incl = local;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    int v = __shfl_up(incl, off, 64);
    if (lane >= off) incl += v;
  }
  if (lane == 63) wave_tot[wave] = incl;
  __syncthreads();
  if (tid == 0) {
    int run = 0;
    for (int w = 0; w < kPackThreads / 64; ++w) {
      int t = wave_tot[w];
      wave_tot[w] = run;
      run += t;
    }
  }
  __syncthreads();
  int run = wave_tot[wave] + incl - local;
  for (int s = s0; s < s1; ++s) {
    cu[s] = run;
    cu_out[s] = run;
    int len = starts[s] + q_lens[s];
    kv_len[s] = len;
    if (len > kv_cap[s]) atomicOr(status, 1);
    run += q_lens[s];
  }
  if (s1 == S && s0 < s1) {
    cu[S] = run;
    cu_out[S] = run;
  }
  if (S == 0 && tid == 0) { cu[0] = 0; cu_out[0] = 0; }
  __syncthreads();
  const int T = cu[S];
  if (T > max_tokens && tid == 0) atomicOr(status, 2);
  const int Tw = min(T, max_tokens);
  for (int t = tid; t < Tw; t += kPackThreads) {
    int lo = 0, hi = S - 1;  // last s with cu[s] <= t
    while (lo < hi) {
      int mid = (lo + hi + 1) >> 1;
      if (cu[mid] <= t) lo = mid; else hi = mid - 1;
    }
    const int b = lo;
    const int slot_pos = starts[b] + (t - cu[b]);
    positions[t] = tree_depth ? starts[b] + tree_depth[t] : slot_pos;
    if (tree_depth) kv_pos[t] = slot_pos;
    seq_id[t] = b;
    kv_slot[t] = (slot_pos < kv_cap[b]) ? kv_base[b] + (int64_t)slot_pos * head_dim : (int64_t)-1;
  }
}

__global__ __launch_bounds__(kPackThreads) void pack_ragged_kernel(
    const int32_t* __restrict__ q_lens, const int32_t* __restrict__ starts,
    const int64_t* __restrict__ kv_base, const int32_t* __restrict__ kv_cap, int S, int head_dim,
    int max_tokens, int32_t* __restrict__ cu_out, int32_t* __restrict__ positions,
    int32_t* __restrict__ seq_id, int32_t* __restrict__ kv_len, int64_t* __restrict__ kv_slot,
    int32_t* __restrict__ status, const int32_t* __restrict__ tree_depth,
    int32_t* __restrict__ kv_pos) {
  pack_ragged_body(q_lens, starts, kv_base, kv_cap, S, head_dim, max_tokens, cu_out, positions, seq_id, kv_len,
                   kv_slot, status, tree_depth, kv_pos);
}

// The step's first two launches as one: workgroup 0 packs the batch, workgroups 1..T RMS-normalise
// the T hidden rows for the first layer (which does not depend on the packing).
static_assert(kPackThreads == kRowThreads, "one block size for both bodies");
__global__ __launch_bounds__(kPackThreads) void pack_norm_kernel(
    const int32_t* __restrict__ q_lens, const int32_t* __restrict__ starts,
    const int64_t* __restrict__ kv_base, const int32_t* __restrict__ kv_cap, int S, int head_dim,
    int max_tokens, int32_t* __restrict__ cu_out, int32_t* __restrict__ positions,
    int32_t* __restrict__ seq_id, int32_t* __restrict__ kv_len, int64_t* __restrict__ kv_slot,
    int32_t* __restrict__ status, const int32_t* __restrict__ tree_depth,
    int32_t* __restrict__ kv_pos, const uint16_t* __restrict__ x, const float* __restrict__ w, int H, float eps,
    uint16_t* __restrict__ y) {
  if (blockIdx.x == 0)
    pack_ragged_body(q_lens, starts, kv_base, kv_cap, S, head_dim, max_tokens, cu_out, positions, seq_id, kv_len,
                     kv_slot, status, tree_depth, kv_pos);
  else
    rmsnorm_row(x, w, H, eps, y, blockIdx.x - 1);
}

}  // namespace flyai

using namespace flyai;

extern "C" int flyai_pack_ragged(const int32_t* q_lens, const int32_t* starts,
                                 const int64_t* kv_base, const int32_t* kv_cap, int32_t n_seqs,
                                 int32_t head_dim, int32_t max_tokens, int32_t* cu_seqlens,
                                 int32_t* positions, int32_t* seq_id, int32_t* kv_len,
                                 int64_t* kv_slot, int32_t* status_dev, flyai_stream_t stream) {
  FLYAI_REQUIRE(n_seqs >= 1 && n_seqs <= kPackMaxSeqs, "pack: n_seqs %d out of [1, %d]", n_seqs,
                kPackMaxSeqs);
  FLYAI_REQUIRE(head_dim > 0 && max_tokens >= 0, "pack: bad head_dim/max_tokens");
  FLYAI_REQUIRE(q_lens && starts && kv_base && kv_cap && cu_seqlens && positions && seq_id &&
                    kv_len && kv_slot && status_dev,
                "pack: null pointer");
  hipLaunchKernelGGL(pack_ragged_kernel, dim3(1), dim3(kPackThreads), 0, as_stream(stream),
                     q_lens, starts, kv_base, kv_cap, n_seqs, head_dim, max_tokens, cu_seqlens,
                     positions, seq_id, kv_len, kv_slot, status_dev, nullptr, nullptr);
  return check_launch("pack_ragged");
}

namespace flyai {

// The step's batch blob from the pinned host staging (mapped into the device's address space) into
// device memory, read by the GPU itself rather than by an H2D copy: on a 9-layer decode step of 32
// sequences (56 tokens, 87 launches) the copy engine's transfer and its hand-over to the compute queue left the GPU idle about
// 20 us before every step (2.835 -> 2.789 ms per step).  The loads are system-coherent (sc0 sc1), so
// they fetch what the host wrote for this step, never a cached line of an earlier one; offsets past
// the blob read zero and are not stored.
__global__ __launch_bounds__(256) void blob_fetch_kernel(const char* __restrict__ src, uint32_t bytes,
                                                         char* __restrict__ dst) {
  const __amdgpu_buffer_rsrc_t rs =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(src), (short)0, bytes, 0x00020000);
  const uint32_t off = (blockIdx.x * 256 + threadIdx.x) * 16;
  typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
  const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, 1 | 16);
  if (off < bytes) *reinterpret_cast<u32x4*>(dst + off) = v;
}

int launch_blob_fetch(const char* src_dev, char* dst, size_t bytes, hipStream_t s) {
  if (bytes == 0) return FLYAI_OK;
  if (bytes % 16 != 0 || bytes > 0x7fffffffu)
    return set_error(FLYAI_EINVAL, "blob_fetch: %zu bytes (multiple of 16 below 2 GiB)", bytes);
  hipLaunchKernelGGL(blob_fetch_kernel, dim3((unsigned)((bytes / 16 + 255) / 256)), dim3(256), 0, s, src_dev,
                     (uint32_t)bytes, dst);
  return check_launch("blob_fetch");
}

// The packing, and with norm_rows > 0 the first layer's RMSNorm of norm_rows rows of x in the same
// launch (pack_norm_kernel).
int launch_pack(const int32_t* q_lens, const int32_t* starts, const int64_t* kv_base,
                const int32_t* kv_cap, int S, int head_dim, int max_tokens, int32_t* cu,
                int32_t* positions, int32_t* seq_id, int32_t* kv_len, int64_t* kv_slot,
                int32_t* status, const int32_t* tree_depth, int32_t* kv_pos, hipStream_t s,
                int norm_rows, const uint16_t* x, const float* w, int H, float eps, uint16_t* y) {
  if (norm_rows > 0) {
    hipLaunchKernelGGL(pack_norm_kernel, dim3(1 + norm_rows), dim3(kPackThreads), 0, s, q_lens, starts, kv_base,
                       kv_cap, S, head_dim, max_tokens, cu, positions, seq_id, kv_len, kv_slot, status,
                       tree_depth, kv_pos, x, w, H, eps, y);
    return check_launch("pack_norm");
  }
  hipLaunchKernelGGL(pack_ragged_kernel, dim3(1), dim3(kPackThreads), 0, s, q_lens, starts, kv_base,
                     kv_cap, S, head_dim, max_tokens, cu, positions, seq_id, kv_len, kv_slot, status,
                     tree_depth, kv_pos);
  return check_launch("pack_ragged");
}

}  // namespace flyai
