// HBM read-streaming ceiling: a kernel that only reads, used to measure the bandwidth the stage's
// weight-streaming kernels can reach on this GPU (the achieved figure they are compared against,
// next to the 8 TB/s datasheet peak).
#include "common.h"

namespace flyai {

typedef unsigned int probe_u32x4 __attribute__((ext_vector_type(4)));

// Every 16-byte vector of src is read exactly once.  A workgroup reads a contiguous chunk of U*256
// vectors per iteration (U loads in flight per thread, U * 4 KiB per workgroup), and the chunks are
// dealt to the workgroups round-robin.  The XOR of everything read decides a store that never happens
// for real data (a 1-in-2^32 value), which keeps the compiler from dropping the loads.
template <int U, bool NT>
__global__ __launch_bounds__(256) void hbm_read_kernel(const probe_u32x4* __restrict__ src, size_t n16,
                                                       uint32_t* __restrict__ sink) {
  constexpr size_t kChunk = (size_t)U * 256;
  uint32_t acc = 0;
  for (size_t c0 = (size_t)blockIdx.x * kChunk; c0 < n16; c0 += (size_t)gridDim.x * kChunk) {
    const probe_u32x4* p = src + c0 + threadIdx.x;
    if (c0 + kChunk <= n16) {
      probe_u32x4 v[U];
#pragma unroll
      for (int j = 0; j < U; ++j) v[j] = NT ? __builtin_nontemporal_load(p + j * 256) : p[j * 256];
#pragma unroll
      for (int j = 0; j < U; ++j) acc ^= v[j].x ^ v[j].y ^ v[j].z ^ v[j].w;
    } else {
      for (int j = 0; j < U; ++j)
        if (c0 + threadIdx.x + (size_t)j * 256 < n16) {
          const probe_u32x4 v = p[j * 256];
          acc ^= v.x ^ v.y ^ v.z ^ v.w;
        }
    }
  }
  if (acc == 0x9e3779b9u) sink[0] = acc;
}

}  // namespace flyai

using namespace flyai;

extern "C" int flyai_hbm_read_probe(const void* src, size_t bytes, int32_t nontemporal, int32_t grid,
                                    uint32_t* sink, flyai_stream_t stream) {
  FLYAI_REQUIRE(src && sink, "hbm_read_probe: null pointer");
  FLYAI_REQUIRE(bytes > 0 && bytes % 16 == 0 && ((uintptr_t)src & 15) == 0,
                "hbm_read_probe: need a 16-byte aligned buffer of a positive multiple of 16 bytes");
  FLYAI_REQUIRE(grid > 0 && grid <= 65536, "hbm_read_probe: grid must be in [1, 65536]");
  const size_t n16 = bytes / 16;
  auto* p = static_cast<const probe_u32x4*>(src);
  if (nontemporal)
    hipLaunchKernelGGL((hbm_read_kernel<8, true>), dim3(grid), dim3(256), 0, as_stream(stream), p, n16, sink);
  else
    hipLaunchKernelGGL((hbm_read_kernel<8, false>), dim3(grid), dim3(256), 0, as_stream(stream), p, n16, sink);
  return check_launch("hbm_read_probe");
}
