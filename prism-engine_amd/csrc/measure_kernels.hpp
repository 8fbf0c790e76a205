// measure_kernels.hpp -- the read floor the GEMVs are compared against.
//
// k_stream_read reads every byte of a buffer once, as a GEMV streams its
// weights, and nothing else: one-wave workgroups, each lane sixteen 16-byte
// loads one kilobyte apart (16 KB per workgroup, nontemporal), an XOR of the
// data, and a store only if that XOR equals a constant (so the loads cannot
// be dropped and the kernel writes essentially nothing).  Of the launch
// shapes tried on MI355X for one 29.8 MB launch (16-byte or 4-byte lanes,
// 1- to 16-wave workgroups, persistent grids of 256..2048 workgroups) this
// one was the fastest.  It has no counterpart in the reference: it is the
// measuring stick for the hot path's kernels (bench.py --workload floor).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace prism {

constexpr int kStreamLoads = 16;                       // 16-byte loads per lane
constexpr uint32_t kStreamBytesPerBlock = 64 * 16 * kStreamLoads;  // 16 KB

__device__ __forceinline__ void stream_read_body(const uint8_t* __restrict__ p, uint32_t bytes,
                                                 uint32_t* __restrict__ sink) {
  typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));
  // every offset is in the VGPR offset: past `bytes` the range check returns zeros
  const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc((void*)p, (short)0, (int)bytes, 0x00020000);
  const uint32_t base = blockIdx.x * kStreamBytesPerBlock + threadIdx.x * 16u;
  u32x4v v[kStreamLoads];
#pragma unroll
  for (int u = 0; u < kStreamLoads; u++) v[u] = __builtin_amdgcn_raw_buffer_load_b128(r, base + u * 1024u, 0u, 2);
  uint32_t acc = 0;
#pragma unroll
  for (int u = 0; u < kStreamLoads; u++) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
  if (acc == 0x9E3779B9u) sink[blockIdx.x & 255u] = acc;
}

__global__ __launch_bounds__(64) void k_stream_read(const uint8_t* __restrict__ p, uint32_t bytes,
                                                    uint32_t* __restrict__ sink) {
  stream_read_body(p, bytes, sink);
}

}  // namespace prism
