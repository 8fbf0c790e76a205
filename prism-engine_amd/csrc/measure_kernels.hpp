// measure_kernels.hpp -- the read floor the GEMVs are compared against.
//
// Measuring sticks, none with a counterpart in the reference.
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

// The cost of one dependent launch (bench.py --workload launch): a kernel of
// one one-wave workgroup that does nothing, launched back to back.
__global__ __launch_bounds__(64) void k_launch_empty() {}

// The matrix cores' rate on register-only work (bench.py --workload mfma):
// each wave (one per SIMD, four per workgroup) runs `iters` rounds of 16
// independent v_mfma_f32_32x32x16_f16 (16 accumulators, 256 registers),
// 524 288 flop a round.  The A operands differ per accumulator and B is
// rotated every round, so the operands keep changing as a GEMM's do; the
// result is written only if it equals a constant, so the work cannot be
// dropped and (almost surely) nothing is written.  Launched over all CUs and
// over three quarters of them, it shows how the rate per CU depends on how
// many CUs run it.
typedef _Float16 probe_half8 __attribute__((ext_vector_type(8)));
typedef float probe_float16 __attribute__((ext_vector_type(16)));
__global__ __launch_bounds__(256) void k_mfma_probe(uint32_t iters, float* __restrict__ sink) {
  typedef uint32_t u32x4p __attribute__((ext_vector_type(4)));
  const uint32_t t = threadIdx.x + 977u * blockIdx.x;
  u32x4p bw;
  for (int i = 0; i < 4; i++) {
    const uint32_t h = (t * 2654435761u + 40503u * (uint32_t)i) >> 9;
    bw[i] = (h & 0x03FF03FFu) | 0x38003800u;  // fp16 pairs in [0.5, 1)
  }
  probe_half8 a[16];
  for (int j = 0; j < 16; j++) {
    u32x4p aw;
    for (int i = 0; i < 4; i++) aw[i] = bw[i] ^ (0x00550055u * (uint32_t)(j + 1)) ^ ((uint32_t)(j & 1) << 15);
    a[j] = __builtin_bit_cast(probe_half8, aw);
  }
  probe_float16 acc[16];
  for (int j = 0; j < 16; j++)
    for (int e = 0; e < 16; e++) acc[j][e] = 0.0f;
  for (uint32_t it = 0; it < iters; it++) {
    const probe_half8 b = __builtin_bit_cast(probe_half8, bw);
#pragma unroll
    for (int j = 0; j < 16; j++) acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[j], b, acc[j], 0, 0, 0);
    bw = u32x4p{bw.y, bw.z, bw.w, bw.x};
  }
  float s = 0.0f;
#pragma unroll
  for (int j = 0; j < 16; j++) {
    const float v = acc[j][0];
    s += v;
  }
  if (s == 1234.5f) sink[threadIdx.x & 255u] = s;
}

}  // namespace prism
