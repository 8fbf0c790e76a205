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

// Issue rate of one instruction kind (bench.py --workload issue): each wave
// runs `iters` rounds of 8 independent instructions of kind OP (0
// v_fma_f32, 1 v_dot2_f32_f16, 2 v_perm_b32, 3 v_mfma_f32_4x4x4f16, whose 16
// blocks are the lane-per-row GEMV's A operands in k_gemv_lpr4q); the
// workgroup's size sets the waves per SIMD.  The result is written only if
// it equals a constant.  It shows how many cycles apart one wave issues
// VALU instructions, how the SIMD's rate grows with more waves, and what a
// 4 x 4 x 4 matrix-core instruction costs beside the v_dot2 it replaces.
template <int OP>
__global__ __launch_bounds__(1024) void k_issue_probe(uint32_t iters, float* __restrict__ sink) {
  typedef _Float16 h2p __attribute__((ext_vector_type(2)));
  typedef _Float16 h4p __attribute__((ext_vector_type(4)));
  typedef float f4p __attribute__((ext_vector_type(4)));
  const uint32_t t = threadIdx.x;
  float s = 0.0f;
  if constexpr (OP == 0) {
    float a[8];
    float b = 1.0001f + (float)t * 1e-7f;
    for (int j = 0; j < 8; j++) a[j] = 0.5f + (float)(j + t);
    for (uint32_t it = 0; it < iters; it++) {
#pragma unroll
      for (int j = 0; j < 8; j++) a[j] = __builtin_fmaf(a[j], b, 0.25f);
      b = b * 0.99999f;
    }
    for (int j = 0; j < 8; j++) s += a[j];
  } else if constexpr (OP == 1) {
    uint32_t a[8];
    uint32_t b = 0x3c003c00u ^ t;
    float c[8];
    for (int j = 0; j < 8; j++) {
      a[j] = 0x3c003c00u + (uint32_t)j * 0x00010001u + t;
      c[j] = 0.0f;
    }
    for (uint32_t it = 0; it < iters; it++) {
#pragma unroll
      for (int j = 0; j < 8; j++)
        c[j] = __builtin_amdgcn_fdot2(__builtin_bit_cast(h2p, a[j]), __builtin_bit_cast(h2p, b), c[j], false);
      b = (b << 1) | (b >> 31);
    }
    for (int j = 0; j < 8; j++) s += c[j];
  } else if constexpr (OP == 2) {
    uint32_t a[8];
    uint32_t b = 0x01020304u ^ t;
    for (int j = 0; j < 8; j++) a[j] = 0x3c003c00u + (uint32_t)j * 0x00010001u + t;
    for (uint32_t it = 0; it < iters; it++) {
#pragma unroll
      for (int j = 0; j < 8; j++) a[j] = __builtin_amdgcn_perm(a[j], b, 0x05040100u + (uint32_t)j);
      b += 0x01010101u;
    }
    uint32_t x = 0;
    for (int j = 0; j < 8; j++) x ^= a[j];
    // an integer test: a float compare that can never hold would let the
    // compiler drop the loop
    if (x == 0x9E3779B9u) sink[t & 255u] = 1.0f;
    return;
  } else {
    h4p a[8], b;
    f4p c[8];
    for (int j = 0; j < 8; j++)
      for (int i = 0; i < 4; i++) a[j][i] = (_Float16)(0.001f * (float)(t + j + i));
    for (int i = 0; i < 4; i++) b[i] = (_Float16)(0.5f + 0.01f * (float)i);
    for (int j = 0; j < 8; j++) c[j] = f4p{0.0f, 0.0f, 0.0f, 0.0f};
    for (uint32_t it = 0; it < iters; it++) {
#pragma unroll
      for (int j = 0; j < 8; j++) c[j] = __builtin_amdgcn_mfma_f32_4x4x4f16(a[j], b, c[j], 0, 0, 0);
      b = h4p{b.y, b.z, b.w, b.x};
    }
    for (int j = 0; j < 8; j++) {
      const float v = c[j][0];
      s += v;
    }
  }
  if (s == 1234.5f) sink[t & 255u] = s;
}

}  // namespace prism
