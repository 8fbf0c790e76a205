// gemv_kernels.hpp -- shared pieces of the palettized-LUT GEMV for gfx950.
//
// y[b, r] = f16( sum_k f32(x[b, k]) * f32(LUT_r[idx(r, k)]) ) is the
// arithmetic of lut_gemv_cpu (compute-core/src/lut/evaluator.rs:21-44) over
// split-block weights (src/lut/compiler.rs:50-61).  This header holds the
// fp16 helpers, the kernel argument block, the generic kernel for shapes
// the tiled kernel (gemv_tile.hpp) does not take (K % 8 != 0, unaligned x)
// and the dense row decode.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace prism {

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float dot2(uint32_t w, uint32_t x, float acc) {
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(half2_t, w), __builtin_bit_cast(half2_t, x), acc, false);
}

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
// 16-byte streaming load (nontemporal hint: the index bytes are read once).
__device__ __forceinline__ uint4 ld_stream(const void* p) {
  const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ float h2f(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }
// fp32 -> fp16, round-to-nearest-even (v_cvt_f16_f32 uses the RNE mode).
// Buffer descriptor word 3 for gfx9-family (CDNA) raw buffers: 32-bit
// data format, no swizzle; the range check is against num_records bytes.
constexpr int kBufferWord3 = 0x00020000;
// Cache-policy operand of the buffer-load builtins: nontemporal.
constexpr int kNontemporal = 2;

__device__ __forceinline__ uint16_t f2h(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }

// Output store at device scope (global_store_short sc1: written through to
// where every XCD reads it, so the end-of-kernel L2 writeback finds nothing
// of it dirty).  MI355X, 4-bit hero GEMV, three alternating rounds on one
// box: 6.41-6.43 us against 6.45-6.46 with ordinary stores (system scope,
// sc0 sc1: 6.41-6.42; sc0 alone: no change; nontemporal stores were
// slower).  Only the 4-bit lane-per-row GEMVs use it: in the tile GEMV the
// decode step took 576 against 529 us per token and 4864 x 896 3.38 against
// 3.06 us, and the 8-bit lane-per-row GEMV at 4 vectors 14.1-14.4 against
// 14.0-14.2.
__device__ __forceinline__ void store_out(uint16_t* p, uint16_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// silu then the gate*up product with the CPU path's fp16 roundings
// (compute-core/src/lut/evaluator.rs:78-83,209-225).
__device__ __forceinline__ uint16_t swiglu_h(float gacc, float uacc) {
  const float g = h2f(f2h(gacc));
  const float u = h2f(f2h(uacc));
  const float s = h2f(f2h(g / (1.0f + expf(-g))));
  return f2h(s * u);
}

template <int G>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
  for (int off = G / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

struct GemvArgs {
  const uint8_t* lut;   // [N][2^BITS] fp16
  const uint8_t* idx;   // [N][row_bytes]
  const uint8_t* lut2;  // up weights (DUAL only)
  const uint8_t* idx2;
  const uint16_t* x;    // [nb][K] fp16
  uint16_t* y;          // [nb][N] fp16
  uint16_t* y2;         // DUAL with the pair epilogue: the up output [N]
  uint32_t N;
  uint32_t K;
  uint32_t nb;          // live batch rows (<= NB)
  float eps;            // RMS-norm epsilon (k_gemv_tile with kEpiNorm)
  const float* xpart;   // attention split partials (k_gemv_tile with kEpiAttnIn)
  uint32_t gi;          // GI layout: rows per group (kernels instantiated for GI)
};

// Generic kernel for shapes the tiled kernel does not take (K % 8 != 0,
// unaligned x): one wave per row, element-strided.  Follows lut_gemv_cpu's
// ragged-K rule for 4-bit weights: row stride K/2 bytes, only the first
// (K/8)*8 elements contribute.
// GI: the group-interleaved device layout (gemv_lpr.hpp describes it), for
// 4- and 8-bit weights: ceil(N/G) groups of [G row LUTs (32 B at 4 bits,
// 512 B at 8)][row bytes / 16 chunks][G rows][16 B], rows past N zero,
// G <= kGiMaxRows rows per group (one per lane of a wave).  A chunk holds 32
// elements at 4 bits, 16 at 8.
constexpr int kGiMaxRows = 64;  // rows per group at most
constexpr int kGiChunk = 16;    // index bytes per chunk

__host__ __device__ __forceinline__ uint32_t gi_lut_bytes(uint32_t bits) { return 2u << bits; }
__host__ __device__ __forceinline__ size_t gi_group_bytes(uint32_t G, uint32_t K, uint32_t bits) {
  return (size_t)G * gi_lut_bytes(bits) + (size_t)G * (K * bits / 8);
}
__host__ __device__ __forceinline__ size_t gi_bytes(uint32_t G, uint32_t N, uint32_t K, uint32_t bits) {
  return (size_t)((N + G - 1) / G) * gi_group_bytes(G, K, bits);
}
// Byte offset of row r's LUT, of its chunk c, and of the byte holding its
// element k.
__host__ __device__ __forceinline__ size_t gi_lut_offset(uint32_t G, uint32_t r, uint32_t K, uint32_t bits) {
  return (size_t)(r / G) * gi_group_bytes(G, K, bits) + (size_t)(r % G) * gi_lut_bytes(bits);
}
__host__ __device__ __forceinline__ size_t gi_chunk_offset(uint32_t G, uint32_t r, uint32_t c, uint32_t K,
                                                           uint32_t bits) {
  return (size_t)(r / G) * gi_group_bytes(G, K, bits) + (size_t)G * gi_lut_bytes(bits) +
         ((size_t)c * G + (r % G)) * kGiChunk;
}
__host__ __device__ __forceinline__ size_t gi_index_at(uint32_t G, uint32_t r, uint32_t k, uint32_t K,
                                                       uint32_t bits) {
  const uint32_t per = 128 / bits;  // elements per chunk
  return gi_chunk_offset(G, r, k / per, K, bits) + (k % per) * bits / 8;
}

// MODE: kGenSingle, or gate + up rows (lut2/idx2) with the SwiGLU
// epilogue (kGenSwiglu) or the two raw outputs y, y2 (kGenPair).
// GI: weights in the GI layout with a.gi rows per group (a.lut and a.idx
// both point at it).
constexpr int kGenSingle = 0, kGenSwiglu = 1, kGenPair = 2;
template <int BITS, int MODE, bool GI = false>
__global__ __launch_bounds__(64) void k_gemv_generic(GemvArgs a) {
  constexpr bool DUAL = MODE != kGenSingle;
  const uint32_t row = blockIdx.x;
  const int lane = threadIdx.x;
  const uint32_t K = a.K, N = a.N;
  const uint32_t stride = (BITS == 4) ? K / 2 : K;
  const uint32_t keff = (BITS == 4) ? (K / 8) * 8 : K;
  constexpr int NM = DUAL ? 2 : 1;
  const uint32_t nb = DUAL ? 1 : a.nb;
  for (uint32_t b = 0; b < nb; b++) {
    float acc[NM];
    for (int m = 0; m < NM; m++) {
      const uint8_t* lut =
          (m == 0 ? a.lut : a.lut2) + (GI ? gi_lut_offset(a.gi, row, K, BITS) : (size_t)row * (2u << BITS));
      const uint8_t* idx = (m == 0 ? a.idx : a.idx2) + (GI ? 0 : (size_t)row * stride);
      float s = 0.0f;
      for (uint32_t k = lane; k < keff; k += 64) {
        uint32_t e;
        if (BITS == 4) {
          const uint8_t byte = GI ? idx[gi_index_at(a.gi, row, k, K, 4)] : idx[k >> 1];
          e = (k & 1) ? (byte >> 4) : (byte & 15u);
        } else {
          e = GI ? idx[gi_index_at(a.gi, row, k, K, 8)] : idx[k];
        }
        const uint16_t lv = (uint16_t)(lut[2 * e] | (lut[2 * e + 1] << 8));
        s += h2f(a.x[(size_t)b * K + k]) * h2f(lv);
      }
      acc[m] = group_sum<64>(s);
    }
    if (lane == 0) {
      if constexpr (MODE == kGenSwiglu) {
        a.y[row] = swiglu_h(acc[0], acc[NM - 1]);
      } else if constexpr (MODE == kGenPair) {
        a.y[row] = f2h(acc[0]);
        a.y2[row] = f2h(acc[NM - 1]);
      } else {
        a.y[(size_t)b * N + row] = f2h(acc[0]);
      }
    }
  }
}

// Dense decode of rows [row0, row0+nrows): out[i][k] = LUT_r[idx(r, k)]
// (the per-row form of lut_embed, compute-core/src/lut/evaluator.rs:176-197).
// For 4-bit weights elements at k >= (K/8)*8 are written as 0, matching
// lut_embed's shorter output zero-padded.
// GI: weights in the GI layout with G rows per group (lut and idx both
// point at it).
template <int BITS, bool GI = false>
__global__ __launch_bounds__(256) void k_decode_rows(const uint8_t* lut, const uint8_t* idx, uint32_t N,
                                                     uint32_t K, uint32_t row0, uint32_t nrows, uint16_t* out,
                                                     uint32_t G) {
  const uint32_t stride = (BITS == 4) ? K / 2 : K;
  const uint32_t keff = (BITS == 4) ? (K / 8) * 8 : K;
  const size_t total = (size_t)nrows * K;
  for (size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x; t < total; t += (size_t)gridDim.x * blockDim.x) {
    const uint32_t i = (uint32_t)(t / K);
    const uint32_t k = (uint32_t)(t % K);
    const uint32_t r = row0 + i;
    uint16_t v = 0;
    if (r < N && k < keff) {
      uint32_t e;
      if (BITS == 4) {
        const uint8_t byte = GI ? idx[gi_index_at(G, r, k, K, 4)] : idx[(size_t)r * stride + (k >> 1)];
        e = (k & 1) ? (byte >> 4) : (byte & 15u);
      } else {
        e = GI ? idx[gi_index_at(G, r, k, K, 8)] : idx[(size_t)r * stride + k];
      }
      const uint8_t* l = lut + (GI ? gi_lut_offset(G, r, K, BITS) : (size_t)r * (2u << BITS)) + 2 * e;
      v = (uint16_t)(l[0] | (l[1] << 8));
    }
    out[t] = v;
  }
}

}  // namespace prism
