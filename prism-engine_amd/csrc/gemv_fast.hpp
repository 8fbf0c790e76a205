// gemv_fast.hpp -- wave-per-row-block palettized GEMV for gfx950.
//
// Same arithmetic as k_gemv (lut_gemv_cpu, compute-core/src/lut/
// evaluator.rs:21-44); different schedule, tuned for the decode shapes whose
// rows are a multiple of 64 16-byte chunks or close to it (the 4096- and
// 3584-wide projections of the BASELINE configs):
//
//  * one workgroup = one wave (64 lanes) owns PR consecutive rows; every
//    index load of those rows (PR * CPL dwordx4 per lane) and the rows'
//    LUTs are issued before any compute, straight-line with clamped
//    addresses, so the compiler counts them with vmcnt and each row is
//    computed as soon as its bytes land while the later rows are in flight;
//  * 4-bit: each row's 16-entry LUT is expanded in LDS into a 256-entry
//    pair table (entry b = {LUT[b & 15], LUT[b >> 4]}, 1 KB) at the bottom
//    of the wave's dynamic LDS (which starts at LDS address 0 when no static
//    LDS is declared).  Decode is then one SDWA shift (byte k of the index
//    word -> 4*b, the table offset; the row's table base is the ds_read
//    immediate) and one ds_read_b32 per index byte, whose result is the
//    fp16 pair that v_dot2_f32_f16 multiplies with the matching x pair:
//    1 VALU op + 1/2 LDS read per element.  Measured on MI355X, random
//    reads over 256 dwords run at ~13 lanes/clk/CU against ~29 for a
//    conflict-free 16-entry table; with the halved read count and no
//    packing op the two decodes time the same on the 4096 x 14336 matrix
//    (8.8-8.9 us, random indices), and the pair table needs fewer VGPRs
//    (69 vs 96), so every wave of the grid is resident at once;
//  * 8-bit: the 256-entry LUT itself is the table; each byte costs one SDWA
//    shift and one ds_read_u16, and pairs are packed with v_lshl_or_b32;
//  * x (the lane's fixed 32*CPL-element slice) is loaded once into VGPRs;
//  * each row's 64 partial sums are reduced with DPP (quad_perm, row
//    mirrors, row_bcast) into lane 63, which writes the fp16 result.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "gemv_kernels.hpp"

namespace prism {

// 8 index bytes (two dwords) -> 8 fp16 pairs {LUT[lo], LUT[hi]} of each
// byte, one ds_read_b32 per byte from the row's 256-entry pair table at LDS
// byte address OFF (entry b = LUT[b & 15] | LUT[b >> 4] << 16).  The SDWA
// shift turns byte k of the index word into the table offset 4*b.  `tbl` is
// the LDS base (an operand so the stores that fill the table are kept).
template <int OFF>
__device__ __forceinline__ void dec8_pair(uint32_t w0, uint32_t w1, const uint32_t* tbl, uint32_t (&p)[8]) {
  uint32_t a[8];
  asm volatile(
      "v_lshlrev_b32_sdwa %[a0], 2, %[w0] dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_0\n"
      "v_lshlrev_b32_sdwa %[a1], 2, %[w0] dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_1\n"
      "v_lshlrev_b32_sdwa %[a2], 2, %[w0] dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_2\n"
      "v_lshlrev_b32_sdwa %[a3], 2, %[w0] dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_3\n"
      "v_lshlrev_b32_sdwa %[a4], 2, %[w1] dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_0\n"
      "v_lshlrev_b32_sdwa %[a5], 2, %[w1] dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_1\n"
      "v_lshlrev_b32_sdwa %[a6], 2, %[w1] dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_2\n"
      "v_lshlrev_b32_sdwa %[a7], 2, %[w1] dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_3\n"
      "ds_read_b32 %[p0], %[a0] offset:%[off]\n"
      "ds_read_b32 %[p1], %[a1] offset:%[off]\n"
      "ds_read_b32 %[p2], %[a2] offset:%[off]\n"
      "ds_read_b32 %[p3], %[a3] offset:%[off]\n"
      "ds_read_b32 %[p4], %[a4] offset:%[off]\n"
      "ds_read_b32 %[p5], %[a5] offset:%[off]\n"
      "ds_read_b32 %[p6], %[a6] offset:%[off]\n"
      "ds_read_b32 %[p7], %[a7] offset:%[off]\n"
      "s_waitcnt lgkmcnt(0)\n"
      : [p0] "=&v"(p[0]), [p1] "=&v"(p[1]), [p2] "=&v"(p[2]), [p3] "=&v"(p[3]), [p4] "=&v"(p[4]), [p5] "=&v"(p[5]), [p6] "=&v"(p[6]), [p7] "=&v"(p[7]), [a0] "=&v"(a[0]), [a1] "=&v"(a[1]), [a2] "=&v"(a[2]), [a3] "=&v"(a[3]), [a4] "=&v"(a[4]), [a5] "=&v"(a[5]), [a6] "=&v"(a[6]), [a7] "=&v"(a[7])
      : [w0] "v"(w0), [w1] "v"(w1), [off] "i"(OFF), [tbl] "v"(tbl)
      : "memory");
}

// 8 index bytes (two dwords) -> 4 fp16 pairs from the 256-entry table at OFF.
template <int OFF>
__device__ __forceinline__ void dec4_byte(uint32_t w0, uint32_t w1, const uint32_t* tbl, uint32_t (&p)[4]) {
  uint32_t h[4], a[8];
  asm volatile(
      "v_lshlrev_b32_sdwa %[a0], 1, %[w0] dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_0\n"
      "v_lshlrev_b32_sdwa %[a1], 1, %[w0] dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_1\n"
      "v_lshlrev_b32_sdwa %[a2], 1, %[w0] dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_2\n"
      "v_lshlrev_b32_sdwa %[a3], 1, %[w0] dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_3\n"
      "v_lshlrev_b32_sdwa %[a4], 1, %[w1] dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_0\n"
      "v_lshlrev_b32_sdwa %[a5], 1, %[w1] dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_1\n"
      "v_lshlrev_b32_sdwa %[a6], 1, %[w1] dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_2\n"
      "v_lshlrev_b32_sdwa %[a7], 1, %[w1] dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_3\n"
      "ds_read_u16 %[p0], %[a0] offset:%[off]\n"
      "ds_read_u16 %[h0], %[a1] offset:%[off]\n"
      "ds_read_u16 %[p1], %[a2] offset:%[off]\n"
      "ds_read_u16 %[h1], %[a3] offset:%[off]\n"
      "ds_read_u16 %[p2], %[a4] offset:%[off]\n"
      "ds_read_u16 %[h2], %[a5] offset:%[off]\n"
      "ds_read_u16 %[p3], %[a6] offset:%[off]\n"
      "ds_read_u16 %[h3], %[a7] offset:%[off]\n"
      "s_waitcnt lgkmcnt(0)\n"
      "v_lshl_or_b32 %[p0], %[h0], 16, %[p0]\n"
      "v_lshl_or_b32 %[p1], %[h1], 16, %[p1]\n"
      "v_lshl_or_b32 %[p2], %[h2], 16, %[p2]\n"
      "v_lshl_or_b32 %[p3], %[h3], 16, %[p3]\n"
      : [p0] "=&v"(p[0]), [p1] "=&v"(p[1]), [p2] "=&v"(p[2]), [p3] "=&v"(p[3]), [h0] "=&v"(h[0]), [h1] "=&v"(h[1]), [h2] "=&v"(h[2]), [h3] "=&v"(h[3]), [a0] "=&v"(a[0]), [a1] "=&v"(a[1]), [a2] "=&v"(a[2]), [a3] "=&v"(a[3]), [a4] "=&v"(a[4]), [a5] "=&v"(a[5]), [a6] "=&v"(a[6]), [a7] "=&v"(a[7])
      : [w0] "v"(w0), [w1] "v"(w1), [off] "i"(OFF), [tbl] "v"(tbl)
      : "memory");
}

// Sum over the 64 lanes of a wave; the total lands in lane 63.
__device__ __forceinline__ float wave_sum_to_lane63(float v) {
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x141, 0xF, 0xF, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x140, 0xF, 0xF, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x142, 0xA, 0xF, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x143, 0xC, 0xF, false));
  return v;
}

// BITS 4 or 8; CPL 16-byte chunks per lane per row; PR rows per wave;
// DUAL: gate + up with the SwiGLU epilogue; NB batch vectors (1, 2 or 4).
template <int BITS, int CPL, int PR, bool DUAL, int NB>
__global__ __launch_bounds__(64) void k_gemv_wave(GemvArgs a) {
  constexpr int TBL_B = (2 << BITS);          // LUT bytes per row (32 or 512)
  constexpr int NM = DUAL ? 2 : 1;
  constexpr int XPC = (BITS == 4) ? 16 : 8;   // x dwords per chunk
  extern __shared__ uint32_t lds[];           // tables at LDS address 0 (layout below)

  const int lane = threadIdx.x;
  const uint32_t N = a.N, K = a.K;
  const uint32_t row_bytes = (BITS == 4) ? K / 2 : K;
  const uint32_t C = row_bytes / 16;
  const uint32_t row0 = blockIdx.x * PR;

  // ---- LUTs of the PR rows (contiguous PR*TBL_B bytes per matrix)
  constexpr int LUT_DW = PR * TBL_B / 4;                   // dwords per matrix
  constexpr int LUT_LD = (LUT_DW + 63) / 64;               // dwords per lane
  uint32_t lreg[NM][LUT_LD];
#pragma unroll
  for (int m = 0; m < NM; m++) {
    const uint32_t* lb = reinterpret_cast<const uint32_t*>(m == 0 ? a.lut : a.lut2);
#pragma unroll
    for (int i = 0; i < LUT_LD; i++) {
      const uint32_t d = (uint32_t)(lane + 64 * i);
      const uint32_t r = row0 + d / (TBL_B / 4);
      const uint32_t rc = r < N ? r : N - 1;
      lreg[m][i] = lb[(size_t)rc * (TBL_B / 4) + d % (TBL_B / 4)];
    }
  }

  // ---- x slice: chunks c_j = lane + 64 j
  uint32_t xr[NB][CPL][XPC];
#pragma unroll
  for (int j = 0; j < CPL; j++) {
    const uint32_t c = (uint32_t)(lane + 64 * j);
    const uint32_t cc = c < C ? c : C - 1;
#pragma unroll
    for (int b = 0; b < NB; b++) {
      const uint32_t bb = (uint32_t)b < a.nb ? (uint32_t)b : 0u;
      const uint4* xp = reinterpret_cast<const uint4*>(a.x + (size_t)bb * K + (size_t)cc * (XPC * 2));
#pragma unroll
      for (int q = 0; q < XPC / 4; q++) {
        const uint4 v = xp[q];
        xr[b][j][4 * q + 0] = v.x;
        xr[b][j][4 * q + 1] = v.y;
        xr[b][j][4 * q + 2] = v.z;
        xr[b][j][4 * q + 3] = v.w;
      }
    }
  }

  // ---- every index chunk of the PR rows, in row order
  uint4 iv[PR][NM][CPL];
#pragma unroll
  for (int r = 0; r < PR; r++) {
    const uint32_t row = row0 + r;
    const uint32_t rc = row < N ? row : N - 1;
#pragma unroll
    for (int m = 0; m < NM; m++) {
      const uint8_t* base = (m == 0 ? a.idx : a.idx2) + (size_t)rc * row_bytes;
#pragma unroll
      for (int j = 0; j < CPL; j++) {
        const uint32_t c = (uint32_t)(lane + 64 * j);
        const uint32_t cc = c < C ? c : C - 1;
        iv[r][m][j] = ld_stream(base + (size_t)cc * 16);
      }
    }
  }

  // ---- LUTs -> LDS.  Branch-free: lanes past the LUT write a scratch
  // slot above the tables, so the LUT loads stay first in issue order and
  // the wait for them does not wait for the index loads.
  // 4-bit: the staged 16-entry LUTs sit above the NM*PR pair tables and are
  // expanded into them; 8-bit: the 256-entry LUTs are the tables.
  constexpr int PAIR_DW = (BITS == 4) ? NM * PR * 256 : 0;
  uint32_t* stage = lds + PAIR_DW;
#pragma unroll
  for (int m = 0; m < NM; m++)
#pragma unroll
    for (int i = 0; i < LUT_LD; i++) {
      const int d = lane + 64 * i;
      stage[d < LUT_DW ? m * LUT_DW + d : NM * LUT_DW + lane] = lreg[m][i];
    }
  __syncthreads();
  if constexpr (BITS == 4) {
    // pair table t = m*PR + r: lane writes entries 4*lane .. 4*lane+3,
    // i.e. hi nibble lane>>2, lo nibbles 4*(lane&3) .. +3.
    const uint16_t* st16 = reinterpret_cast<const uint16_t*>(stage);
#pragma unroll
    for (int t = 0; t < NM * PR; t++) {
      const uint32_t hi = (uint32_t)st16[t * 16 + (lane >> 2)] << 16;
      const uint16_t* lo = st16 + t * 16 + 4 * (lane & 3);
      reinterpret_cast<uint4*>(lds + t * 256)[lane] =
          make_uint4(lo[0] | hi, lo[1] | hi, lo[2] | hi, lo[3] | hi);
    }
    __syncthreads();
  }

#pragma unroll
  for (int r = 0; r < PR; r++) {
    float acc[NM][NB];
#pragma unroll
    for (int m = 0; m < NM; m++)
#pragma unroll
      for (int b = 0; b < NB; b++) acc[m][b] = 0.0f;
#pragma unroll
    for (int m = 0; m < NM; m++) {
#pragma unroll
      for (int j = 0; j < CPL; j++) {
        const bool live = (uint32_t)(lane + 64 * j) < C;
        if (j == CPL - 1 && !live) continue;  // only the last chunk can be partial
        const uint32_t wv[4] = {iv[r][m][j].x, iv[r][m][j].y, iv[r][m][j].z, iv[r][m][j].w};
        if constexpr (BITS == 4) {
          uint32_t p[8];
#pragma unroll
          for (int q = 0; q < 4; q += 2) {
            // pair table of (matrix m, row r) at byte (m*PR + r)*1024
            switch (m * PR + r) {
#define PRISM_D4(o) \
  case o:           \
    dec8_pair<(o)*1024>(wv[q], wv[q + 1], lds, p); break;
              PRISM_D4(0) PRISM_D4(1) PRISM_D4(2) PRISM_D4(3) PRISM_D4(4) PRISM_D4(5) PRISM_D4(6) PRISM_D4(7)
#undef PRISM_D4
            }
#pragma unroll
            for (int e = 0; e < 8; e++)
#pragma unroll
              for (int b = 0; b < NB; b++) acc[m][b] = dot2(p[e], xr[b][j][4 * q + e], acc[m][b]);
          }
        } else {
          uint32_t p[4];
#pragma unroll
          for (int q = 0; q < 4; q += 2) {
            switch (m * PR + r) {
#define PRISM_D8(o) \
  case o:           \
    dec4_byte<(o)*512>(wv[q], wv[q + 1], lds, p); break;
              PRISM_D8(0) PRISM_D8(1) PRISM_D8(2) PRISM_D8(3) PRISM_D8(4) PRISM_D8(5) PRISM_D8(6) PRISM_D8(7)
#undef PRISM_D8
            }
#pragma unroll
            for (int e = 0; e < 4; e++)
#pragma unroll
              for (int b = 0; b < NB; b++) acc[m][b] = dot2(p[e], xr[b][j][2 * q + e], acc[m][b]);
          }
        }
      }
    }
#pragma unroll
    for (int m = 0; m < NM; m++)
#pragma unroll
      for (int b = 0; b < NB; b++) acc[m][b] = wave_sum_to_lane63(acc[m][b]);
    const uint32_t row = row0 + r;
    if (lane == 63 && row < N) {
      if constexpr (DUAL) {
        a.y[row] = swiglu_h(acc[0][0], acc[NM - 1][0]);
      } else {
#pragma unroll
        for (int b = 0; b < NB; b++)
          if ((uint32_t)b < a.nb) a.y[(size_t)b * N + row] = f2h(acc[0][b]);
      }
    }
  }
}

template <int BITS, int CPL, int PR, bool DUAL, int NB>
constexpr size_t gemv_wave_lds_bytes() {
  // [4-bit pair tables] + staged / 8-bit LUTs + per-lane scratch slot
  return (size_t)(DUAL ? 2 : 1) * PR * ((BITS == 4 ? 1024 : 0) + (2 << BITS)) + 64 * 4;
}

}  // namespace prism
