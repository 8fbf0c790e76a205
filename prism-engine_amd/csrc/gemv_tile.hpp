// gemv_tile.hpp -- palettized GEMV for gfx950: one workgroup per R rows,
// K split across the workgroup's lanes.
//
// y[b, r] = f16( sum_k f32(x[b, k]) * f32(LUT_r[idx(r, k)]) ) over
// split-block weights, the arithmetic of lut_gemv_cpu
// (compute-core/src/lut/evaluator.rs:21-44); DUAL computes gate and up rows
// together and applies the SwiGLU epilogue (evaluator.rs:78-83,209-225).
//
// Work layout (T = 64*W threads, W = blockDim.x / 64 chosen by the host):
//  * a row is cut into 8-element units (4 index bytes at 4 bits, 8 at
//    8 bits; 16 bytes of x).  Thread `tid` owns units u = tid + T*t,
//    t < UPL, of each of the workgroup's R rows, so every global load is
//    contiguous across the wave (x: 16 bytes per lane, indices 4 or 8);
//  * x is read once per workgroup for R rows (2*K/R bytes per row).  All
//    workgroups read the same x, so its re-reads land on a few L2 channels;
//    keeping them well below the streamed index bytes matters;
//  * the LUT dwords, the x units and every index unit of the R rows are
//    issued up front (straight-line code), so the compiler counts them with
//    vmcnt and each row is decoded as soon as its bytes land; x and index
//    loads are buffer loads whose whole offset (row, unit) is the per-lane
//    VGPR offset: the descriptor's range check covers the VGPR and
//    immediate offsets only, never the scalar one, so a unit past the end
//    of x or of the index block reads as 0 only because its offset is
//    there;
//  * lookup tables live in LDS at fixed addresses (table t at byte t*1024),
//    built once per workgroup:
//      4-bit: pair table, entry b = LUT[b & 15] | LUT[b >> 4] << 16, so one
//             index byte is one SDWA shift (byte k -> 4*b) and one
//             ds_read_b32 giving the fp16 pair for v_dot2_f32_f16;
//      8-bit: expanded table, entry b = LUT[b] in the low half of a dword,
//             one SDWA shift and one ds_read_b32 per byte, two entries
//             packed per v_perm;
//    the reads are plain LDS loads, so the compiler keeps many in flight
//    and waits with partial lgkmcnt counts;
//  * each wave reduces its R partial sums with DPP into lane 63, which
//    writes them to LDS; R*NB threads add the W wave totals and round once
//    (RNE).
// Only the last unit pass can be partial (U % T live threads); those lanes
// skip it.  Requires K % 8 == 0, 16-byte aligned x rows and an index block
// (N * row bytes) below 2 GiB, so buffer offsets stay in 31 bits.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "gemv_kernels.hpp"
#include "step_kernels.hpp"

namespace prism {

// byte K of w shifted left by S: the LDS byte offset of table entry b for
// 4-byte (S = 2) entries.  SDWA selects the byte inside the shift.
#define PRISM_SDWA_SHL(S, K) \
  "v_lshlrev_b32_sdwa %0, " #S ", %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_" #K
template <int K>
__device__ __forceinline__ uint32_t byte_x4(uint32_t w) {
  uint32_t a;
  if constexpr (K == 0) asm(PRISM_SDWA_SHL(2, 0) : "=v"(a) : "v"(w));
  if constexpr (K == 1) asm(PRISM_SDWA_SHL(2, 1) : "=v"(a) : "v"(w));
  if constexpr (K == 2) asm(PRISM_SDWA_SHL(2, 2) : "=v"(a) : "v"(w));
  if constexpr (K == 3) asm(PRISM_SDWA_SHL(2, 3) : "=v"(a) : "v"(w));
  return a;
}
#undef PRISM_SDWA_SHL

// 4 lookups (one per byte of w) into the dword table at `tbl`.
__device__ __forceinline__ void look4(uint32_t w, const uint32_t* tbl, uint32_t (&p)[4]) {
  const char* b = reinterpret_cast<const char*>(tbl);
  p[0] = *reinterpret_cast<const uint32_t*>(b + byte_x4<0>(w));
  p[1] = *reinterpret_cast<const uint32_t*>(b + byte_x4<1>(w));
  p[2] = *reinterpret_cast<const uint32_t*>(b + byte_x4<2>(w));
  p[3] = *reinterpret_cast<const uint32_t*>(b + byte_x4<3>(w));
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

// Prologue / epilogue options of k_gemv_tile (bit flags; NB must be 1):
//  kEpiNorm  x is RMS-normalised first, rms_norm_inplace
//            (compute-core/src/lut/evaluator.rs:49-64) without a norm
//            weight: inv = 1 / sqrt(sum(x^2) / K + eps), x <- f16(x * inv).
//            Every workgroup holds all of x across its lanes, so it sums the
//            squares of its own units and reduces across its waves.
//  kEpiResid y is the residual stream, updated in place:
//            y[row] <- f16(f16(acc) + y[row]) (vec_add_inplace after the
//            projection, src/lut/engine_impl.rs:1158-1162,1208-1213).
//  kEpiAttnIn x is the attention output of the decode step, given as the
//            split partials of k_step_attention (a.xpart, [K/64 heads]
//            [kAttnSplits][2 + 64] fp32): each thread combines its own units
//            (head u/8, dims 8*(u%8)..+7) and rounds them to fp16: the
//            attention output of attention_cpu (evaluator.rs:104-146).
//  kEpiPair  DUAL only: instead of the SwiGLU epilogue, the raw gate and up
//            outputs y[row] = f16(gate), y2[row] = f16(up) (the outputs of
//            templates/fused_gate_up.metal:16-97; the CPU path computes them
//            as two lut_gemv_cpu calls).
constexpr int kEpiNorm = 1;
constexpr int kEpiResid = 2;
constexpr int kEpiAttnIn = 4;
constexpr int kEpiPair = 8;

// Index loads stream (nontemporal) except in the decode step's per-layer
// projections (norm / residual / attention-input options, 2 rows per
// workgroup): those weights are re-read every token, and keeping them
// cacheable measured 1792 against 1745 tokens/s on the Qwen2.5-0.5B step
// (its LM head, R = 4, still streams).
template <int EPI, int R>
constexpr int tile_index_aux() {
  return ((EPI & ~kEpiPair) != 0 && R == 2) ? 0 : kNontemporal;
}

// Minimum threads per workgroup by index width: the 8-bit LUT loads are
// laid out for at least 256 threads (fewer still work, with more loads).
template <int BITS>
constexpr int tile_min_threads() {
  return BITS == 4 ? 64 : 256;
}

// LDS bytes for one workgroup of `threads` threads.
template <int BITS, int R, bool DUAL, int NB>
constexpr size_t gemv_tile_lds_bytes(int threads) {
  constexpr int NT = (DUAL ? 2 : 1) * R;
  const size_t tables = (size_t)NT * 256;
  const size_t stage = (BITS == 4) ? (size_t)NT * 8 + threads : (size_t)2 * threads;
  const size_t parts = (size_t)(threads / 64) * NT * NB;
  const size_t norm = (size_t)(threads / 64);
  return 4 * (tables + stage + parts + norm);
}

// LDS bytes of one wave's region when WI > 1 independent waves share a
// workgroup (16-byte aligned: the tables are written as uint4).
template <int BITS, int R, bool DUAL, int NB>
constexpr size_t gemv_tile_wave_lds_bytes() {
  return (gemv_tile_lds_bytes<BITS, R, DUAL, NB>(64) + 15) & ~(size_t)15;
}

// Orders a workgroup's LDS writes before its reads.  With WI > 1 every wave
// works on its own rows in its own LDS region, so waiting for the wave's own
// LDS operations is enough and the waves never wait for each other.
template <int WI>
__device__ __forceinline__ void tile_sync() {
  if constexpr (WI > 1)
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  else
    __syncthreads();
}

// WI > 1: WI independent one-wave tiles per workgroup (wave v takes rows
// (WI blockIdx.x + v) R ..), for matrices whose many small tiles would
// otherwise cost more to dispatch than to run.
template <int BITS, int UPL, int R, bool DUAL, int NB, int EPI = 0, int WI = 1>
__global__ __launch_bounds__(512) void k_gemv_tile(GemvArgs a) {
  static_assert(EPI == 0 || NB == 1, "norm / residual options are single-vector");
  static_assert((EPI & kEpiPair) == 0 || DUAL, "the pair epilogue is gate + up");
  constexpr int NM = DUAL ? 2 : 1;
  constexpr int NT = NM * R;                 // lookup tables (matrix-major)
  constexpr int IW = (BITS == 4) ? 1 : 2;    // index dwords per unit
  constexpr int LUT_DW = (BITS == 4) ? 8 : 128;  // LUT dwords per row
  static_assert(NT <= 16, "table offsets must stay within 16 KB");
  extern __shared__ uint32_t lds_all[];      // dynamic LDS only: starts at address 0
  // LDS: [NT tables x 256 dwords][4-bit: NT*8 staged LUT dwords + T scratch |
  //       8-bit: 2T scratch][W * NT * NB partial sums][W norm partials]

  const int T = WI > 1 ? 64 : (int)blockDim.x;
  const int W = T >> 6;
  const int tid = WI > 1 ? (int)(threadIdx.x & 63) : (int)threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const uint32_t vw = WI > 1 ? threadIdx.x >> 6 : 0u;  // this wave's tile in the workgroup
  uint32_t* lds = lds_all + vw * (uint32_t)(gemv_tile_wave_lds_bytes<BITS, R, DUAL, NB>() / 4);
  const uint32_t N = a.N, K = a.K;
  const uint32_t U = K / 8;
  const uint32_t row_dw = U * IW;
  const uint32_t row0 = (blockIdx.x * WI + vw) * R;
  uint32_t* stage = lds + NT * 256;
  float* part = reinterpret_cast<float*>(stage + ((BITS == 4) ? NT * 8 + T : 2 * T));
  float* nsum = part + W * NT * NB;

  // ---- LUT dwords of the NT rows (matrix-major, contiguous per matrix)
  constexpr int LUT_TOTAL = NT * LUT_DW;
  constexpr int LUT_LD = (LUT_TOTAL + tile_min_threads<BITS>() - 1) / tile_min_threads<BITS>();
  uint32_t lreg[LUT_LD];
#pragma unroll
  for (int i = 0; i < LUT_LD; i++) {
    const uint32_t d = (uint32_t)(tid + T * i);
    const uint32_t dc = d < (uint32_t)LUT_TOTAL ? d : (uint32_t)LUT_TOTAL - 1;
    const uint32_t m = dc / (R * LUT_DW), dd = dc % (R * LUT_DW);
    const uint32_t r = row0 + dd / LUT_DW;
    const uint32_t rc = r < N ? r : N - 1;
    const uint32_t* lb = reinterpret_cast<const uint32_t*>(m == 0 ? a.lut : a.lut2);
    lreg[i] = lb[(size_t)rc * LUT_DW + dd % LUT_DW];
  }

  // ---- x units and the index units of the R rows, as buffer loads.  The
  // row and unit offsets go in the VGPR offset (the compiler moves constant
  // parts to the immediate field), which the descriptor's range check
  // covers; the scalar offset, which it does not cover, stays 0.  So a unit
  // past the end of x or of the index block reads as 0 and touches no
  // memory; lanes past the row's last unit never use theirs.  Index loads:
  // tile_index_aux.
  typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
  typedef uint32_t u32x4v_t __attribute__((ext_vector_type(4)));
  uint32_t xr[NB][UPL][4];
  if constexpr ((EPI & kEpiAttnIn) != 0) {
#pragma unroll
    for (int t = 0; t < UPL; t++) {
      const uint32_t u = (uint32_t)(tid + T * t);
      const uint32_t cu = u < U ? u : U - 1;
      const float* hp = a.xpart + (size_t)(cu / 8) * kAttnSplits * 66;
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const uint32_t lo = f2h(attn_combine(hp, 8 * (cu % 8) + 2 * e));
        const uint32_t hi = f2h(attn_combine(hp, 8 * (cu % 8) + 2 * e + 1));
        xr[0][t][e] = lo | (hi << 16);
      }
    }
  } else
#pragma unroll
  for (int b = 0; b < NB; b++) {
    const uint32_t bb = (uint32_t)b < a.nb ? (uint32_t)b : 0u;
    const __amdgpu_buffer_rsrc_t rx =
        __builtin_amdgcn_make_buffer_rsrc((void*)(a.x + (size_t)bb * K), (short)0, (int)(K * 2), kBufferWord3);
#pragma unroll
    for (int t = 0; t < UPL; t++) {
      const u32x4v_t v = __builtin_amdgcn_raw_buffer_load_b128(rx, (uint32_t)(tid + T * t) * 16u, 0u, 0);
      xr[b][t][0] = v.x;
      xr[b][t][1] = v.y;
      xr[b][t][2] = v.z;
      xr[b][t][3] = v.w;
    }
  }

  uint32_t iv[R][NM][UPL][IW];
  __amdgpu_buffer_rsrc_t ri[NM];
#pragma unroll
  for (int m = 0; m < NM; m++)
    ri[m] = __builtin_amdgcn_make_buffer_rsrc((void*)(m == 0 ? a.idx : a.idx2), (short)0, (int)(N * row_dw * 4u),
                                              kBufferWord3);
#pragma unroll
  for (int r = 0; r < R; r++) {
    const uint32_t row = row0 + r;
    const uint32_t rc = row < N ? row : N - 1;
#pragma unroll
    for (int m = 0; m < NM; m++) {
#pragma unroll
      for (int t = 0; t < UPL; t++) {
        const uint32_t vo = rc * row_dw * 4u + (uint32_t)(tid + T * t) * (4u * IW);
        if constexpr (IW == 1) {
          iv[r][m][t][0] = __builtin_amdgcn_raw_buffer_load_b32(ri[m], vo, 0u, tile_index_aux<EPI, R>());
        } else {
          const u32x2_t v = __builtin_amdgcn_raw_buffer_load_b64(ri[m], vo, 0u, kNontemporal);
          iv[r][m][t][0] = v.x;
          iv[r][m][t][1] = v.y;
        }
      }
    }
  }

  // ---- lookup tables.  Stores are branch-free: threads whose load index is
  // past the LUTs write their scratch slot, so the LUT loads stay first in
  // issue order and waiting for them does not wait for the index loads.
  if constexpr (BITS == 4) {
#pragma unroll
    for (int i = 0; i < LUT_LD; i++) {
      const int d = tid + T * i;
      stage[d < LUT_TOTAL ? d : LUT_TOTAL + tid] = lreg[i];
    }
    tile_sync<WI>();
    // table t, uint4 q = entries 4q .. 4q+3 = {LUT[4(q&3) + i] | LUT[q>>2] << 16}
    const uint16_t* st16 = reinterpret_cast<const uint16_t*>(stage);
    for (int i = tid; i < NT * 64; i += T) {
      const int t = i >> 6, q = i & 63;
      const uint32_t hi = st16[t * 16 + (q >> 2)];
      const uint2 lo = *reinterpret_cast<const uint2*>(st16 + t * 16 + 4 * (q & 3));
      reinterpret_cast<uint4*>(lds + t * 256)[q] =
          make_uint4(__builtin_amdgcn_perm(hi, lo.x, 0x05040100u), __builtin_amdgcn_perm(hi, lo.x, 0x05040302u),
                     __builtin_amdgcn_perm(hi, lo.y, 0x05040100u), __builtin_amdgcn_perm(hi, lo.y, 0x05040302u));
    }
  } else {
    // LUT dword d of table t holds entries 2d, 2d+1 -> expanded dwords 2d, 2d+1
#pragma unroll
    for (int i = 0; i < LUT_LD; i++) {
      const int d = tid + T * i;
      const int t = d / LUT_DW, e = d % LUT_DW;
      uint2* dst = reinterpret_cast<uint2*>(d < LUT_TOTAL ? lds + t * 256 + 2 * e : stage + 2 * tid);
      *dst = make_uint2(lreg[i] & 0xFFFFu, lreg[i] >> 16);
    }
  }
  tile_sync<WI>();

  const bool last_live = (uint32_t)(tid + T * (UPL - 1)) < U;
  if constexpr ((EPI & kEpiNorm) != 0) {
    // sum of squares of this thread's units; a unit past K is skipped (its
    // load already read 0 through the range check)
    float ss = 0.0f;
#pragma unroll
    for (int t = 0; t < UPL; t++)
#pragma unroll
      for (int e = 0; e < 4; e++) {
        if (t == UPL - 1 && !last_live) continue;
        const float lo = h2f((uint16_t)(xr[0][t][e] & 0xFFFFu)), hi = h2f((uint16_t)(xr[0][t][e] >> 16));
        ss += lo * lo;
        ss += hi * hi;
      }
    ss = wave_sum_to_lane63(ss);
    if (lane == 63) nsum[wave] = ss;
    tile_sync<WI>();
    float tot = 0.0f;
    for (int w = 0; w < W; w++) tot += nsum[w];
    const float inv = 1.0f / sqrtf(tot / (float)K + a.eps);
#pragma unroll
    for (int t = 0; t < UPL; t++)
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const uint32_t lo = f2h(h2f((uint16_t)(xr[0][t][e] & 0xFFFFu)) * inv);
        const uint32_t hi = f2h(h2f((uint16_t)(xr[0][t][e] >> 16)) * inv);
        xr[0][t][e] = lo | (hi << 16);
      }
  }

  float acc[R][NM][NB];
#pragma unroll
  for (int r = 0; r < R; r++) {
#pragma unroll
    for (int m = 0; m < NM; m++) {
      const uint32_t* tbl = lds + (m * R + r) * 256;
#pragma unroll
      for (int b = 0; b < NB; b++) acc[r][m][b] = 0.0f;
#pragma unroll
      for (int t = 0; t < UPL; t++) {
        if (t == UPL - 1 && !last_live) continue;
        uint32_t p[4];
        if constexpr (BITS == 4) {
          look4(iv[r][m][t][0], tbl, p);  // fp16 pairs of elements (0,1) (2,3) (4,5) (6,7)
        } else {
          uint32_t e0[4], e1[4];
          look4(iv[r][m][t][0], tbl, e0);
          look4(iv[r][m][t][1], tbl, e1);
          p[0] = __builtin_amdgcn_perm(e0[1], e0[0], 0x05040100u);
          p[1] = __builtin_amdgcn_perm(e0[3], e0[2], 0x05040100u);
          p[2] = __builtin_amdgcn_perm(e1[1], e1[0], 0x05040100u);
          p[3] = __builtin_amdgcn_perm(e1[3], e1[2], 0x05040100u);
        }
#pragma unroll
        for (int e = 0; e < 4; e++)
#pragma unroll
          for (int b = 0; b < NB; b++) acc[r][m][b] = dot2(p[e], xr[b][t][e], acc[r][m][b]);
      }
    }
  }

  // ---- wave totals -> LDS -> workgroup totals
#pragma unroll
  for (int r = 0; r < R; r++)
#pragma unroll
    for (int m = 0; m < NM; m++)
#pragma unroll
      for (int b = 0; b < NB; b++) {
        const float v = wave_sum_to_lane63(acc[r][m][b]);
        if (lane == 63) part[((wave * R + r) * NM + m) * NB + b] = v;
      }
  tile_sync<WI>();
  if (tid < R * NB) {
    const int r = tid / NB, b = tid % NB;
    const uint32_t row = row0 + r;
    float s[NM];
#pragma unroll
    for (int m = 0; m < NM; m++) {
      s[m] = 0.0f;
      for (int w = 0; w < W; w++) s[m] += part[((w * R + r) * NM + m) * NB + b];
    }
    if (row < N && (uint32_t)b < a.nb) {
      if constexpr (DUAL && (EPI & kEpiPair) != 0) {
        a.y[row] = f2h(s[0]);
        a.y2[row] = f2h(s[NM - 1]);
      } else if constexpr (DUAL)
        a.y[row] = swiglu_h(s[0], s[NM - 1]);
      else if constexpr ((EPI & kEpiResid) != 0)
        a.y[row] = f2h(h2f(f2h(s[0])) + h2f(a.y[row]));
      else
        a.y[(size_t)b * N + row] = f2h(s[0]);
    }
  }
}

}  // namespace prism
