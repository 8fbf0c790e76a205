// gemv_kernels.hpp -- palettized-LUT GEMV kernels for gfx950 (CDNA4, wave64).
//
// Computes y[b, r] = f16( sum_k f32(x[b, k]) * f32(LUT_r[idx(r, k)]) ), the
// arithmetic of lut_gemv_cpu (compute-core/src/lut/evaluator.rs:21-44), over
// split-block weights (src/lut/compiler.rs:50-61).  The decode GEMV is
// HBM-bound: every index byte and LUT byte is read exactly once per launch
// and the per-element work is kept to an LDS table lookup plus half of a
// v_dot2_f32_f16.
//
// Work layout of the fast kernel (k_gemv):
//   * a workgroup is KW waves; all of them work on the same RPW = 64/G rows
//     per pass, G lanes per row inside each wave, the KW waves splitting K;
//   * a row's index bytes are cut into 16-byte chunks (32 nibbles or 16
//     bytes); lane (wave w, lane-in-row g) owns chunks c = w*G + g + j*KW*G,
//     j < CPL, so its slice of x is fixed for the whole launch and is held
//     in VGPRs (loaded once), packed as fp16 pairs;
//   * each chunk is one 16-byte (dwordx4) load; consecutive lanes read
//     consecutive chunks of a row, so a wave reads G*16 contiguous bytes per
//     row and instruction;
//   * the RPW rows' LUTs are staged in LDS (double-buffered, the next pass's
//     LUT bytes are loaded while the current pass computes) and looked up
//     with ds_read_u16 -- 16 fp16 entries of a row sit in 8 consecutive
//     dwords, so a wave's lookups into one row never bank-conflict;
//   * decoded pairs feed v_dot2_f32_f16 (exact fp16 products, fp32 sums);
//   * the partial sums of a row are reduced across its G lanes with xor
//     shuffles and across the KW waves through LDS, then rounded to fp16
//     (round-to-nearest-even) once.
// Rows are visited with a grid-stride loop over passes; the index loads of
// the next pass are issued before the current pass is computed.
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
__device__ __forceinline__ uint16_t f2h(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }

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
  uint32_t N;
  uint32_t K;
  uint32_t nb;          // live batch rows (<= NB)
};

// BITS: 4 or 8.  NB: compile-time batch capacity.  G: lanes per row (64,
// 32, 16).  CPL: chunks per lane.  KW: waves per workgroup splitting K.
// DUAL: gate+up with SwiGLU epilogue (NB must be 1).
template <int BITS, int NB, int G, int CPL, int KW, bool DUAL>
__global__ __launch_bounds__(64 * KW) void k_gemv(GemvArgs a) {
  constexpr int RPW = 64 / G;                      // rows per pass
  constexpr int NT = 64 * KW;                      // threads
  constexpr int TBL = 1 << BITS;                   // LUT entries per row
  constexpr int TBL_DW = TBL / 2;                  // dwords per row LUT
  constexpr int NM = DUAL ? 2 : 1;                 // matrices
  constexpr int XPC = (BITS == 4) ? 16 : 8;        // x dwords (fp16 pairs) per chunk
  constexpr int LUT_U4 = RPW * TBL_DW / 4;         // uint4 per pass per matrix (8-bit)
  constexpr int LUT_LD = (BITS == 4) ? 1 : (LUT_U4 + NT - 1) / NT;  // staging regs per thread

  __shared__ uint32_t s_tbl[2][NM][RPW][TBL_DW];
  __shared__ float s_red[(KW > 1) ? KW : 1][RPW][NB * NM];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int rig = lane / G;          // row in pass
  const int gl = lane % G;           // lane within row
  const uint32_t N = a.N, K = a.K;
  const uint32_t row_bytes = K * BITS / 8;
  const uint32_t C = row_bytes / 16;
  const uint32_t npass = (N + RPW - 1) / RPW;

  // ---- x slice in registers (fp16 pairs), zero for chunks past the row
  uint32_t xr[NB][CPL][XPC];
#pragma unroll
  for (int j = 0; j < CPL; j++) {
    const uint32_t c = (uint32_t)(wave * G + gl + j * KW * G);
#pragma unroll
    for (int b = 0; b < NB; b++) {
      const bool live = (c < C) && ((uint32_t)b < a.nb);
      const uint4* xp = reinterpret_cast<const uint4*>(a.x + (size_t)b * K + (size_t)c * (XPC * 2));
#pragma unroll
      for (int q = 0; q < XPC / 4; q++) {
        uint4 v = live ? xp[q] : make_uint4(0, 0, 0, 0);
        xr[b][j][4 * q + 0] = v.x;
        xr[b][j][4 * q + 1] = v.y;
        xr[b][j][4 * q + 2] = v.z;
        xr[b][j][4 * q + 3] = v.w;
      }
    }
  }

  // ---- per-pass loads: index chunks and this thread's share of the LUTs
  auto load_idx = [&](uint32_t pass, uint4 (&dst)[NM][CPL]) {
    const uint32_t row = pass * RPW + rig;
#pragma unroll
    for (int m = 0; m < NM; m++) {
      const uint8_t* base = (m == 0 ? a.idx : a.idx2) + (size_t)row * row_bytes;
#pragma unroll
      for (int j = 0; j < CPL; j++) {
        const uint32_t c = (uint32_t)(wave * G + gl + j * KW * G);
        dst[m][j] = (row < N && c < C) ? ld_stream(base + (size_t)c * 16)
                                       : make_uint4(0, 0, 0, 0);
      }
    }
  };
  // LUT staging: 4-bit -> thread t < RPW*8 loads dword t of the pass's
  // 32*RPW contiguous LUT bytes; 8-bit -> uint4 slots t, t+NT, ...
  auto load_lut = [&](uint32_t pass, uint4 (&dst)[NM][LUT_LD]) {
#pragma unroll
    for (int m = 0; m < NM; m++) {
      const uint8_t* lb = (m == 0 ? a.lut : a.lut2);
      if (BITS == 4) {
        const uint32_t r = pass * RPW + (uint32_t)(tid >> 3);
        const bool live = tid < RPW * 8 && r < N;
        dst[m][0].x = live ? reinterpret_cast<const uint32_t*>(lb + (size_t)r * 32)[tid & 7] : 0u;
      } else {
#pragma unroll
        for (int i = 0; i < LUT_LD; i++) {
          const int s = tid + i * NT;               // uint4 slot in the pass's LUT block
          const uint32_t r = pass * RPW + (uint32_t)(s / (TBL_DW / 4));
          const bool live = s < LUT_U4 && r < N;
          dst[m][i] = live ? reinterpret_cast<const uint4*>(lb + (size_t)pass * RPW * 512)[s]
                           : make_uint4(0, 0, 0, 0);
        }
      }
    }
  };
  auto store_lut = [&](int buf, const uint4 (&src)[NM][LUT_LD]) {
#pragma unroll
    for (int m = 0; m < NM; m++) {
      if (BITS == 4) {
        if (tid < RPW * 8) (&s_tbl[buf][m][0][0])[tid] = src[m][0].x;
      } else {
#pragma unroll
        for (int i = 0; i < LUT_LD; i++) {
          const int s = tid + i * NT;
          if (s < LUT_U4) reinterpret_cast<uint4*>(&s_tbl[buf][m][0][0])[s] = src[m][i];
        }
      }
    }
  };

  uint32_t pass = blockIdx.x;
  if (pass >= npass) return;  // uniform over the workgroup
  uint4 cur[NM][CPL];
  uint4 lst[NM][LUT_LD];
  load_idx(pass, cur);
  load_lut(pass, lst);
  store_lut(0, lst);
  __syncthreads();

  int buf = 0;
  for (;;) {
    const uint32_t next = pass + gridDim.x;
    const bool more = next < npass;  // uniform
    uint4 nxt[NM][CPL];
    if (more) {
      load_idx(next, nxt);
      load_lut(next, lst);
    }

    float acc[NM][NB];
#pragma unroll
    for (int m = 0; m < NM; m++)
#pragma unroll
      for (int b = 0; b < NB; b++) acc[m][b] = 0.0f;

#pragma unroll
    for (int m = 0; m < NM; m++) {
      const uint16_t* tb = reinterpret_cast<const uint16_t*>(&s_tbl[buf][m][rig][0]);
#pragma unroll
      for (int j = 0; j < CPL; j++) {
        const uint32_t wv[4] = {cur[m][j].x, cur[m][j].y, cur[m][j].z, cur[m][j].w};
#pragma unroll
        for (int q = 0; q < 4; q++) {
          const uint32_t w = wv[q];
          if (BITS == 4) {
            // 8 nibbles -> 4 fp16 pairs (element 2i = low nibble of byte i)
#pragma unroll
            for (int p = 0; p < 4; p++) {
              const uint32_t lo = tb[(w >> (8 * p)) & 15u];
              const uint32_t hi = tb[(w >> (8 * p + 4)) & 15u];
              const uint32_t pr = lo | (hi << 16);
#pragma unroll
              for (int b = 0; b < NB; b++) acc[m][b] = dot2(pr, xr[b][j][4 * q + p], acc[m][b]);
            }
          } else {
            // 4 bytes -> 2 fp16 pairs
#pragma unroll
            for (int p = 0; p < 2; p++) {
              const uint32_t lo = tb[(w >> (16 * p)) & 255u];
              const uint32_t hi = tb[(w >> (16 * p + 8)) & 255u];
              const uint32_t pr = lo | (hi << 16);
#pragma unroll
              for (int b = 0; b < NB; b++) acc[m][b] = dot2(pr, xr[b][j][2 * q + p], acc[m][b]);
            }
          }
        }
      }
    }

    // ---- reduce over the row's lanes, then over the KW waves
#pragma unroll
    for (int m = 0; m < NM; m++)
#pragma unroll
      for (int b = 0; b < NB; b++) acc[m][b] = group_sum<G>(acc[m][b]);

    if (more) store_lut(buf ^ 1, lst);

    const uint32_t row = pass * RPW + rig;
    if (KW > 1) {
      if (gl == 0) {
#pragma unroll
        for (int m = 0; m < NM; m++)
#pragma unroll
          for (int b = 0; b < NB; b++) s_red[wave][rig][m * NB + b] = acc[m][b];
      }
      __syncthreads();
      if (wave == 0 && gl == 0 && row < N) {
#pragma unroll
        for (int m = 0; m < NM; m++)
#pragma unroll
          for (int b = 0; b < NB; b++) {
            float s = 0.0f;
#pragma unroll
            for (int w2 = 0; w2 < KW; w2++) s += s_red[w2][rig][m * NB + b];
            acc[m][b] = s;
          }
      }
    }
    if (wave == 0 && gl == 0 && row < N) {
      if (DUAL) {
        a.y[row] = swiglu_h(acc[0][0], acc[NM - 1][0]);
      } else {
#pragma unroll
        for (int b = 0; b < NB; b++)
          if ((uint32_t)b < a.nb) a.y[(size_t)b * N + row] = f2h(acc[0][b]);
      }
    }
    __syncthreads();  // next LUT visible; s_tbl[buf] / s_red free for reuse
    if (!more) break;
    pass = next;
    buf ^= 1;
#pragma unroll
    for (int m = 0; m < NM; m++)
#pragma unroll
      for (int j = 0; j < CPL; j++) cur[m][j] = nxt[m][j];
  }
}

// Generic kernel for shapes the fast kernel does not take (rows whose byte
// length is not a multiple of 16, or unaligned x): one wave per row,
// element-strided.  Follows lut_gemv_cpu's ragged-K rule for 4-bit weights:
// row stride K/2 bytes, only the first (K/8)*8 elements contribute.
template <int BITS, bool DUAL>
__global__ __launch_bounds__(64) void k_gemv_generic(GemvArgs a) {
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
      const uint8_t* lut = (m == 0 ? a.lut : a.lut2) + (size_t)row * (2u << BITS);
      const uint8_t* idx = (m == 0 ? a.idx : a.idx2) + (size_t)row * stride;
      float s = 0.0f;
      for (uint32_t k = lane; k < keff; k += 64) {
        uint32_t e;
        if (BITS == 4) {
          const uint8_t byte = idx[k >> 1];
          e = (k & 1) ? (byte >> 4) : (byte & 15u);
        } else {
          e = idx[k];
        }
        const uint16_t lv = (uint16_t)(lut[2 * e] | (lut[2 * e + 1] << 8));
        s += h2f(a.x[(size_t)b * K + k]) * h2f(lv);
      }
      acc[m] = group_sum<64>(s);
    }
    if (lane == 0) {
      if (DUAL)
        a.y[row] = swiglu_h(acc[0], acc[NM - 1]);
      else
        a.y[(size_t)b * N + row] = f2h(acc[0]);
    }
  }
}

// Dense decode of rows [row0, row0+nrows): out[i][k] = LUT_r[idx(r, k)]
// (the per-row form of lut_embed, compute-core/src/lut/evaluator.rs:176-197).
// For 4-bit weights elements at k >= (K/8)*8 are written as 0, matching
// lut_embed's shorter output zero-padded.
template <int BITS>
__global__ __launch_bounds__(256) void k_decode_rows(const uint8_t* lut, const uint8_t* idx, uint32_t N,
                                                     uint32_t K, uint32_t row0, uint32_t nrows, uint16_t* out) {
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
        const uint8_t byte = idx[(size_t)r * stride + (k >> 1)];
        e = (k & 1) ? (byte >> 4) : (byte & 15u);
      } else {
        e = idx[(size_t)r * stride + k];
      }
      const uint8_t* l = lut + (size_t)r * (2u << BITS) + 2 * e;
      v = (uint16_t)(l[0] | (l[1] << 8));
    }
    out[t] = v;
  }
}

}  // namespace prism
