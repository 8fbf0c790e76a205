// gemm_kernels.hpp -- palettized prefill GEMM for gfx950 (MFMA fp16 -> fp32).
//
// Y[M x N] = X[M x K] . W^T with W[N x K] palettized (split-block), fp32
// accumulation and fp16 (RNE) output: M independent lut_gemv_cpu rows
// (compute-core/src/lut/evaluator.rs:21-44); the reference's own GEMM
// template (templates/palettized_gemm.metal) is never dispatched.
//
// Block tile BM x BN = 128 x 128, K step 32, 256 threads (4 waves as 2 x 2,
// 64 x 64 per wave = 2 x 2 v_mfma_f32_32x32x16_f16 tiles).
//  * The block's 128 row LUTs are copied to LDS once (4-bit: 4 KB, 8-bit:
//    64 KB) and stay there for the whole K loop.
//  * Each K step, the 128 x 32 index tile is decoded through those LUTs
//    straight into an LDS fp16 tile (the MFMA B operand), and the X tile is
//    copied to LDS; both tiles use an 80-byte row pitch so the 16-byte
//    fragment reads of 8 consecutive rows hit 32 distinct banks.
//  * The next step's global loads are issued before the current step's
//    MFMAs (register double buffering).
//  * Blocks are mapped XCD-aware: hardware dispatches block b to XCD b % 8;
//    the remap gives each XCD a contiguous range of tiles (N-fastest) so the
//    W tiles and X rows one XCD works on stay in its own L2.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>
#include <utility>

#include "gemv_lpr.hpp"
#include "lut_perm.hpp"

namespace prism {

typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int GEMM_BM = 128;
constexpr int GEMM_BN = 128;
constexpr int GEMM_BK = 32;
constexpr int GEMM_LDS_PITCH = GEMM_BK + 8;  // halves per LDS tile row (80 B)

template <int BITS>
__global__ __launch_bounds__(256) void k_gemm(const uint8_t* __restrict__ lut, const uint8_t* __restrict__ idx,
                                              const uint16_t* __restrict__ X, uint16_t* __restrict__ Y, uint32_t M,
                                              uint32_t N, uint32_t K) {
  constexpr int BM = GEMM_BM, BN = GEMM_BN, BK = GEMM_BK, P = GEMM_LDS_PITCH;
  constexpr int TBL = 1 << BITS;
  __shared__ __attribute__((aligned(16))) uint16_t sA[BM * P];
  __shared__ __attribute__((aligned(16))) uint16_t sB[BN * P];
  __shared__ __attribute__((aligned(16))) uint16_t sL[BN * TBL];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  const uint32_t mt = (M + BM - 1) / BM;
  const uint32_t nt = (N + BN - 1) / BN;
  const uint32_t ntiles = mt * nt;
  // XCD-aware remap: block b runs on XCD b % 8; give XCD x the contiguous
  // tile range [x*per, (x+1)*per).
  uint32_t t = blockIdx.x;
  {
    const uint32_t per = ntiles / 8, rem = ntiles % 8;
    const uint32_t xcd = t % 8, slot = t / 8;
    // XCDs < rem own per+1 tiles.
    const uint32_t start = xcd * per + (xcd < rem ? xcd : rem);
    const uint32_t cnt = per + (xcd < rem ? 1u : 0u);
    t = (slot < cnt) ? start + slot : t;  // blocks past an XCD's share keep identity (only when ntiles%8)
  }
  const uint32_t n0 = (t % nt) * BN;
  const uint32_t m0 = (t / nt) * BM;
  const uint32_t row_bytes = K * BITS / 8;

  // ---- LUTs of this block's rows -> LDS (rows past N are zero)
  {
    constexpr int U4 = BN * TBL * 2 / 16;
    const uint4* src = reinterpret_cast<const uint4*>(lut + (size_t)n0 * TBL * 2);
    uint4* dst = reinterpret_cast<uint4*>(sL);
    const uint32_t live_u4 = (N - n0 < (uint32_t)BN ? N - n0 : (uint32_t)BN) * TBL * 2 / 16;
    for (int i = tid; i < U4; i += 256) dst[i] = (uint32_t)i < live_u4 ? src[i] : make_uint4(0, 0, 0, 0);
  }

  // ---- per-thread global load slots
  // X tile: 128 rows x 64 B; thread -> rows (tid/4) and (tid/4 + 64), 16 B column (tid%4)
  const int xa_r = tid >> 2, xa_c = tid & 3;
  // W index tile: 4-bit: 128 rows x 16 B -> thread: row tid/2, 8 B half (tid%2)
  //               8-bit: 128 rows x 32 B -> thread: row tid/2, 16 B half (tid%2)
  const int wb_r = tid >> 1, wb_h = tid & 1;

  uint4 ra[2];
  uint4 rb;  // 4-bit uses .x,.y
  auto gload = [&](uint32_t k0) {
#pragma unroll
    for (int i = 0; i < 2; i++) {
      const uint32_t m = m0 + xa_r + 64 * i;
      ra[i] = (m < M) ? *reinterpret_cast<const uint4*>(X + (size_t)m * K + k0 + 8 * xa_c) : make_uint4(0, 0, 0, 0);
    }
    const uint32_t n = n0 + wb_r;
    if (BITS == 4) {
      const uint2 v = (n < N) ? *reinterpret_cast<const uint2*>(idx + (size_t)n * row_bytes + k0 / 2 + 8 * wb_h)
                              : make_uint2(0, 0);
      rb = make_uint4(v.x, v.y, 0, 0);
    } else {
      rb = (n < N) ? *reinterpret_cast<const uint4*>(idx + (size_t)n * row_bytes + k0 + 16 * wb_h)
                   : make_uint4(0, 0, 0, 0);
    }
  };
  auto lstore = [&]() {
#pragma unroll
    for (int i = 0; i < 2; i++) *reinterpret_cast<uint4*>(&sA[(xa_r + 64 * i) * P + 8 * xa_c]) = ra[i];
    // decode 16 elements of row wb_r, k = 16*wb_h .. +16
    const uint16_t* tb = &sL[wb_r * TBL];
    uint32_t o[8];
    if (BITS == 4) {
      const uint32_t w2[2] = {rb.x, rb.y};
#pragma unroll
      for (int q = 0; q < 2; q++)
#pragma unroll
        for (int p = 0; p < 4; p++) {
          const uint32_t lo = tb[(w2[q] >> (8 * p)) & 15u];
          const uint32_t hi = tb[(w2[q] >> (8 * p + 4)) & 15u];
          o[4 * q + p] = lo | (hi << 16);
        }
    } else {
      const uint32_t w4[4] = {rb.x, rb.y, rb.z, rb.w};
#pragma unroll
      for (int q = 0; q < 4; q++)
#pragma unroll
        for (int p = 0; p < 2; p++) {
          const uint32_t lo = tb[(w4[q] >> (16 * p)) & 255u];
          const uint32_t hi = tb[(w4[q] >> (16 * p + 8)) & 255u];
          o[2 * q + p] = lo | (hi << 16);
        }
    }
    uint4* d = reinterpret_cast<uint4*>(&sB[wb_r * P + 16 * wb_h]);
    d[0] = make_uint4(o[0], o[1], o[2], o[3]);
    d[1] = make_uint4(o[4], o[5], o[6], o[7]);
  };

  floatx16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; i++)
#pragma unroll
    for (int j = 0; j < 2; j++)
#pragma unroll
      for (int e = 0; e < 16; e++) acc[i][j][e] = 0.0f;

  const uint32_t nk = K / BK;
  gload(0);
  __syncthreads();  // sL ready
  for (uint32_t ks = 0; ks < nk; ks++) {
    lstore();
    __syncthreads();
    if (ks + 1 < nk) gload((ks + 1) * BK);
#pragma unroll
    for (int kk = 0; kk < BK; kk += 16) {
      half8_t af[2], bf[2];
#pragma unroll
      for (int i = 0; i < 2; i++) {
        const int r = wm * 64 + i * 32 + (lane & 31);
        af[i] = *reinterpret_cast<const half8_t*>(&sA[r * P + kk + 8 * (lane >> 5)]);
      }
#pragma unroll
      for (int j = 0; j < 2; j++) {
        const int r = wn * 64 + j * 32 + (lane & 31);
        bf[j] = *reinterpret_cast<const half8_t*>(&sB[r * P + kk + 8 * (lane >> 5)]);
      }
#pragma unroll
      for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
    }
    __syncthreads();
  }

  // ---- epilogue: D[i][j] lane layout: col = lane%32, row = 8*(e/4) + 4*(lane/32) + e%4
#pragma unroll
  for (int i = 0; i < 2; i++)
#pragma unroll
    for (int j = 0; j < 2; j++) {
      const uint32_t n = n0 + wn * 64 + j * 32 + (lane & 31);
#pragma unroll
      for (int e = 0; e < 16; e++) {
        const uint32_t m = m0 + wm * 64 + i * 32 + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
        if (m < M && n < N) Y[(size_t)m * N + n] = __builtin_bit_cast(uint16_t, (_Float16)acc[i][j][e]);
      }
    }
}

// ---------------------------------------------------------------------------
// k_gemm8: 8-bit prefill GEMM.  The LDS-decode scheme of k_gemm (the block's
// 128 row LUTs in LDS, each K step's index tile decoded through them into
// an fp16 B tile) with a 256 (M) x 128 (N) block tile and a 64-wide K step:
// each decoded weight feeds twice the MFMAs, and a step's two barriers cover
// twice the K.
//  * 4 waves as 2 (M) x 2 (N): wave (wm, wn) owns rows [128 wm, +128) x
//    columns [64 wn, +64) = 4 x 2 v_mfma_f32_32x32x16_f16 tiles.
//  * LDS: LUTs 64 KB, X tile 256 x 64 and B tile 128 x 64 fp16 with a
//    144-byte row pitch (16 rows at one 16-byte column land in 16 distinct
//    4-bank groups).
//  * The next step's global loads are issued before the current step's
//    MFMAs; blocks are mapped XCD-aware like k_gemm's.
constexpr int GM8_BM = 256;
constexpr int GM8_BN = 128;
constexpr int GM8_BK = 64;

// SPLIT: block (x, y) covers K steps [y kps, min(K / 64, (y + 1) kps)) and
// writes its fp32 partial tile to part[y][M][N], as k_gemm_w4<MI, true> does.
// GI: the weights are in the GI layout with G rows per group (gemv_lpr.hpp;
// lut and idx both point at it); a thread's 16 index bytes of a K step are
// one chunk of its row.
template <bool SPLIT, bool GI = false>
__global__ __launch_bounds__(256) void k_gemm8(const uint8_t* __restrict__ lut, const uint8_t* __restrict__ idx,
                                               const uint16_t* __restrict__ X, uint16_t* __restrict__ Y, uint32_t M,
                                               uint32_t N, uint32_t K, float* __restrict__ part, uint32_t kps,
                                               uint32_t G) {
  constexpr int BM = GM8_BM, BN = GM8_BN, BK = GM8_BK, P = BK + 8;
  constexpr int XU = BM * BK / 8 / 256;  // 16-byte X chunks per thread per step (8)
  constexpr int WU = BN * BK / 16 / 256; // 16-byte index chunks per thread per step (2)
  __shared__ __attribute__((aligned(16))) uint16_t sA[BM * P];
  __shared__ __attribute__((aligned(16))) uint16_t sB[BN * P];
  __shared__ __attribute__((aligned(16))) uint16_t sL[BN * 256];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  const uint32_t mt = (M + BM - 1) / BM;
  const uint32_t nt = (N + BN - 1) / BN;
  const uint32_t ntiles = mt * nt;
  uint32_t t = blockIdx.x;
  {
    const uint32_t per = ntiles / 8, rem = ntiles % 8;
    const uint32_t xcd = t % 8, slot = t / 8;
    const uint32_t start = xcd * per + (xcd < rem ? xcd : rem);
    const uint32_t cnt = per + (xcd < rem ? 1u : 0u);
    t = (slot < cnt) ? start + slot : t;
  }
  const uint32_t n0 = (t % nt) * BN;
  const uint32_t m0 = (t / nt) * BM;

  // ---- LUTs of this block's rows -> LDS (rows past N are zero)
  {
    constexpr int U4 = BN * 256 * 2 / 16;
    uint4* dst = reinterpret_cast<uint4*>(sL);
    const uint32_t live_u4 = (N - n0 < (uint32_t)BN ? N - n0 : (uint32_t)BN) * 32;
    for (int i = tid; i < U4; i += 256) {
      // piece i % 32 of row n0 + i / 32 (GI: the block's rows may span groups)
      const uint32_t r = n0 + (uint32_t)i / 32;
      const uint4* src =
          reinterpret_cast<const uint4*>(lut + (GI ? gi_lut_offset(G, r, K, 8) : (size_t)r * 512) + 16 * (i % 32));
      dst[i] = (uint32_t)i < live_u4 ? *src : make_uint4(0, 0, 0, 0);
    }
  }

  // chunk c = tid + 256 i: X row c / 8, column chunk c % 8; index row c / 4, chunk c % 4
  uint4 ra[XU], rb[WU];
  // GI: byte offset of chunk 0 of each of the thread's index rows
  size_t wrow[WU];
#pragma unroll
  for (int i = 0; i < WU; i++) {
    const uint32_t n = n0 + ((tid + 256 * i) >> 2);
    wrow[i] = GI ? gi_chunk_offset(G, n < N ? n : 0u, 0, K, 8) : (size_t)n * K;
  }
  auto gload = [&](uint32_t k0) {
#pragma unroll
    for (int i = 0; i < XU; i++) {
      const int c = tid + 256 * i;
      const uint32_t m = m0 + (c >> 3);
      ra[i] = (m < M) ? *reinterpret_cast<const uint4*>(X + (size_t)m * K + k0 + 8 * (c & 7)) : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < WU; i++) {
      const int c = tid + 256 * i;
      const uint32_t n = n0 + (c >> 2);
      const size_t off = GI ? wrow[i] + (size_t)(k0 / 16 + (c & 3)) * G * 16 : wrow[i] + k0 + 16 * (c & 3);
      rb[i] = (n < N) ? *reinterpret_cast<const uint4*>(idx + off) : make_uint4(0, 0, 0, 0);
    }
  };
  auto lstore = [&]() {
#pragma unroll
    for (int i = 0; i < XU; i++) {
      const int c = tid + 256 * i;
      *reinterpret_cast<uint4*>(&sA[(c >> 3) * P + 8 * (c & 7)]) = ra[i];
    }
#pragma unroll
    for (int i = 0; i < WU; i++) {
      const int c = tid + 256 * i, r = c >> 2;
      const uint16_t* tb = &sL[r * 256];
      const uint32_t w4[4] = {rb[i].x, rb[i].y, rb[i].z, rb[i].w};
      uint32_t o[8];
#pragma unroll
      for (int q = 0; q < 4; q++)
#pragma unroll
        for (int p = 0; p < 2; p++) {
          const uint32_t lo = tb[(w4[q] >> (16 * p)) & 255u];
          const uint32_t hi = tb[(w4[q] >> (16 * p + 8)) & 255u];
          o[2 * q + p] = lo | (hi << 16);
        }
      uint4* d = reinterpret_cast<uint4*>(&sB[r * P + 16 * (c & 3)]);
      d[0] = make_uint4(o[0], o[1], o[2], o[3]);
      d[1] = make_uint4(o[4], o[5], o[6], o[7]);
    }
  };

  floatx16 acc[4][2];
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int j = 0; j < 2; j++)
#pragma unroll
      for (int e = 0; e < 16; e++) acc[i][j][e] = 0.0f;

  const uint32_t kb = SPLIT ? blockIdx.y * kps : 0u;  // first K step
  const uint32_t nk = SPLIT ? (K / BK - kb < kps ? K / BK - kb : kps) : K / BK;
  gload(kb * BK);
  __syncthreads();  // sL ready
  for (uint32_t ks = 0; ks < nk; ks++) {
    lstore();
    __syncthreads();
    if (ks + 1 < nk) gload((kb + ks + 1) * BK);
#pragma unroll
    for (int kk = 0; kk < BK; kk += 16) {
      half8_t af[4], bf[2];
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int r = wm * 128 + i * 32 + (lane & 31);
        af[i] = *reinterpret_cast<const half8_t*>(&sA[r * P + kk + 8 * (lane >> 5)]);
      }
#pragma unroll
      for (int j = 0; j < 2; j++) {
        const int r = wn * 64 + j * 32 + (lane & 31);
        bf[j] = *reinterpret_cast<const half8_t*>(&sB[r * P + kk + 8 * (lane >> 5)]);
      }
#pragma unroll
      for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
    }
    __syncthreads();
  }

  // ---- epilogue: D lane layout: col = lane%32, row = 8*(e/4) + 4*(lane/32) + e%4
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int j = 0; j < 2; j++) {
      const uint32_t n = n0 + wn * 64 + j * 32 + (lane & 31);
#pragma unroll
      for (int e = 0; e < 16; e++) {
        const uint32_t m = m0 + wm * 128 + i * 32 + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
        if (m < M && n < N) {
          if constexpr (SPLIT)
            part[((size_t)blockIdx.y * M + m) * N + n] = acc[i][j][e];
          else
            Y[(size_t)m * N + n] = __builtin_bit_cast(uint16_t, (_Float16)acc[i][j][e]);
        }
      }
    }
}

constexpr int GW4_BN = 256;
constexpr int GW4_BK = 64;
constexpr int GW4_PITCH = GW4_BK + 8;  // halves per LDS row (144 B)
// Buffer descriptor word 3 (gfx9-family raw buffer, 32-bit data format).
constexpr int kGwdWord3 = 0x00020000;

// ---------------------------------------------------------------------------
// k_gemm_w4: 4-bit prefill GEMM.  W is decoded straight into MFMA B-operand
// registers; X and the index chunks reach LDS by DMA.
//
// * Block tile 256 (M) x 256 (N), 4 waves (one per SIMD); wave w owns all
//   256 M rows and N columns [64w, +64): 8 x 2 tiles of
//   v_mfma_f32_32x32x16_f16, 256 fp32 accumulators per lane (AGPRs).  Each
//   decoded B operand feeds 8 MFMAs and each A fragment 2.
// * B operand (weights): lane (j = lane%32, h = lane/32) of N-subtile s
//   always holds weight row n0 + 64w + 32s + j, so it keeps that row's LUT
//   in 8 VGPRs as byte planes for the whole K loop, and one index dword (8
//   nibbles) becomes one B operand with v_perm_b32 byte selects
//   (decode_nib8_nat, 29 VALU ops) that co-issue under the MFMAs.  Per
//   64-wide K step the lane uses 16 index bytes of each of its rows (bytes
//   [32 it + 16h, +16)); MFMA step q uses dword q, so lane half h covers
//   k = 64 it + 32h + 8q + 0..7, and the A fragment of the same lane holds
//   the same k (logical chunk 4h + q of the X tile row).
// * Both global streams -- the X tile and the index chunks -- are fetched
//   by the LDS DMA (buffer_load ... lds) into a ring of gwd_stages<MI>() LDS
//   stages, so no VGPR-destination global load is left in the K loop:
//   - X part of a stage: 256 rows x 64 halves = 2048 16-byte slots,
//     unpadded; slot (r, p) holds logical chunk p ^ f(r) of row r, f(r) =
//     (r & 7) ^ ((r >> 3) & 1).  A 16-byte-per-lane LDS read serves 16
//     lanes per clock on gfx950 (64 banks); the 16 rows a fragment read
//     touches at one logical chunk then land in 16 distinct 16-byte bank
//     groups (measured: as fast as a contiguous read, where f(r) = r & 7
//     loses ~30 %).  One DMA instruction fills 8 rows (64 slots, lane l ->
//     slot l): lane l loads row 8i + l/8, chunk (l%8) ^ (l/8) ^ (i & 1).
//     The row goes in the per-lane VGPR offset, which the descriptor's
//     range check covers, and only the K step in the scalar offset, which
//     it does not: a row past M then reads as 0 without touching memory,
//     and a row inside it stays inside it at every K step;
//   - index part: 256 weight rows x 32 bytes (this K step's 64 nibbles),
//     2 slots per row; wave w fills its own 64 rows with 2 instructions,
//     the row again in the VGPR offset and the K step in the scalar one.
// * Schedule of K step it (stage it % S, S = gwd_stages<MI>()): MFMA steps
//   0..2 each read the next step's A fragments and decode its B operands
//   (double buffers) under their own MFMAs.  Before MFMA step 3 the wave
//   waits for its reads of the stage (lgkmcnt) and for its own DMA of step
//   it+1 (loads return in issue order, so vmcnt <= the instructions of the
//   up to S-2 steps issued after it); the barrier then publishes step
//   it+1's stage and frees stage it % S, which the wave refills with step
//   it+S.  Step it+1's index chunks and first A
//   fragments are read under step 3's MFMAs and its first B operands are
//   decoded after them, while the matrix core drains the queued MFMAs.
// * Blocks are mapped XCD-aware: hardware dispatches block b to XCD b % 8;
//   the remap gives each XCD a contiguous range of tiles (N-fastest) so the
//   W tiles and X rows one XCD works on stay in its own L2.
// Requires K % 64 == 0, 16-byte aligned X, an index block below 2 GiB and
// 256 * K * 2 bytes of X per block below 2 GiB (the buffer descriptors'
// 32-bit ranges; rows past M or N read as 0 through the range check of the
// VGPR offset).
constexpr int GWD_WSLOTS = GW4_BN * 2;  // 16-byte index slots per stage
// Ring depth (stages of the DMA ring).  Deeper rings for the shorter blocks
// (6 stages of 24 KB for 128-row blocks, 8 of 16 KB for 64-row blocks)
// measured no faster on short prefills (14336 x 4096, M = 64: 39.4 against
// 37.2-38.0 us; M = 128..512 within 2 %), so every block height keeps 3.
template <int MI>
constexpr int gwd_stages() {
  return 3;
}

__device__ __forceinline__ void gwd_barrier() { asm volatile("s_barrier" ::: "memory"); }

// One 16-byte-per-lane LDS DMA: lane l's 16 bytes at voff + soff of the
// buffer land at LDS byte address `lds` + 16 l (lds wave-uniform).  Issued as
// inline asm so the compiler's wait-count pass, which cannot tell the stages
// of the ring apart, does not drain the whole ring before every LDS read;
// the kernel's own vmcnt waits and barriers order the ring.  The kernel
// uses M0 for nothing else.
__device__ __forceinline__ void gwd_dma16(__amdgpu_buffer_rsrc_t r, const void* lds, uint32_t voff, uint32_t soff) {
  const uint32_t la = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)lds);
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds" ::"s"(la), "v"(voff), "s"(r), "s"(soff)
               : "memory", "m0");
}

template <int N_>
__device__ __forceinline__ void gwd_wait_vm() {
  // vmcnt <= N_, expcnt and lgkmcnt unconstrained (gfx9 s_waitcnt encoding)
  static_assert(N_ >= 0 && N_ < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N_ & 0xF) | ((N_ >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// vmcnt <= n * OPS for a wave-uniform n <= MAXN (the immediate is chosen by
// a branch per value).
template <int OPS, int MAXN>
__device__ __forceinline__ void gwd_wait_steps(uint32_t n) {
  if constexpr (MAXN > 0) {
    if (n >= (uint32_t)MAXN) {
      gwd_wait_vm<MAXN * OPS>();
      return;
    }
    gwd_wait_steps<OPS, MAXN - 1>(n);
  } else {
    gwd_wait_vm<0>();
  }
}

// f(integral_constant<int, I>, it + I) for each I with it + I < nk, as a
// flat sequence of tests (nesting them kept more values live: the 256-row
// kernel spilled).
template <class F, int... I>
__device__ __forceinline__ void gwd_steps(uint32_t it, uint32_t nk, F& f, std::integer_sequence<int, I...>) {
  ((it + I < nk ? (f(std::integral_constant<int, I>{}, it + I), 0) : 0), ...);
}

// MI = 32-row M subtiles per block (BM = 32 MI): 8 for long prefills; 2 and
// 4 give short ones (65..1024 rows) more blocks.
// GI: the weights are in the GI layout with G rows per group (gemv_lpr.hpp;
// lut and idx both point at it).  A K step's index bytes of a row are two
// 16-byte chunks; DMA instruction i of wave w carries chunk i of its 64 rows
// (lane l -> row 64 w + l; G consecutive rows' chunks are contiguous), and
// slot (c, r) of the index part holds chunk c of row r.
// SPLIT: block (x, y) covers K steps [y kps, min(K / 64, (y + 1) kps)) and
// writes its fp32 partial tile to P[y][M][N] (k_gemm_split_sum adds the
// partials); otherwise the whole K range, fp16 to Y.
template <int MI, bool SPLIT, bool GI = false>
__global__ __launch_bounds__(256) void k_gemm_w4(const uint8_t* __restrict__ lut, const uint8_t* __restrict__ idx,
                                                 const uint16_t* __restrict__ X, uint16_t* __restrict__ Y, uint32_t M,
                                                 uint32_t N, uint32_t K, float* __restrict__ P, uint32_t kps,
                                                 uint32_t G) {
  static_assert(MI == 2 || MI == 4 || MI == 8, "32-row M subtiles per block");
  constexpr int BM = 32 * MI, BN = GW4_BN, BK = GW4_BK, S = gwd_stages<MI>();
  constexpr int XS = BM * BK / 8;     // 16-byte X slots per stage
  constexpr int SL = XS + GWD_WSLOTS;
  constexpr int OPS = MI + 2;         // DMA instructions per wave per K step (MI X + 2 index)
  constexpr int XR = 8 * MI;          // X rows each wave fetches
  constexpr int VPI = 56 / MI;        // decode VALU ops scheduled per M subtile (2 MFMAs)
  __shared__ __attribute__((aligned(16))) uint4 sx[S * SL];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int j = lane & 31, h = lane >> 5;

  const uint32_t mt = (M + BM - 1) / BM;
  const uint32_t nt = (N + BN - 1) / BN;
  const uint32_t ntiles = mt * nt;
  uint32_t t = blockIdx.x;
  {
    const uint32_t per = ntiles / 8, rem = ntiles % 8;
    const uint32_t xcd = t % 8, slot = t / 8;
    t = xcd * per + (xcd < rem ? xcd : rem) + slot;
  }
  const uint32_t n0 = (t % nt) * BN;
  const uint32_t m0 = (t / nt) * BM;
  const uint32_t row_bytes = K / 2;
  const uint32_t kb = SPLIT ? blockIdx.y * kps : 0u;  // first K step
  const uint32_t nk = SPLIT ? (K / BK - kb < kps ? K / BK - kb : kps) : K / BK;

  // ---- LUT planes of this lane's two weight rows (rows past N: the last row)
  LutPlanes pl[2];
#pragma unroll
  for (int s = 0; s < 2; s++) {
    uint32_t n = n0 + 64 * wave + 32 * s + j;
    n = n < N ? n : N - 1;
    const uint4* lr = reinterpret_cast<const uint4*>(lut + (GI ? gi_lut_offset(G, n, K, 4) : (size_t)n * 32));
    pl[s] = make_planes(lr[0], lr[1]);
  }
  // ---- DMA sources; reads past the descriptors' ranges return 0
  const uint32_t live = (M - m0 < (uint32_t)BM) ? M - m0 : (uint32_t)BM;
  const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(X + (size_t)m0 * K), (short)0, (int)(live * K * 2u), kGwdWord3);
  const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(
      (void*)idx, (short)0, (int)(GI ? (uint32_t)gi_bytes(G, N, K, 4) : N * row_bytes), kGwdWord3);
  const uint32_t lr8 = (uint32_t)lane >> 3, lc = ((uint32_t)lane & 7u) ^ lr8;
  // Per-lane VGPR offsets of each DMA instruction (row and chunk); the
  // scalar offset carries only the K step.
  const uint32_t xv0 = ((uint32_t)XR * wave + lr8) * K * 2u + 16u * lc;  // even DMA index
  uint32_t xv[MI];
#pragma unroll
  for (int i = 0; i < MI; i++) xv[i] = ((i & 1) ? (xv0 ^ 16u) : xv0) + (uint32_t)i * 16u * K;  // odd: chunk lc ^ 1
  // GI: instruction i reads chunk 2 (it + kb) + i of row 64 w + l (rows past
  // N get an offset past the range: zeros); a K step moves 2 chunks
  const uint32_t grow = n0 + 64u * wave + (uint32_t)lane;
  const uint32_t wv0 = GI ? (grow < N ? (uint32_t)gi_chunk_offset(G, grow, 0, K, 4) : 0x80000000u)
                          : (n0 + 64u * wave + ((uint32_t)lane >> 1)) * row_bytes + 16u * ((uint32_t)lane & 1u);
  const uint32_t wv[2] = {wv0, GI ? wv0 + G * (uint32_t)kGiChunk : wv0 + 32u * row_bytes};

  auto issue = [&](uint32_t it, int stage) {
    uint4* st = sx + stage * SL;
#pragma unroll
    for (int i = 0; i < MI; i++) gwd_dma16(rx, st + 64 * (MI * wave + i), xv[i], (it + kb) * 128u);
#pragma unroll
    for (int i = 0; i < 2; i++)
      gwd_dma16(rw, st + XS + 64 * (2 * wave + i), wv[i], (it + kb) * (GI ? 2u * G * (uint32_t)kGiChunk : 32u));
  };
  auto wdword = [](const uint4& v, int q) { return q == 0 ? v.x : q == 1 ? v.y : q == 2 ? v.z : v.w; };

  floatx16 acc[MI][2];
#pragma unroll
  for (int i = 0; i < MI; i++)
#pragma unroll
    for (int s = 0; s < 2; s++)
#pragma unroll
      for (int e = 0; e < 16; e++) acc[i][s][e] = 0.0f;

  // A fragment of M-subtile i, logical chunk c (= 4h + q): row r = 32i + j,
  // slot (r, c ^ f(r)) with f(r) == f(j).  Index chunk of row s: slot
  // 2 * (64 wave + 32 s + j) + h of the index part.
  const uint32_t arow = (uint32_t)j * 8u;
  const uint32_t asw = ((uint32_t)j & 7u) ^ (((uint32_t)j >> 3) & 1u);
  const uint32_t wsl = GI ? 128u * wave + 64u * h + j : 2u * (64u * wave + j) + h;
  constexpr uint32_t WS1 = GI ? 32u : 64u;  // slot step from row j to row 32 + j

  half8_t a[2][MI];
  half8_t bop[2][2];
  uint4 wch[2];
  auto read_first = [&](const uint4* st) {  // index chunks + MFMA step 0's A fragments
    wch[0] = st[XS + wsl];
    wch[1] = st[XS + wsl + WS1];
#pragma unroll
    for (int i = 0; i < MI; i++) a[0][i] = __builtin_bit_cast(half8_t, st[256 * i + arow + ((4u * h) ^ asw)]);
  };
  auto decode_b = [&](int buf, int q) {
    bop[buf][0] = decode_nib8_nat(wdword(wch[0], q), pl[0]);
    bop[buf][1] = decode_nib8_nat(wdword(wch[1], q), pl[1]);
  };

  // Prologue: steps 0..S-1 in flight, step 0 landed everywhere.
#pragma unroll
  for (int u = 0; u < S; u++)
    if ((uint32_t)u < nk) issue(u, u);
  gwd_wait_steps<OPS, S - 1>((nk < (uint32_t)S ? nk : (uint32_t)S) - 1);
  gwd_barrier();
  read_first(sx);
  decode_b(0, 0);

  auto kstep = [&](auto sc_tag, uint32_t it) {
    constexpr int SC = decltype(sc_tag)::value;
    constexpr int SNX = (SC + 1) % S;
    const uint4* st = sx + SC * SL;
#pragma unroll
    for (int q = 0; q < 3; q++) {
      const int cur = q & 1, nxt = cur ^ 1;
#pragma unroll
      for (int i = 0; i < MI; i++)
        a[nxt][i] = __builtin_bit_cast(half8_t, st[256 * i + arow + ((4u * h + q + 1) ^ asw)]);
      decode_b(nxt, q + 1);
#pragma unroll
      for (int i = 0; i < MI; i++) {
        acc[i][0] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[cur][i], bop[cur][0], acc[i][0], 0, 0, 0);
        acc[i][1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[cur][i], bop[cur][1], acc[i][1], 0, 0, 0);
      }
#pragma unroll
      for (int i = 0; i < MI; i++) {
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
        __builtin_amdgcn_sched_group_barrier(0x002, (VPI + 1) / 2, 0);  // VALU
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
        __builtin_amdgcn_sched_group_barrier(0x002, VPI / 2, 0);  // VALU
      }
    }
    // MFMA step 3 (operands in buffer 1).  Its B decode, issued under step
    // 2's MFMAs, is pinned ahead of the barrier (the compiler would sink it
    // past the asm).
    asm volatile("" : "+v"(bop[1][0]), "+v"(bop[1][1]));
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's reads of stage SC are done
    // step it + 1 must have landed; the steps after it may stay in flight
    const uint32_t ahead = it + 2 < nk ? (nk - it - 2 < (uint32_t)(S - 2) ? nk - it - 2 : (uint32_t)(S - 2)) : 0u;
    gwd_wait_steps<OPS, S - 2>(ahead);
    gwd_barrier();
    if (it + S < nk) issue(it + S, SC);
    const bool more = it + 1 < nk;
    const uint4* sn = sx + SNX * SL;
    if (more) {
      wch[0] = sn[XS + wsl];
      wch[1] = sn[XS + wsl + WS1];
    }
#pragma unroll
    for (int i = 0; i < MI; i++) {
      if (more) a[0][i] = __builtin_bit_cast(half8_t, sn[256 * i + arow + ((4u * h) ^ asw)]);
      acc[i][0] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[1][i], bop[1][0], acc[i][0], 0, 0, 0);
      acc[i][1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[1][i], bop[1][1], acc[i][1], 0, 0, 0);
    }
    if (more) decode_b(0, 0);
    __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);  // DS read: index chunks
#pragma unroll
    for (int i = 0; i < MI; i++) {
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
      __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);  // MFMA
    }
    __builtin_amdgcn_sched_group_barrier(0x002, 64, 0);  // VALU: next step's decode
  };

  for (uint32_t it = 0; it < nk; it += S) gwd_steps(it, nk, kstep, std::make_integer_sequence<int, S>{});

  // ---- epilogue: D lane layout: col j = lane%32, row 8*(e/4) + 4*(lane/32) + e%4
  const bool full = (m0 + BM <= M) && (n0 + BN <= N);
  if (full) {
    // every element in range: buffer stores with the lane's column and
    // half-row in the VGPR offset and the element's row within the tile (a
    // compile-time multiple of N) in the scalar offset, so a store costs one
    // scalar multiply, no per-element address arithmetic or exec-mask branch
    // (the range check only sees the VGPR offset, which stays below 2^31)
    const uint32_t lane_off = 4u * h * N + n0 + 64u * wave + j;  // elements from row m0
    if constexpr (SPLIT) {
      const __amdgpu_buffer_rsrc_t rp = __builtin_amdgcn_make_buffer_rsrc(
          (void*)(P + (size_t)blockIdx.y * M * N + (size_t)m0 * N), (short)0, -1, kBufferWord3);
#pragma unroll
      for (int i = 0; i < MI; i++)
#pragma unroll
        for (int e = 0; e < 16; e++) {
          const uint32_t so = (uint32_t)(32 * i + 8 * (e >> 2) + (e & 3)) * N * 4u;  // both columns' stores share it
#pragma unroll
          for (int s = 0; s < 2; s++) {
            // the element is copied out first: a bit cast applied to the
            // vector-element lvalue itself reads element 0 (hipcc 7.2)
            const float v = acc[i][s][e];
            __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), rp,
                                                  (lane_off + 32u * s) * 4u, so, 0);
          }
        }
    } else {
      const __amdgpu_buffer_rsrc_t ry =
          __builtin_amdgcn_make_buffer_rsrc((void*)(Y + (size_t)m0 * N), (short)0, -1, kBufferWord3);
#pragma unroll
      for (int i = 0; i < MI; i++)
#pragma unroll
        for (int e = 0; e < 16; e++) {
          const uint32_t so = (uint32_t)(32 * i + 8 * (e >> 2) + (e & 3)) * N * 2u;  // both columns' stores share it
#pragma unroll
          for (int s = 0; s < 2; s++)
            __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(uint16_t, (_Float16)acc[i][s][e]), ry,
                                                  (lane_off + 32u * s) * 2u, so, 0);
        }
    }
    return;
  }
#pragma unroll
  for (int s = 0; s < 2; s++) {
    const uint32_t n = n0 + 64 * wave + 32 * s + j;
    uint16_t* yc = Y + n;
    float* pc = SPLIT ? P + (size_t)blockIdx.y * M * N + n : nullptr;
#pragma unroll
    for (int i = 0; i < MI; i++)
#pragma unroll
      for (int e = 0; e < 16; e++) {
        const uint32_t m = m0 + 32 * i + 8 * (e >> 2) + 4 * h + (e & 3);
        if (m < M && n < N) {
          if constexpr (SPLIT)
            pc[(size_t)m * N] = acc[i][s][e];
          else
            yc[(size_t)m * N] = __builtin_bit_cast(uint16_t, (_Float16)acc[i][s][e]);
        }
      }
  }
}

// Y[i] = f16(P[0][i] + P[1][i] + ... + P[S-1][i]) over mn = M N elements,
// the splits added in order in fp32 (deterministic), four elements a thread.
__global__ __launch_bounds__(256) void k_gemm_split_sum(const float* __restrict__ P, uint16_t* __restrict__ Y,
                                                        uint64_t mn, uint32_t S) {
  const uint64_t i0 = ((uint64_t)blockIdx.x * 256u + threadIdx.x) * 4u;
  if (i0 >= mn) return;
  if (mn % 4 == 0) {  // i0 + 4 <= mn and every split's row of 4 is 16-byte aligned
    float4 a = *reinterpret_cast<const float4*>(P + i0);
    for (uint32_t s = 1; s < S; s++) {
      const float4 b = *reinterpret_cast<const float4*>(P + s * mn + i0);
      a.x += b.x;
      a.y += b.y;
      a.z += b.z;
      a.w += b.w;
    }
    Y[i0 + 0] = __builtin_bit_cast(uint16_t, (_Float16)a.x);
    Y[i0 + 1] = __builtin_bit_cast(uint16_t, (_Float16)a.y);
    Y[i0 + 2] = __builtin_bit_cast(uint16_t, (_Float16)a.z);
    Y[i0 + 3] = __builtin_bit_cast(uint16_t, (_Float16)a.w);
    return;
  }
  for (uint64_t i = i0; i < i0 + 4 && i < mn; i++) {
    float a = P[i];
    for (uint32_t s = 1; s < S; s++) a += P[s * mn + i];
    Y[i] = __builtin_bit_cast(uint16_t, (_Float16)a);
  }
}

}  // namespace prism
