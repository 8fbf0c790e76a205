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
// k_gemm_w4: 4-bit prefill GEMM that decodes W straight into MFMA B-operand
// registers (no decoded-W tile in LDS).
//
// * Block tile 256 (M) x 256 (N), 4 waves (one per SIMD); wave w owns all
//   256 M rows and N columns [64w, +64): 8 x 2 tiles of
//   v_mfma_f32_32x32x16_f16, 256 fp32 accumulators per lane (AGPRs).  Each
//   decoded B operand feeds 8 MFMAs and each A fragment 2, which keeps the
//   VALU decode at ~40 % and the LDS fragment reads at ~50 % of the MFMA
//   time; the step loop is software-pipelined (next step's B decoded while
//   the current step's MFMAs run) and interleaved with
//   sched_group_barrier so one wave per SIMD keeps the matrix core fed.
// * B operand (weights): lane (j = lane%32, h = lane/32) of N-subtile t
//   always holds weight row n0 + 64w + 32t + j, so it keeps that row's LUT
//   in 8 VGPRs as byte planes (lo / hi bytes of entries 0-3, 4-7, 8-11,
//   12-15) for the whole K loop.  One index dword (8 nibbles) is decoded
//   with v_perm_b32 byte selects (two 8-byte windows and a bit-3 v_bfi
//   merge for lo and hi bytes, then two interleaving perms): 25 VALU ops
//   for the 4 VGPRs of one MFMA B operand, which co-issue under the 8
//   MFMAs (8 M-subtiles) that consume it.
// * The decoded halves come out in k order (0,2,4,6,1,3,5,7) of the
//   dword's 8 nibbles; the X tile is stored in LDS with every group of 8
//   halves permuted the same way, so A (X) and B agree on k.
// * X tile (A operand) 256 x 64 fp16 in LDS, double-buffered, 144-byte row
//   pitch (16-byte fragment reads of 8 consecutive rows hit 32 distinct
//   banks); the next K step's X tile and index chunks are loaded from global
//   memory while the current step's MFMAs run; one barrier per K step.
// * Per 64-wide K step a lane loads 16 index bytes of each of its two rows
//   (bytes [32*it + 16h, +16), i.e. nibbles [64*it + 32h, +32)); MFMA step
//   q in {0..3} uses dword q, so lane half h covers k = 64*it + 32h + 8q +
//   {0,2,4,6,1,3,5,7}.
// Requires K % 64 == 0.
constexpr int GW4_BM = 256;
constexpr int GW4_BN = 256;
constexpr int GW4_BK = 64;
constexpr int GW4_PITCH = GW4_BK + 8;  // halves per LDS row (144 B)

__global__ __launch_bounds__(256) void k_gemm_w4(const uint8_t* __restrict__ lut, const uint8_t* __restrict__ idx,
                                                 const uint16_t* __restrict__ X, uint16_t* __restrict__ Y, uint32_t M,
                                                 uint32_t N, uint32_t K) {
  constexpr int BM = GW4_BM, BN = GW4_BN, BK = GW4_BK, P = GW4_PITCH;
  __shared__ __attribute__((aligned(16))) uint16_t sX[2][BM * P];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;  // wave tile: all 256 M rows, N cols [64*wave, +64)
  const int j = lane & 31, h = lane >> 5;

  const uint32_t mt = (M + BM - 1) / BM;
  const uint32_t nt = (N + BN - 1) / BN;
  const uint32_t ntiles = mt * nt;
  uint32_t t = blockIdx.x;
  {
    // XCD-aware: block b runs on XCD b % 8; XCD x takes a contiguous tile
    // range, N-fastest, so its W rows and X rows stay in its own L2.
    const uint32_t per = ntiles / 8, rem = ntiles % 8;
    const uint32_t xcd = t % 8, slot = t / 8;
    const uint32_t start = xcd * per + (xcd < rem ? xcd : rem);
    t = start + slot;
  }
  const uint32_t n0 = (t % nt) * BN;
  const uint32_t m0 = (t / nt) * BM;
  const uint32_t row_bytes = K / 2;
  const uint32_t nk = K / BK;

  // ---- this lane's two weight rows: LUT planes and index row pointers
  LutPlanes pl[2];
  const uint8_t* wrow[2];
#pragma unroll
  for (int s = 0; s < 2; s++) {
    uint32_t n = n0 + 64 * wave + 32 * s + j;
    n = n < N ? n : N - 1;
    const uint4* lr = reinterpret_cast<const uint4*>(lut + (size_t)n * 32);
    pl[s] = make_planes(lr[0], lr[1]);
    wrow[s] = idx + (size_t)n * row_bytes + 16 * h;
  }

  // ---- X tile loads: 256 rows x 128 B = 2048 chunks of 16 B, 8 per thread
  uint4 xs[8];
  auto load_x = [&](uint32_t it) {
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const int c = tid + 256 * i;
      uint32_t m = m0 + (c >> 3);
      m = m < M ? m : M - 1;
      xs[i] = *reinterpret_cast<const uint4*>(X + (size_t)m * K + (size_t)it * BK + 8 * (c & 7));
    }
  };
  // permute each group of 8 halves to k order (0,2,4,6,1,3,5,7) and store
  auto store_x = [&](int buf) {
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const int c = tid + 256 * i;
      const uint4 v = xs[i];
      uint4 o;
      o.x = __builtin_amdgcn_perm(v.y, v.x, 0x05040100u);
      o.y = __builtin_amdgcn_perm(v.w, v.z, 0x05040100u);
      o.z = __builtin_amdgcn_perm(v.y, v.x, 0x07060302u);
      o.w = __builtin_amdgcn_perm(v.w, v.z, 0x07060302u);
      *reinterpret_cast<uint4*>(&sX[buf][(c >> 3) * P + 8 * (c & 7)]) = o;
    }
  };
  uint4 wc[2], wn2[2];
  auto load_w = [&](uint32_t it, uint4 (&dst)[2]) {
#pragma unroll
    for (int s = 0; s < 2; s++) {
      dst[s] = *reinterpret_cast<const uint4*>(wrow[s] + (size_t)it * 32);
      // opaque to the optimizer: keep the loaded words in registers instead
      // of re-issuing the (read-only) load next to a later use
      asm volatile("" : "+v"(dst[s].x), "+v"(dst[s].y), "+v"(dst[s].z), "+v"(dst[s].w));
    }
  };
  auto wdword = [](const uint4& v, int q) { return q == 0 ? v.x : q == 1 ? v.y : q == 2 ? v.z : v.w; };

  floatx16 acc[8][2];
#pragma unroll
  for (int i = 0; i < 8; i++)
#pragma unroll
    for (int s = 0; s < 2; s++)
#pragma unroll
      for (int e = 0; e < 16; e++) acc[i][s][e] = 0.0f;

  load_x(0);
  load_w(0, wc);
  store_x(0);
  __syncthreads();
  // Software pipeline over MFMA steps: the B operands of the next step are
  // decoded while the current step's 16 MFMAs run (two register sets,
  // indexed by step parity); A fragments are read next to their MFMAs.
  half8_t bop[2][2];
  bop[0][0] = decode_nib8(wc[0].x, pl[0]);
  bop[0][1] = decode_nib8(wc[1].x, pl[1]);
  int buf = 0;
  for (uint32_t it = 0; it < nk; it++) {
    // next K block's global loads (clamped on the last block: a re-read of
    // the same tile, L2 hits) -- keeps the loop body one straight-line block
    const uint32_t itn = it + 1 < nk ? it + 1 : it;
    load_x(itn);
    load_w(itn, wn2);
    const uint16_t* xb = &sX[buf][j * P + 32 * h];
#pragma unroll
    for (int q = 0; q < 4; q++) {
      const int cur = q & 1, nxt = cur ^ 1;
      half8_t a[8];
#pragma unroll
      for (int i = 0; i < 8; i++) a[i] = *reinterpret_cast<const half8_t*>(xb + 32 * i * P + 8 * q);
      if (q < 3) {
        bop[nxt][0] = decode_nib8(wdword(wc[0], q + 1), pl[0]);
        bop[nxt][1] = decode_nib8(wdword(wc[1], q + 1), pl[1]);
      } else {
        bop[nxt][0] = decode_nib8(wn2[0].x, pl[0]);
        bop[nxt][1] = decode_nib8(wn2[1].x, pl[1]);
      }
#pragma unroll
      for (int i = 0; i < 8; i++) {
        acc[i][0] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[i], bop[cur][0], acc[i][0], 0, 0, 0);
        acc[i][1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[i], bop[cur][1], acc[i][1], 0, 0, 0);
      }
      // interleave: per MFMA pair, one A fragment read and ~3 VALU ops each
#pragma unroll
      for (int i = 0; i < 8; i++) {
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
        __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);  // VALU
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
        __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);  // VALU
      }
    }
    store_x(buf ^ 1);
    wc[0] = wn2[0];
    wc[1] = wn2[1];
    __syncthreads();
    buf ^= 1;
  }

  // ---- epilogue: D lane layout: col j = lane%32, row 8*(e/4) + 4*(lane/32) + e%4
  const bool full = (m0 + BM <= M) && (n0 + BN <= N);
#pragma unroll
  for (int s = 0; s < 2; s++) {
    const uint32_t n = n0 + 64 * wave + 32 * s + j;
    uint16_t* yc = Y + n;
#pragma unroll
    for (int i = 0; i < 8; i++)
#pragma unroll
      for (int e = 0; e < 16; e++) {
        const uint32_t m = m0 + 32 * i + 8 * (e >> 2) + 4 * h + (e & 3);
        if (full || (m < M && n < N)) yc[(size_t)m * N] = __builtin_bit_cast(uint16_t, (_Float16)acc[i][s][e]);
      }
  }
}

}  // namespace prism
