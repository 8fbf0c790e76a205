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

namespace prism {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
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

}  // namespace prism
