// gemv_mfma.hpp -- 8-bit palettized GEMV for several batch vectors on the
// matrix cores.
//
// y[b, n] = f16( sum_k f32(x[b, k]) * f32(LUT_n[idx(n, k)]) ): the 8-bit
// extension of lut_gemv_cpu (compute-core/src/lut/evaluator.rs:21-44; the
// format of compute-core/tests/palettized_vs_direct.rs:108-135 laid out
// split-block), fp32 accumulation, fp16 output.
//
// With several batch vectors the VALU kernel spends 2 to 4 v_dot2 per weight
// element; here v_mfma_f32_16x16x32_f16 does the products (batch vectors are
// the A rows, padded to 16 with zeros; weight rows the B columns) and each
// element costs one LDS lookup:
//  * a workgroup owns 32 weight rows (two 16-column tiles) and their
//    256-entry fp16 LUTs in LDS (16 KB, entry b of row r at 2 (256 r + b));
//  * its waves split K into 128-wide groups (group g to wave g % W); lane
//    (n = lane % 16, kq = lane / 16) supplies, in MFMA step s of a group at
//    k0, the elements k0 + 32 kq + 8 s .. +7 -- A and B only need to agree
//    on which k a lane and register hold -- so a lane reads 32 contiguous
//    index bytes of each of its two rows and 64 contiguous bytes of x per
//    group, and the next group's loads are in flight while one is looked up;
//  * the first group is requested before the tables are built;
//  * the waves' partial tiles are added in LDS and rounded once.
// The lookups are random reads of a shared table and cost about 7 LDS
// cycles per wave instruction in bank conflicts; a bank-private layout
// (each lane's row copied into its own bank, 64 KB for 32 rows with a
// 32x32 MFMA tile) removes the conflicts but measured slower, its x operand
// padded to 32 rows and its table build costing more than they save.
// Requires K % 128 == 0, 16-byte aligned x, nb <= 8 and N * K below 2 GiB.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "gemv_tile.hpp"
#include "lut_perm.hpp"

namespace prism {

typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int kG8Tiles = 2;   // 16-row MFMA tiles per workgroup
constexpr int kG8Rows = 16 * kG8Tiles;
constexpr int kG8Waves = 8;   // waves splitting K
constexpr int kG8MaxNb = 8;
constexpr int kG8Group = 128; // K elements per wave per loop trip (4 MFMA steps)

__global__ __launch_bounds__(64 * kG8Waves) void k_gemv8_mfma(GemvArgs a) {
  constexpr int T = kG8Tiles, RN = kG8Rows, KW = kG8Waves;
  __shared__ __attribute__((aligned(16))) uint16_t tbl[RN * 256];
  __shared__ float red[KW][RN][kG8MaxNb];

  const uint32_t tid = threadIdx.x, lane = tid & 63;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: scalar buffer offsets
  const uint32_t N = a.N, K = a.K, nb = a.nb;
  const uint32_t n0 = blockIdx.x * RN;

  const uint32_t n = lane & 15, kq = lane >> 4;
  typedef uint32_t u32x4v_t __attribute__((ext_vector_type(4)));
  // x: batch row n of the A operand; rows past nb fall outside the range
  const __amdgpu_buffer_rsrc_t rx =
      __builtin_amdgcn_make_buffer_rsrc((void*)a.x, (short)0, (int)(nb * K * 2u), kBufferWord3);
  const __amdgpu_buffer_rsrc_t ri =
      __builtin_amdgcn_make_buffer_rsrc((void*)a.idx, (short)0, (int)(N * K), kBufferWord3);
  const uint32_t xv = n * K * 2u + kq * 64u;
  uint32_t iv[T];
#pragma unroll
  for (int t = 0; t < T; t++) {
    const uint32_t r = n0 + 16 * t + n;
    iv[t] = (r < N ? r : N - 1) * K + kq * 32u;
  }

  struct Group {
    u32x4v_t x[4];
    u32x4v_t w[T][2];
  };
  auto load = [&](uint32_t g, Group& d) {
    const uint32_t k0 = (wave + KW * g) * kG8Group;
#pragma unroll
    for (int j = 0; j < 4; j++) d.x[j] = __builtin_amdgcn_raw_buffer_load_b128(rx, xv + 16 * j, k0 * 2u, 0);
#pragma unroll
    for (int t = 0; t < T; t++)
#pragma unroll
      for (int j = 0; j < 2; j++)
        d.w[t][j] = __builtin_amdgcn_raw_buffer_load_b128(ri, iv[t] + 16 * j, k0, kNontemporal);
  };
  // 8 lookups into one row's table
  auto look8 = [](const uint16_t* tb, uint32_t lo, uint32_t hi) {
    const _Float16* th = reinterpret_cast<const _Float16*>(tb);
    half8_t b;
    b[0] = th[lo & 0xFFu];
    b[1] = th[(lo >> 8) & 0xFFu];
    b[2] = th[(lo >> 16) & 0xFFu];
    b[3] = th[lo >> 24];
    b[4] = th[hi & 0xFFu];
    b[5] = th[(hi >> 8) & 0xFFu];
    b[6] = th[(hi >> 16) & 0xFFu];
    b[7] = th[hi >> 24];
    return b;
  };
  floatx4 acc[T];
#pragma unroll
  for (int t = 0; t < T; t++) acc[t] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
  auto compute = [&](const Group& d) {
#pragma unroll
    for (int s = 0; s < 4; s++) {
      const half8_t av = __builtin_bit_cast(half8_t, d.x[s]);
      const int h = s >> 1, q = 2 * (s & 1);
#pragma unroll
      for (int t = 0; t < T; t++)
        acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, look8(tbl + (16 * t + n) * 256, d.w[t][h][q],
                                                                  d.w[t][h][q + 1]),
                                                        acc[t], 0, 0, 0);
    }
  };

  const uint32_t ng = K / kG8Group;
  const uint32_t mine = ng > wave ? (ng - wave + KW - 1) / KW : 0;
  Group ga, gb;
  if (mine > 0) load(0, ga);

  // ---- LUTs of the workgroup's rows (rows past N: zeros).  A raw barrier:
  // __syncthreads would also wait for the group loads above.
  {
    const uint4* src = reinterpret_cast<const uint4*>(a.lut + (size_t)n0 * 512);
    uint4* dst = reinterpret_cast<uint4*>(tbl);
    const uint32_t live = (N - n0 < (uint32_t)RN ? N - n0 : (uint32_t)RN) * 32;  // uint4 per row: 32
#pragma unroll
    for (int i = 0; i < RN * 32 / (64 * KW); i++) {
      const uint32_t e = tid + 64 * KW * i;
      dst[e] = e < live ? src[e] : make_uint4(0, 0, 0, 0);
    }
  }
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");

  if (mine > 0) {
    uint32_t g = 1;
    for (; g + 1 < mine; g += 2) {
      load(g, gb);
      __builtin_amdgcn_sched_barrier(0);  // keep the loads ahead of the lookups
      compute(ga);
      load(g + 1, ga);
      __builtin_amdgcn_sched_barrier(0);
      compute(gb);
    }
    if (g < mine) {
      load(g, gb);
      __builtin_amdgcn_sched_barrier(0);
      compute(ga);
      compute(gb);
    } else {
      compute(ga);
    }
  }

  // ---- acc[t][i] = partial y[m = 4 kq + i][n0 + 16 t + n]
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const uint32_t m = 4 * kq + i;
    if (m < (uint32_t)kG8MaxNb)
#pragma unroll
      for (int t = 0; t < T; t++) red[wave][16 * t + n][m] = acc[t][i];
  }
  __syncthreads();
  for (uint32_t e = tid; e < (uint32_t)(RN * kG8MaxNb); e += 64 * KW) {
    const uint32_t r = e / kG8MaxNb, m = e % kG8MaxNb;
    float v = 0.0f;
#pragma unroll
    for (int w = 0; w < KW; w++) v += red[w][r][m];
    if (m < nb && n0 + r < N) a.y[(size_t)m * N + n0 + r] = f2h(v);
  }
}

}  // namespace prism
