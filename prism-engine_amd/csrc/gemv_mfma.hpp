// gemv_mfma.hpp -- palettized GEMV for several batch vectors on the matrix
// cores, 4- and 8-bit.
//
// y[b, n] = f16( sum_k f32(x[b, k]) * f32(LUT_n[idx(n, k)]) ): lut_gemv_cpu
// (compute-core/src/lut/evaluator.rs:21-44) and its 8-bit extension (the
// format of compute-core/tests/palettized_vs_direct.rs:108-135 laid out
// split-block), fp32 accumulation, fp16 output.
//
// With several batch vectors the VALU kernel spends 2 to 4 v_dot2 per pair
// of weight elements; here v_mfma_f32_16x16x32_f16 does the products (batch
// vectors are the A rows, up to 16, padded with zeros; weight rows the B
// columns) and the lookups are all that is left per element:
//  * a workgroup owns 32 weight rows (two 16-column tiles); its waves split
//    K into 128-wide groups (group g to wave g % W);
//  * lane (n = lane % 16, kq = lane / 16) supplies, in MFMA step s of a
//    group at k0, the elements k0 + 32 kq + 8 s .. +7 -- A and B only need
//    to agree on which k a lane and register hold -- so a lane reads 32
//    contiguous elements' index bytes of each of its two rows and 64
//    contiguous bytes of x per group, and the next group's loads are in
//    flight while one is looked up; the first group is requested before the
//    tables are built;
//  * 8-bit: each row's 256-entry fp16 LUT in LDS (16 KB, entry b of row r at
//    2 (256 r + b)), one 16-bit lookup per element;
//  * 4-bit: each row's pair table, entry b = LUT[b & 15] | LUT[b >> 4] << 16
//    (one index byte -> the fp16 pair of two elements), laid out
//    [tile][entry][row] (entry b of tile row n at dword 4096 t + 16 b + n):
//    the four lanes of a row read banks n, n + 16, n + 32, n + 48 by b % 4,
//    so only lanes of one row can conflict; one dword lookup per two
//    elements (32 KB);
//  * the waves' partial tiles are added in LDS and rounded once.
// The lookups are random reads of shared tables and cost LDS cycles in bank
// conflicts; a bank-private layout (each lane's row copied into its own
// bank, 64 KB for 32 8-bit rows with a 32x32 MFMA tile) removes them but
// measured slower, its x operand padded to 32 rows and its table build
// costing more than they save.
// GI: the weights are in the GI layout with a.gi rows per group
// (gemv_lpr.hpp; a.lut and a.idx both point at it): a lane's index bytes of
// a K group are one 16-byte chunk of its row (4-bit) or two consecutive
// chunks, G * 16 bytes apart (8-bit).
// Requires K % 128 == 0, 16-byte aligned x, nb <= 16 and the weight bytes
// below 2 GiB.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "gemv_tile.hpp"
#include "gemv_lpr.hpp"
#include "lut_perm.hpp"

namespace prism {

typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int kGmTiles = 2;   // 16-row MFMA tiles per workgroup
constexpr int kGmRows = 16 * kGmTiles;
constexpr int kGmWaves = 8;   // waves splitting K
constexpr int kGmMaxNb = 16;  // batch vectors per pass: the A operand's 16 rows
constexpr int kGmGroup = 128; // K elements per wave per loop trip (4 MFMA steps)

template <int BITS, bool GI = false>
__global__ __launch_bounds__(64 * kGmWaves) void k_gemv_mfma(GemvArgs a) {
  static_assert(BITS == 4 || BITS == 8, "4- or 8-bit indices");
  constexpr int T = kGmTiles, RN = kGmRows, KW = kGmWaves, NT = 64 * kGmWaves;
  constexpr int IB = 32 * BITS / 8;  // index bytes per lane, row and group
  // 8-bit: [row][256] fp16; 4-bit: [tile][256][16] pair dwords
  __shared__ __attribute__((aligned(16))) uint32_t tbl[BITS == 8 ? RN * 128 : T * 4096];
  __shared__ float red[KW][RN][kGmMaxNb];

  const uint32_t tid = threadIdx.x, lane = tid & 63;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: scalar buffer offsets
  const uint32_t N = a.N, K = a.K, nb = a.nb;
  const uint32_t n0 = blockIdx.x * RN;

  const uint32_t n = lane & 15, kq = lane >> 4;
  typedef uint32_t u32x4v_t __attribute__((ext_vector_type(4)));
  typedef uint32_t u32x2v_t __attribute__((ext_vector_type(2)));
  // x: batch row n of the A operand; rows past nb fall outside the range
  const __amdgpu_buffer_rsrc_t rx =
      __builtin_amdgcn_make_buffer_rsrc((void*)a.x, (short)0, (int)(nb * K * 2u), kBufferWord3);
  const uint32_t G = GI ? a.gi : 0u;
  const uint32_t wbytes = GI ? (uint32_t)gi_bytes(G, N, K, BITS) : N * (K * BITS / 8);
  const __amdgpu_buffer_rsrc_t ri = __builtin_amdgcn_make_buffer_rsrc((void*)a.idx, (short)0, (int)wbytes, kBufferWord3);
  const uint32_t xv = n * K * 2u + kq * 64u;
  // per-lane VGPR offset of the lane's index bytes in group 0; the group's
  // K offset is the scalar offset, which stays inside the row (GI: inside
  // the row's group)
  uint32_t iv[T];
#pragma unroll
  for (int t = 0; t < T; t++) {
    uint32_t r = n0 + 16 * t + n;
    r = r < N ? r : N - 1;
    iv[t] = GI ? (uint32_t)gi_chunk_offset(G, r, kq * (IB / 16), K, BITS) : r * (K * BITS / 8) + kq * IB;
  }

  struct Group {
    u32x4v_t x[4];
    u32x4v_t w[T][IB / 16];
  };
  auto load = [&](uint32_t g, Group& d) {
    const uint32_t k0 = (wave + KW * g) * kGmGroup;
#pragma unroll
    for (int j = 0; j < 4; j++) d.x[j] = __builtin_amdgcn_raw_buffer_load_b128(rx, xv + 16 * j, k0 * 2u, 0);
#pragma unroll
    for (int t = 0; t < T; t++)
#pragma unroll
      for (int j = 0; j < IB / 16; j++)
        d.w[t][j] = __builtin_amdgcn_raw_buffer_load_b128(ri, iv[t] + (GI ? G * 16u : 16u) * j,
                                                          GI ? k0 * BITS / 8u * G : k0 * BITS / 8, kNontemporal);
  };
  // B operand of tile t: the 8 elements whose index bits are `w`
  auto lookb = [&](int t, u32x2v_t w) {
    if constexpr (BITS == 8) {
      const _Float16* th = reinterpret_cast<const _Float16*>(tbl) + (16 * t + n) * 256;
      half8_t b;
      b[0] = th[w.x & 0xFFu];
      b[1] = th[(w.x >> 8) & 0xFFu];
      b[2] = th[(w.x >> 16) & 0xFFu];
      b[3] = th[w.x >> 24];
      b[4] = th[w.y & 0xFFu];
      b[5] = th[(w.y >> 8) & 0xFFu];
      b[6] = th[(w.y >> 16) & 0xFFu];
      b[7] = th[w.y >> 24];
      return b;
    } else {
      const uint32_t* tt = tbl + 4096 * t + n;
      u32x4v_t b;
      b[0] = tt[16 * (w.x & 0xFFu)];
      b[1] = tt[16 * ((w.x >> 8) & 0xFFu)];
      b[2] = tt[16 * ((w.x >> 16) & 0xFFu)];
      b[3] = tt[16 * (w.x >> 24)];
      return __builtin_bit_cast(half8_t, b);
    }
  };
  floatx4 acc[T];
#pragma unroll
  for (int t = 0; t < T; t++) acc[t] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
  auto compute = [&](const Group& d) {
#pragma unroll
    for (int s = 0; s < 4; s++) {
      const half8_t av = __builtin_bit_cast(half8_t, d.x[s]);
#pragma unroll
      for (int t = 0; t < T; t++) {
        u32x2v_t w;
        if constexpr (BITS == 8) {
          w.x = d.w[t][s >> 1][2 * (s & 1)];
          w.y = d.w[t][s >> 1][2 * (s & 1) + 1];
        } else {
          w.x = d.w[t][0][s];
          w.y = 0;
        }
        acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, lookb(t, w), acc[t], 0, 0, 0);
      }
    }
  };

  const uint32_t ng = K / kGmGroup;
  const uint32_t mine = ng > wave ? (ng - wave + KW - 1) / KW : 0;
  Group ga, gb;
  if (mine > 0) load(0, ga);

  // ---- lookup tables of the workgroup's rows (rows past N: zeros).  Raw
  // barriers: __syncthreads would also wait for the group loads above.
  const uint32_t live = N - n0 < (uint32_t)RN ? N - n0 : (uint32_t)RN;
  if constexpr (BITS == 8) {
    uint4* dst = reinterpret_cast<uint4*>(tbl);
#pragma unroll
    for (int i = 0; i < RN * 32 / NT; i++) {
      const uint32_t e = tid + NT * i;  // uint4 e % 32 of row n0 + e / 32 (GI: the rows may span two groups)
      const uint4* src = reinterpret_cast<const uint4*>(
          a.lut + (GI ? gi_lut_offset(G, n0 + e / 32, K, 8) : (size_t)(n0 + e / 32) * 512) + 16 * (e % 32));
      dst[e] = e < live * 32 ? *src : make_uint4(0, 0, 0, 0);
    }
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  } else {
    // the 32 rows' 16-entry LUTs (1 KB) in the reduction buffer, then the
    // pair tables from them
    static_assert(sizeof(red) >= RN * 32, "LUT staging fits the reduction buffer");
    uint16_t* stage = reinterpret_cast<uint16_t*>(&red[0][0][0]);
    if (tid < (uint32_t)RN * 2) {
      // half tid % 2 of row n0 + tid / 2 (GI: the workgroup's rows may span two groups)
      const uint32_t r = n0 + tid / 2;
      const uint4* src =
          reinterpret_cast<const uint4*>(a.lut + (GI ? gi_lut_offset(G, r, K, 4) : (size_t)r * 32) + (tid % 2) * 16);
      reinterpret_cast<uint4*>(stage)[tid] = tid < live * 2 ? *src : make_uint4(0, 0, 0, 0);
    }
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
#pragma unroll
    for (int i = 0; i < T * 4096 / NT; i++) {
      const uint32_t e = tid + NT * i;  // dword 4096 t + 16 b + r
      const uint32_t r = 16 * (e >> 12) + (e & 15), b = (e >> 4) & 255;
      tbl[e] = (uint32_t)stage[r * 16 + (b & 15)] | ((uint32_t)stage[r * 16 + (b >> 4)] << 16);
    }
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");  // before the staging copy is overwritten
  }

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
#pragma unroll
    for (int t = 0; t < T; t++) red[wave][16 * t + n][m] = acc[t][i];
  }
  __syncthreads();
  for (uint32_t e = tid; e < (uint32_t)(RN * kGmMaxNb); e += NT) {
    const uint32_t r = e / kGmMaxNb, m = e % kGmMaxNb;
    float v = 0.0f;
#pragma unroll
    for (int w = 0; w < KW; w++) v += red[w][r][m];
    if (m < nb && n0 + r < N) a.y[(size_t)m * N + n0 + r] = f2h(v);
  }
}

}  // namespace prism
