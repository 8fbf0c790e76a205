// gemv_lpr8m.hip -- k_gemv_lpr8m, k_gemv_lpr4m and k_gemv_lpr4q (lane-per-row
// lookups feeding the matrix cores, 8- and 4-bit), built in their own translation
// unit with the max-ilp machine scheduler (-mllvm
// -amdgpu-sched-strategy=max-ilp in the Makefile).  That schedule suits
// only these kernels: config 4 at 8
// vectors 14.50-14.61 against 15.32-15.38 us with the default scheduler,
// while the same flag on the whole library slowed the hero GEMV (6.63-6.68
// against 6.49-6.57 us), config 4 at 4 vectors (14.8 against 13.6), cfg2,
// cfg1 and the decode step (542 against 529 us per token).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "gemv_kernels.hpp"
#include "gemv_lpr_args.hpp"

namespace prism {

// 8-bit lane-per-row lookups feeding the matrix cores: the GEMV of 3..8
// vectors over 8-bit GI weights (config 4 at batch 4 and 8), one workgroup of
// 8 waves per group.  The lookups stay lane-private as in k_gemv_lpr8; the
// products go to v_mfma_f32_32x32x16_f16, whose A operand is 32 weight rows
// x 16 k (lane l: row l % 32, k 8 (l / 32) .. + 7) and whose B operand is up
// to 32 vectors x the same 16 k, so the per-vector v_dot2 work of
// k_gemv_lpr8 (half a v_dot2 per element and vector) becomes two MFMAs per
// 32 elements of a row, whatever the vector count.
//  * Waves: tile t = w & 1 holds the group's rows 32 t .. 32 t + 31, K
//    quarter q = w >> 1 a contiguous quarter of the chunks.
//  * Table: dword 64 b + l holds entry b of row l % 32 of tile 0 in its low
//    half and of tile 1 in its high half (64 KB, bank-private: lane l reads
//    bank l); one v_perm per element builds the address, one ds_read_b32
//    returns both tiles' values and one v_perm per two elements keeps the
//    wave's tile.
//  * A double step covers two chunks: lane (r, h) (r = l % 32, h = l / 32)
//    loads chunk 2 s + h of its quarter for row 32 t + r (16 bytes); MFMA j
//    of the step takes bytes 8 j .. 8 j + 7 of that chunk, and its B operand
//    is x[r][16 (chunk) + 8 j .. + 7].  K is permuted between the lanes'
//    halves, identically for weights and x, so the products are the same.
//  * x (nb * K halves, at most 64 KB) is copied to LDS once per workgroup,
//    each vector followed by 16 bytes of padding so that the lanes r < nb,
//    which read their vector's 16 bytes per MFMA (the others read nothing),
//    fall in distinct bank groups (unpadded, vectors K * 2 bytes apart all
//    start in bank 0: bank-conflict cycles exceeded the LDS-active cycles at
//    8 vectors).  The LDS then holds the four quarters' fp32 partials, added
//    in quarter order.
//  * kLpr8mAhead double steps of index bytes in flight per wave.
// Per 32 elements of a row: 32 lookups, 48 VALU ops, 2 MFMAs.  Requires
// K % 512 == 0, nb <= 32, nb * (K / 2 + kLpr8mXPad) <= kLpr8mXDw, 16-byte
// aligned x and the weight block below 2 GiB.  Config 4 (14336 x 4096, 56-row groups), MI355X,
// both kernels in one run, before the lanes past nb stopped reading x:
// 8 vectors 15.0-15.2 us against 17.9-18.2 for k_gemv_lpr8; 2 / 3 / 4
// vectors 14.1-14.4 / 14.2-14.3 / 14.3-14.4 against 12.1 / 13.5-13.6 /
// 13.5-13.8.  With those reads gone it also takes 3 and 4 vectors (the
// dispatch in prism_hip.hip has the numbers).  With x read from global
// memory per MFMA 17.7 / 18.1 us at 4 / 8; 2 or 8 double steps ahead, or
// two accumulators, no faster.
__device__ __forceinline__ void lpr8m_body(const LprArgs& a) {
  constexpr int Q = 4;  // K quarters
  constexpr int AH = kLpr8mAhead;
  typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));
  typedef float f32x16 __attribute__((ext_vector_type(16)));
  typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
  // one static array with the lookup table first: the table's LDS address
  // is 0, so a lookup's v_perm-built address is its ds_read address (with the
  // table behind x, at 66 KB, past ds_read's 16-bit immediate offset, every
  // lookup took one more v_add)
  __shared__ __attribute__((aligned(16))) uint32_t lds_all[kLprTableDw + kLpr8mXDw];
  uint32_t* const lds = lds_all;
  uint32_t* const xs = lds_all + kLprTableDw;  // x, then the partials
  float* red = reinterpret_cast<float*>(xs);  // [Q][2 tiles][32 vectors][33]

  const uint32_t tid = threadIdx.x, lane = tid & 63;
  const uint32_t w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t t = w & 1, q = w >> 1;
  const uint32_t g = blockIdx.x;
  const uint32_t N = a.N, K = a.K, G = a.G, nb = a.nb;
  const uint32_t r32 = lane & 31, h = lane >> 5;
  const uint32_t gbytes = gi_group_bytes(G, K, 8);
  const uint32_t gbase = g * gbytes;
  const __amdgpu_buffer_rsrc_t ri =
      __builtin_amdgcn_make_buffer_rsrc((void*)a.w, (short)0, (int)(gridDim.x * gbytes), kBufferWord3);
  const __amdgpu_buffer_rsrc_t rx =
      __builtin_amdgcn_make_buffer_rsrc((void*)a.x, (short)0, (int)(nb * K * 2u), kBufferWord3);

  // ---- LUT slices (wave w: entries 32 w .. 32 w + 31 of rows r32 and
  // 32 + r32), x, and the first index chunks
  u32x4v L0[4], L1[4];
  {
    const uint32_t ra = r32, rb = 32 + r32;
    const uint32_t la = ra < G ? gbase + gi_lut_offset(G, ra, K, 8) + w * 64u : 0x80000000u;
    const uint32_t lb = rb < G ? gbase + gi_lut_offset(G, rb, K, 8) + w * 64u : 0x80000000u;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      L0[i] = __builtin_amdgcn_raw_buffer_load_b128(ri, la + 16u * i, 0u, 0);
      L1[i] = __builtin_amdgcn_raw_buffer_load_b128(ri, lb + 16u * i, 0u, 0);
    }
  }
  const uint32_t xq = nb * K / 8;  // 16-byte pieces of x (<= 8 per thread)
  u32x4v xv[8];
#pragma unroll
  for (int i = 0; i < 8; i++) {
    const uint32_t p = tid + 512u * i;
    xv[i] = __builtin_amdgcn_raw_buffer_load_b128(rx, p < xq ? p * 16u : 0x80000000u, 0u, 0);
  }
  const uint32_t nd = K / (Q * 32);  // double steps per wave (a multiple of AH)
  const uint32_t c0 = q * (K / (Q * 16));
  const uint32_t row = 32 * t + r32;
  const uint32_t ibase = row < G ? gbase + gi_chunk_offset(G, row, c0 + h, K, 8) : 0x80000000u;
  const uint32_t istep = 2u * G * 16u;  // two chunks of the group
  u32x4v ir[AH];
  auto ld = [&](uint32_t s, int slot) {
    ir[slot] = __builtin_amdgcn_raw_buffer_load_b128(ri, s < nd ? ibase + s * istep : 0x80000000u, 0u, kNontemporal);
  };
#pragma unroll
  for (int u = 0; u < AH; u++) ld(u, u);

  const uint32_t xrow = K / 2 + kLpr8mXPad;  // dwords per vector in LDS
#pragma unroll
  for (int i = 0; i < 8; i++) {
    const uint32_t p = tid + 512u * i;
    if (p < xq) {
      const uint32_t b = p / (K / 8), o = p % (K / 8);
      *reinterpret_cast<u32x4v*>(&xs[b * xrow + 4 * o]) = xv[i];
    }
  }
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int c = 0; c < 4; c++) {
      const uint32_t e = w * 32 + 8 * i + 2 * c;
      const uint32_t a0 = L0[i][c], a1 = L1[i][c];
      lds[e * 64 + lane] = (a0 & 0xFFFFu) | (a1 << 16);
      lds[(e + 1) * 64 + lane] = (a0 >> 16) | (a1 & 0xFFFF0000u);
    }
  __syncthreads();

  const uint32_t lanebase = lane * 4u;
  const uint32_t psel = t ? 0x07060302u : 0x05040100u;  // this tile's halves of two dwords
  // dwords: vector r32, chunk c0 + h (lanes of vectors past nb skip their
  // reads below; their offset stays inside x all the same)
  const uint32_t xoff = (r32 < nb ? r32 : nb - 1) * xrow + 8u * (c0 + h);
  f32x16 acc;
#pragma unroll
  for (int e = 0; e < 16; e++) acc[e] = 0.0f;
  // Only the lanes of real vectors read x: the others' B columns keep stale
  // values, which reach only the output columns r32 >= nb (never stored).
  // LDS returns data for active lanes only, so at 8 vectors a step's x reads
  // take 16 lanes' worth of LDS cycles instead of 64 (config 4 at 8 vectors
  // 13.13-13.21 against 13.83-13.86 us, at 5 vectors 13.00-13.09 against
  // 13.54-13.61, alternating on one box).
  u32x4v xb[2] = {{0u, 0u, 0u, 0u}, {0u, 0u, 0u, 0u}};
  const bool xlive = r32 < nb;
  auto step = [&](uint32_t s, int slot) {
    const u32x4v* xp = reinterpret_cast<const u32x4v*>(&xs[xoff + s * 16u]);
    if (xlive) {
      xb[0] = xp[0];
      xb[1] = xp[1];
    }
#pragma unroll
    for (int j = 0; j < 2; j++) {
      uint32_t v[8];
#pragma unroll
      for (int i = 0; i < 8; i++) {
        const uint32_t wd = ir[slot][2 * j + (i >> 2)];
        const uint32_t ad = __builtin_amdgcn_perm(wd, lanebase, 0x0C0C0000u | ((4u + (i & 3)) << 8));
        v[i] = *reinterpret_cast<const uint32_t*>(reinterpret_cast<const char*>(lds) + ad);
      }
      u32x4v A;
      A.x = __builtin_amdgcn_perm(v[1], v[0], psel);
      A.y = __builtin_amdgcn_perm(v[3], v[2], psel);
      A.z = __builtin_amdgcn_perm(v[5], v[4], psel);
      A.w = __builtin_amdgcn_perm(v[7], v[6], psel);
      acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, A), __builtin_bit_cast(f16x8, xb[j]), acc,
                                                   0, 0, 0);
    }
  };
  for (uint32_t s = 0; s < nd; s += AH) {
#pragma unroll
    for (int u = 0; u < AH; u++) {
      step(s + u, u);
      ld(s + u + AH, u);
    }
  }

  // ---- D: lane (r, h) holds vector r, rows 8 (e / 4) + 4 h + e % 4 of its tile
  __syncthreads();  // x is no longer read: the region takes the partials
#pragma unroll
  for (int e = 0; e < 16; e++) red[((q * 2 + t) * 32 + r32) * 33 + 8 * (e >> 2) + 4 * h + (e & 3)] = acc[e];
  __syncthreads();
  for (uint32_t i = tid; i < 64u * nb; i += 512) {
    const uint32_t b = i / 64, r = i % 64;
    const uint32_t tt = r / 32, rr = r % 32;
    float sum = red[(tt * 32 + b) * 33 + rr];
#pragma unroll
    for (int v = 1; v < Q; v++) sum += red[((v * 2 + tt) * 32 + b) * 33 + rr];
    const uint32_t grow = g * G + r;
    if (r < G && grow < N) a.y[(size_t)b * N + grow] = f2h(sum);
  }
}

// The 4-bit form: the same waves (tile t = w & 1, K quarter q = w >> 1),
// x in LDS read by the lanes of live vectors only, one accumulator of
// v_mfma_f32_32x32x16_f16 per wave; the table is the 4-bit lane-per-row
// pair table (entry b = LUT[b & 15] | LUT[b >> 4] << 16, the fp16 pair of
// an index byte, at LDS dword 64 b + row), so one lookup gives two
// consecutive k of the A operand and four lookups (one index dword) are a
// whole MFMA operand, with no packing.  The two lanes of a row (h = 0, 1)
// read the same bank.  A double step covers two 32-element chunks: lane
// (r, h) takes chunk 2 s + h of its quarter for row 32 t + r; MFMA j of the
// step takes index dword j of that chunk (elements 8 j .. 8 j + 7) and x[r]
// at the same k.  Requires K % 256 == 0.
__device__ __forceinline__ void lpr4m_body(const LprArgs& a) {
  constexpr int Q = 4;
  constexpr int AH = kLpr8mAhead;
  typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));
  typedef float f32x16 __attribute__((ext_vector_type(16)));
  typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
  __shared__ __attribute__((aligned(16))) uint32_t lds_all[kLprTableDw + kLpr8mXDw];
  uint32_t* const lds = lds_all;
  uint32_t* const xs = lds_all + kLprTableDw;
  float* red = reinterpret_cast<float*>(xs);  // [Q][2 tiles][32 vectors][33]

  const uint32_t tid = threadIdx.x, lane = tid & 63;
  const uint32_t w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t t = w & 1, q = w >> 1;
  const uint32_t g = blockIdx.x;
  const uint32_t N = a.N, K = a.K, G = a.G, nb = a.nb;
  const uint32_t r32 = lane & 31, h = lane >> 5;
  const uint32_t gbytes = gi_group_bytes(G, K, 4);
  const uint32_t gbase = g * gbytes;
  const __amdgpu_buffer_rsrc_t ri =
      __builtin_amdgcn_make_buffer_rsrc((void*)a.w, (short)0, (int)(gridDim.x * gbytes), kBufferWord3);
  const __amdgpu_buffer_rsrc_t rx =
      __builtin_amdgcn_make_buffer_rsrc((void*)a.x, (short)0, (int)(nb * K * 2u), kBufferWord3);

  // ---- the LUT of row `lane` (every wave builds 1/8 of every row's table),
  // x, and the first index chunks
  uint32_t L[8];
  {
    const uint32_t lo = lane < G ? gbase + lane * 32u : 0x80000000u;
    const u32x4v l0 = __builtin_amdgcn_raw_buffer_load_b128(ri, lo, 0u, 0);
    const u32x4v l1 = __builtin_amdgcn_raw_buffer_load_b128(ri, lo + 16u, 0u, 0);
    L[0] = l0.x; L[1] = l0.y; L[2] = l0.z; L[3] = l0.w;
    L[4] = l1.x; L[5] = l1.y; L[6] = l1.z; L[7] = l1.w;
  }
  const uint32_t xq = nb * K / 8;
  u32x4v xv[8];
#pragma unroll
  for (int i = 0; i < 8; i++) {
    const uint32_t p = tid + 512u * i;
    xv[i] = __builtin_amdgcn_raw_buffer_load_b128(rx, p < xq ? p * 16u : 0x80000000u, 0u, 0);
  }
  const uint32_t nc = K / 32;              // chunks per row
  const uint32_t nd = nc / (Q * 2);        // double steps per wave
  const uint32_t c0 = q * (nc / Q);
  const uint32_t row = 32 * t + r32;
  const uint32_t ibase = row < G ? gbase + G * 32u + ((c0 + h) * G + row) * kGiChunk : 0x80000000u;
  const uint32_t istep = 2u * G * kGiChunk;  // two chunks of the group
  u32x4v ir[AH];
  auto ld = [&](uint32_t s, int slot) {
    ir[slot] = __builtin_amdgcn_raw_buffer_load_b128(ri, s < nd ? ibase + s * istep : 0x80000000u, 0u, kNontemporal);
  };
#pragma unroll
  for (int u = 0; u < AH; u++) ld(u, u);

  const uint32_t xrow = K / 2 + kLpr8mXPad;
#pragma unroll
  for (int i = 0; i < 8; i++) {
    const uint32_t p = tid + 512u * i;
    if (p < xq) {
      const uint32_t b = p / (K / 8), o = p % (K / 8);
      *reinterpret_cast<u32x4v*>(&xs[b * xrow + 4 * o]) = xv[i];
    }
  }
  // entries e = w + 8 i: low nibble w + 8 (i % 2) (from the LUT registers
  // with the wave-uniform w), high nibble i / 2
  uint32_t hv[2];
#pragma unroll
  for (int j = 0; j < 2; j++) {
    const uint32_t e = w + 8u * j;
    uint32_t d = L[0];
#pragma unroll
    for (int k = 1; k < 8; k++) d = (e >> 1) == (uint32_t)k ? L[k] : d;
    hv[j] = (e & 1) ? (d >> 16) : (d & 0xFFFFu);
  }
#pragma unroll
  for (int i = 0; i < 32; i++) {
    const int hi = i / 2;
    lds[(w + 8 * i) * 64 + lane] = __builtin_amdgcn_perm(L[hi >> 1], hv[i % 2], (hi & 1) ? 0x07060100u : 0x05040100u);
  }
  __syncthreads();

  const uint32_t rowbase = row * 4u;  // byte 0 of a lookup address: the row's bank
  const uint32_t xoff = (r32 < nb ? r32 : nb - 1) * xrow + 16u * (c0 + h);
  f32x16 acc;
#pragma unroll
  for (int e = 0; e < 16; e++) acc[e] = 0.0f;
  u32x4v xb[4] = {{0u, 0u, 0u, 0u}, {0u, 0u, 0u, 0u}, {0u, 0u, 0u, 0u}, {0u, 0u, 0u, 0u}};
  const bool xlive = r32 < nb;
  auto step = [&](uint32_t s, int slot) {
    const u32x4v* xp = reinterpret_cast<const u32x4v*>(&xs[xoff + s * 32u]);
    if (xlive) {
#pragma unroll
      for (int j = 0; j < 4; j++) xb[j] = xp[j];
    }
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const uint32_t wd = ir[slot][j];
      u32x4v A;
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const uint32_t ad = __builtin_amdgcn_perm(wd, rowbase, 0x0C0C0000u | ((4u + i) << 8));
        A[i] = *reinterpret_cast<const uint32_t*>(reinterpret_cast<const char*>(lds) + ad);
      }
      acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, A), __builtin_bit_cast(f16x8, xb[j]), acc,
                                                   0, 0, 0);
    }
  };
  for (uint32_t s = 0; s < nd; s += AH) {
#pragma unroll
    for (int u = 0; u < AH; u++) {
      if (s + u < nd) step(s + u, u);
      ld(s + u + AH, u);
    }
  }

  __syncthreads();
#pragma unroll
  for (int e = 0; e < 16; e++) red[((q * 2 + t) * 32 + r32) * 33 + 8 * (e >> 2) + 4 * h + (e & 3)] = acc[e];
  __syncthreads();
  for (uint32_t i = tid; i < 64u * nb; i += 512) {
    const uint32_t b = i / 64, r = i % 64;
    const uint32_t tt = r / 32, rr = r % 32;
    float sum = red[(tt * 32 + b) * 33 + rr];
#pragma unroll
    for (int v = 1; v < Q; v++) sum += red[((v * 2 + tt) * 32 + b) * 33 + rr];
    const uint32_t grow = g * G + r;
    if (r < G && grow < N) a.y[(size_t)b * N + grow] = f2h(sum);
  }
}

__global__ __launch_bounds__(512) void k_gemv_lpr4m(const uint8_t* w, const uint8_t* w2, const uint16_t* x,
                                                     uint16_t* y, uint16_t* y2, uint32_t N, uint32_t K, uint32_t nb,
                                                     uint32_t G) {
  lpr4m_body(lpr_args(w, w2, x, y, y2, N, K, nb, G));
}

hipError_t launch_gemv_lpr4m(dim3 groups, hipStream_t st, const LprArgs& a) {
  note_launch(reinterpret_cast<const void*>(&k_gemv_lpr4m));
  hipLaunchKernelGGL(k_gemv_lpr4m, groups, dim3(512), 0, st, a.w, a.w2, a.x, a.y, a.y2, a.N, a.K, a.nb, a.G);
  return hipGetLastError();
}

// 4-bit GI GEMV of 3..4 vectors with k_gemv_lpr's work layout and the
// products on v_mfma_f32_4x4x4f16 (16 independent 4 x 4 x 4 blocks per
// instruction).  Lane l owns row G g + l and wave w a contiguous eighth of
// the row's chunks, as in k_gemv_lpr; the lookups are its bank-private pair
// tables (entry b = LUT[b & 15] | LUT[b >> 4] << 16 at LDS dword 64 b + l),
// so two lookups are the row's four consecutive k, exactly the A operand a
// lane gives its 4 x 4 x 4 block (block l / 4, row l % 4).  The B operand of
// lane l is x[l % 4][those four k] from LDS (x copied there once per
// workgroup, as in k_gemv_lpr4m; vectors past nb read vector nb - 1, whose
// output columns are never stored), and the block's result in lane l holds
// rows 4 (l / 4) .. + 3 for vector l % 4.  Per 32 elements of a row: 16
// lookups, 16 v_perm addresses, 4 16-byte x reads and 8 MFMAs, whatever the
// vector count, where k_gemv_lpr issues 16 v_dot2 per vector and
// k_gemv_lpr4m's 32 x 32 x 16 operands put both lanes of a row on one bank.
// MI355X, 14336 x 4096, bench.py (graph-launched), the library with and
// without it alternating on one box, three rounds: 3 / 4 vectors 8.04-8.21
// / 8.10-8.25 us against 8.39-8.50 / 8.43-8.61 for k_gemv_lpr4m.  In one
// process (both with this unit's max-ilp schedule): 2 vectors 7.78-8.02
// against 7.91-8.09 for k_gemv_lpr (kept there), 1 and 8 vectors slower
// (7.8-8.0 against 6.7-7.2, 10.3-10.6 against 9.2-9.5).  The eight waves' partials are added in wave
// order.  Requires K % 256 == 0, G <= 64, 16-byte aligned x and
// nb * (K / 2 + kLpr8mXPad) <= kLpr8mXDw; NCH > 0: the wave's chunk count
// (K / 256) as a compile-time constant.
template <int NCH>
__device__ __forceinline__ void lpr4q_body(const LprArgs& a) {
  constexpr int S = 8;
  constexpr int LO = 16 / S;  // low nibbles of the table entries a wave builds
  constexpr int R = NCH == 0 ? kLpr4qRing : (NCH < kLpr4qFirst ? NCH : kLpr4qFirst);
  constexpr int DR = NCH == 0 ? kLpr4qRing : (R < kLpr4qAhead ? R : kLpr4qAhead);
  typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));
  typedef uint32_t u32x2v __attribute__((ext_vector_type(2)));
  typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
  typedef float f32x4 __attribute__((ext_vector_type(4)));
  // the table at LDS address 0 (a lookup needs no add), then x, then the
  // waves' partials
  __shared__ __attribute__((aligned(16))) uint32_t lds[kLprTableDw + kLpr8mXDw + S * 256];
  uint32_t* const xs = lds + kLprTableDw;
  float* const red = reinterpret_cast<float*>(xs + kLpr8mXDw);

  const uint32_t tid = threadIdx.x, lane = tid & 63;
  const uint32_t w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t N = a.N, K = a.K, G = a.G, nb = a.nb;
  const uint32_t NC = K / 32, c0 = (w * NC) / S, nch = ((w + 1) * NC) / S - c0;
  const uint32_t gbytes = gi_group_bytes(G, K, 4);
  const uint32_t g = blockIdx.x;
  const uint32_t gbase = g * gbytes;
  const bool live = lane < G;
  const __amdgpu_buffer_rsrc_t ri =
      __builtin_amdgcn_make_buffer_rsrc((void*)a.w, (short)0, (int)(gridDim.x * gbytes), kBufferWord3);
  const __amdgpu_buffer_rsrc_t rx =
      __builtin_amdgcn_make_buffer_rsrc((void*)a.x, (short)0, (int)(nb * K * 2u), kBufferWord3);

  // ---- loads in the order they are needed (they return in issue order):
  // the LUT of row `lane`, x, the first chunks.  Lanes past G read zeros
  // through the range check.
  uint32_t L[8];
  {
    const uint32_t lo = live ? gbase + lane * 32u : 0x80000000u;
    const u32x4v l0 = __builtin_amdgcn_raw_buffer_load_b128(ri, lo, 0u, 0);
    const u32x4v l1 = __builtin_amdgcn_raw_buffer_load_b128(ri, lo + 16u, 0u, 0);
    L[0] = l0.x; L[1] = l0.y; L[2] = l0.z; L[3] = l0.w;
    L[4] = l1.x; L[5] = l1.y; L[6] = l1.z; L[7] = l1.w;
  }
  const uint32_t xq = nb * K / 8;  // 16-byte pieces of x (at most 4096: x <= 64 KB)
  u32x4v xv[8];
#pragma unroll
  for (int i = 0; i < 8; i++) {
    const uint32_t p = tid + 512u * i;
    xv[i] = __builtin_amdgcn_raw_buffer_load_b128(rx, p < xq ? p * 16u : 0x80000000u, 0u, 0);
  }
  const uint32_t cstride = G * kGiChunk;  // bytes from chunk c to c + 1 of a row
  const uint32_t vbase = live ? gbase + G * 32u + (c0 * G + lane) * kGiChunk : 0x80000000u;
  u32x4v ring[R];
  auto ldc = [&](uint32_t i, u32x4v& dst) {
    dst = __builtin_amdgcn_raw_buffer_load_b128(ri, i < nch ? vbase + i * cstride : 0x80000000u, 0u, kNontemporal);
  };
#pragma unroll
  for (int u = 0; u < R; u++) ldc(u, ring[u]);

  // ---- pair tables (wave w builds entries w + 8 i: low nibble w + 8 (i % 2)
  // from the LUT registers with the wave-uniform w, high nibble i / 2) and x
  uint32_t hv[LO];
#pragma unroll
  for (int j = 0; j < LO; j++) {
    const uint32_t e = w + S * j;
    uint32_t d = L[0];
#pragma unroll
    for (int q = 1; q < 8; q++) d = (e >> 1) == (uint32_t)q ? L[q] : d;
    hv[j] = (e & 1) ? (d >> 16) : (d & 0xFFFFu);
  }
#pragma unroll
  for (int i = 0; i < 256 / S; i++) {
    const int hi = i / LO;
    lds[(w + S * i) * 64 + lane] = __builtin_amdgcn_perm(L[hi >> 1], hv[i % LO], (hi & 1) ? 0x07060100u : 0x05040100u);
  }
  const uint32_t xrow = K / 2 + kLpr8mXPad;  // LDS dwords from one vector to the next
#pragma unroll
  for (int i = 0; i < 8; i++) {
    const uint32_t p = tid + 512u * i;
    if (p < xq) {
      const uint32_t b = p / (K / 8), o = p % (K / 8);
      *reinterpret_cast<u32x4v*>(&xs[b * xrow + 4 * o]) = xv[i];
    }
  }
  __syncthreads();
  __builtin_amdgcn_sched_barrier(0);

  // ---- lookups and products.  The B operand of lane l: vector l % 4 (nb - 1
  // past nb), the wave's chunks from c0 on: 64 bytes of x per chunk.
  const uint32_t lanebase = lane * 4u;
  const uint32_t xv_lane = (lane & 3u) < nb ? (lane & 3u) : nb - 1;
  const char* const xsb = reinterpret_cast<const char*>(xs) + (xv_lane * xrow * 4u + c0 * 64u);
  f32x4 acc[2] = {{0.0f, 0.0f, 0.0f, 0.0f}, {0.0f, 0.0f, 0.0f, 0.0f}};
  auto chunk = [&](uint32_t c, int slot, bool refill) {
    uint32_t pr[16];
#pragma unroll
    for (int j = 0; j < 16; j++) {
      const uint32_t ad = __builtin_amdgcn_perm(ring[slot][j >> 2], lanebase, 0x0C0C0000u | ((4u + (j & 3)) << 8));
      pr[j] = *reinterpret_cast<const uint32_t*>(reinterpret_cast<const char*>(lds) + ad);
    }
    if (refill) ldc(c + DR, ring[(slot + DR) % R]);
    u32x4v xb[4];
#pragma unroll
    for (int m = 0; m < 4; m++) xb[m] = *reinterpret_cast<const u32x4v*>(xsb + c * 64u + 16u * m);
    // step i: k 4 i .. 4 i + 3 of the chunk = the pairs of index bytes 2 i, 2 i + 1
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const u32x4v X = xb[i / 2];
      const f16x4 A = __builtin_bit_cast(f16x4, u32x2v{pr[2 * i], pr[2 * i + 1]});
      const f16x4 B = __builtin_bit_cast(f16x4, (i & 1) ? u32x2v{X.z, X.w} : u32x2v{X.x, X.y});
      acc[i & 1] = __builtin_amdgcn_mfma_f32_4x4x4f16(A, B, acc[i & 1], 0, 0, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
  };
  if constexpr (NCH > 0) {
#pragma unroll
    for (int c = 0; c < NCH; c++) chunk(c, c % R, c >= R - DR && c + DR < NCH);
  } else {
    // blocks of R chunks with the next block in flight; the last partial
    // block skips its missing chunks (its requests read zeros)
    uint32_t i = 0;
    for (const uint32_t nfull = nch / R; i < nfull * R; i += R) {
#pragma unroll
      for (int u = 0; u < R; u++) chunk(i + u, u, true);
    }
#pragma unroll
    for (int u = 0; u < R - 1; u++)
      if (i + u < nch) chunk(i + u, u, true);
  }

  // ---- the eight waves' partials, added in wave order; lane l's result
  // holds rows 4 (l / 4) .. + 3 of vector l % 4
  *reinterpret_cast<f32x4*>(&red[(w * 64 + lane) * 4]) = acc[0] + acc[1];
  __syncthreads();
  for (uint32_t i = tid; i < 64u * nb; i += 512) {
    const uint32_t v = i / 64, r = i % 64;
    const uint32_t src = (4 * (r / 4) + v) * 4 + r % 4;
    float sum = 0.0f;
#pragma unroll
    for (int v2 = 0; v2 < S; v2++) sum += red[v2 * 256 + src];
    const uint32_t grow = g * G + r;
    if (r < G && grow < N) a.y[(size_t)v * N + grow] = f2h(sum);
  }
}

template <int NCH>
__global__ __launch_bounds__(512) void k_gemv_lpr4q(const uint8_t* w, const uint8_t* w2, const uint16_t* x,
                                                     uint16_t* y, uint16_t* y2, uint32_t N, uint32_t K, uint32_t nb,
                                                     uint32_t G) {
  lpr4q_body<NCH>(lpr_args(w, w2, x, y, y2, N, K, nb, G));
}

hipError_t launch_gemv_lpr4q(dim3 groups, hipStream_t st, const LprArgs& a) {
  const uint32_t nch = a.K / 256;  // chunks per wave (K % 256 == 0)
#define PRISM_LPR4Q(NCH_)                                                                                        \
  do {                                                                                                           \
    note_launch(reinterpret_cast<const void*>(&k_gemv_lpr4q<NCH_>));                                             \
    hipLaunchKernelGGL(k_gemv_lpr4q<NCH_>, groups, dim3(512), 0, st, a.w, a.w2, a.x, a.y, a.y2, a.N, a.K, a.nb, a.G); \
  } while (0)
  if (nch == 16)
    PRISM_LPR4Q(16);
  else if (nch == 8)
    PRISM_LPR4Q(8);
  else
    PRISM_LPR4Q(0);
#undef PRISM_LPR4Q
  return hipGetLastError();
}

__global__ __launch_bounds__(512) void k_gemv_lpr8m(const uint8_t* w, const uint8_t* w2, const uint16_t* x,
                                                     uint16_t* y, uint16_t* y2, uint32_t N, uint32_t K, uint32_t nb,
                                                     uint32_t G) {
  lpr8m_body(lpr_args(w, w2, x, y, y2, N, K, nb, G));
}

hipError_t launch_gemv_lpr8m(dim3 groups, hipStream_t st, const LprArgs& a) {
  note_launch(reinterpret_cast<const void*>(&k_gemv_lpr8m));
  hipLaunchKernelGGL(k_gemv_lpr8m, groups, dim3(512), 0, st, a.w, a.w2, a.x, a.y, a.y2, a.N, a.K, a.nb, a.G);
  return hipGetLastError();
}

}  // namespace prism
