// gemv_lpr.hpp -- lane-per-row palettized GEMVs for gfx950 over the
// group-interleaved device layout (GI), 4-bit (k_gemv_lpr) and 8-bit
// (k_gemv_lpr8, further down), and the layout itself.
//
// y[b, r] = f16( sum_k f32(x[b, k]) * f32(LUT_r[idx(r, k)]) ): the
// arithmetic of lut_gemv_cpu (compute-core/src/lut/evaluator.rs:21-44),
// fp32 accumulation, fp16 output (RNE).  NM = 2 runs a gate and an up
// matrix of the same shape over the same x: either the SwiGLU epilogue of
// the CPU path (evaluator.rs:78-83,209-225, engine_impl.rs:1349-1374) or the
// two raw outputs of fused_gate_up.metal (templates/fused_gate_up.metal:16-97).
//
// GI device layout (written at upload by k_gi_pack; 4-bit with K % 64 == 0,
// 8-bit with K % 512 == 0), G <= 64 rows per group, chosen at upload so that
// the groups fill the GPU:
//   ceil(N/G) row groups of gi_group_bytes(G, K, bits) bytes each:
//     [G row LUTs (32 B fp16 at 4 bits, 512 B at 8)][row bytes / 16 chunks][G rows][16 B]
//   chunk c of row r holds index bytes 16c .. 16c+15 of the split-block row
//   (4-bit: elements 32c .. 32c+31, element 2i = low nibble of byte i;
//   8-bit: elements 16c .. 16c+15).  Rows past
//   N in the last group are zero.  A wave's 16-byte-per-lane load reads
//   chunk c of the group's G rows: 16 G bytes contiguous.  A group's LUTs
//   sit right before its chunks, so they come from the same DRAM pages as
//   the first chunks (in a separate block the LUT requests returned late,
//   behind the index stream).  Bytes are the split-block payload's,
//   rearranged (plus the zero rows of the last group).
//
// Work layout: one workgroup of S waves per group.  Lane l < G owns row
// G g + l for the whole kernel (lanes past G load nothing and store
// nothing); wave w owns a contiguous range of the
// row's chunks (the S ranges partition K/32), so every lane of a wave
// reads the same x elements at the same time and x lives in SGPRs
// (scalar loads; v_dot2 takes it as its scalar operand).
//  * Lookup tables are bank-private: the 256-entry pair table of the row
//    of lane l (entry b = LUT[b & 15] | LUT[b >> 4] << 16, the fp16 pair of
//    an index byte) sits at LDS dword 64 b + l, so lane l only ever reads
//    bank l and no lookup conflicts (a table shared by the wave loses about
//    half its LDS cycles to conflicts).  One v_perm builds the address
//    (lane*4 in byte 0, the index byte in byte 1) and one ds_read_b32 reads
//    the pair: per element one VALU op and half an LDS read, plus the v_dot2.
//  * Loads: the LUTs (two 16-byte loads per lane), the first chunks of each
//    wave (kLprFirst when the wave's chunk count is a compile-time constant,
//    else one x block's worth) and the first x block go out first; after
//    the table build each wave keeps a fixed number of chunk loads ahead of
//    its lookups (kLprAhead, or one x block), so the index stream is
//    requested at the rate the lookups consume it (with every chunk
//    requested up front, the waves whose chunks return last decode all of
//    theirs at the end).  Chunk loads are unconditional or statically
//    conditional (past the wave's range they read zeros through the range
//    check), so the compiler's wait counts stay exact instead of falling
//    back to waiting for every load.
//  * The S wave partials of each row are added in LDS in wave order and
//    rounded once.
// Requires K % 64 == 0, 16-byte aligned x (scalar loads need dword alignment)
// and the weight block below 2 GiB (32-bit buffer offsets; each offset, row
// and chunk included, is the per-lane VGPR offset, which the range check
// covers).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "gemv_kernels.hpp"
#include "gemv_lpr_args.hpp"
#include "gemv_tile.hpp"

namespace prism {

// Epilogues of k_gemv_lpr.
constexpr int kLprPlain = 0;   // y[b][row] = f16(acc)
constexpr int kLprSwiglu = 1;  // NM = 2: y[row] = swiglu(f16(gate), f16(up))
constexpr int kLprPair = 2;    // NM = 2: y[row] = f16(gate), y2[row] = f16(up)

// Chunk loads of a wave whose chunk count is a compile-time constant (NCH):
// kLprFirst requested before the table build, then kLprAhead ahead of the
// chunk being looked up (the first kLprFirst - kLprAhead chunks request
// nothing), with x in scalar blocks of kLprXBlock chunks.  Hero shape,
// MI355X, timing copies on one box: x blocks of 4 chunks, (first, ahead) =
// (6, 5) 6.59-6.60 us against 6.88-6.91 for the run-time loop with 4 in
// flight; (4, 4) 6.72-6.77, (8, 4) 6.62-6.67, (10, 4) 6.96-6.99, (12, 4)
// 7.41, everything first 8.17; x blocks of 2 chunks on another box: (5, 5)
// 6.49-6.65 and (4, 4) 6.52-6.60 against 6.62-6.68 for (6, 5) with blocks of
// 4; blocks of 1 or 8, or double-buffered x, were slower.  The
// straight-line sequence is part of the gain: (4, 4) unrolled beats the loop.
constexpr int kLprFirst = 5;
constexpr int kLprAhead = 5;
constexpr int kLprXBlock = 2;
// The half-group form (HG below) runs two workgroups per CU and prefers a
// shallower ring: config 2 (NCH = 14) 13.58-13.71 us with (4, 4) against
// 13.68-13.79 with (5, 5), three alternating rounds on one box ((6, 5),
// (6, 6) and 4-chunk x blocks in between); the hero kept (5, 5): 6.40-6.41
// against 6.46-6.54 for each of those.
constexpr int kLprHgFirst = 4;
constexpr int kLprHgAhead = 4;

// HG (half-groups, G = 32): lanes 0..31 and 32..63 of every wave take the 32
// rows of two different groups, each lane still one row, all 64 tables in
// one bank-private set: NM = 2, group g of the gate matrix in lanes 0..31
// and group g of the up matrix in lanes 32..63 (workgroup g), so gate and up
// of the same rows meet in one workgroup with one 64 KB table set; NM = 1,
// groups 2g and 2g + 1 of one matrix (workgroup g).  Used where a matrix has
// more than 64 rows per CU (64 KB of tables per 64 rows: two workgroups per
// CU fill the LDS).  With NM = 2 the two matrices may lie anywhere, so
// the loads are global loads from a per-lane 64-bit pointer (lanes 0..31
// the gate matrix, 32..63 the up matrix) instead of buffer loads: every
// lane's row exists in memory (the last group is zero-padded), and a
// chunk load past the wave's range (the run-time loop's last ring slots)
// re-reads the lane's first chunk instead of relying on the range check.
// (One buffer descriptor per matrix, each load issued twice with the other
// half's offsets out of range, took 19.6 against 13.9 us on config 2.)
template <int S, int NM, int NB, int EPI, int NCH = 0, bool HG = false>
__device__ __forceinline__ void lpr_body(const LprArgs& a) {
  static_assert(S == 4 || S == 8 || S == 16, "waves per group");
  static_assert(NM == 1 || NM == 2, "one matrix or gate + up");
  static_assert(NB == 1 || NB == 2, "batch vectors per pass");
  static_assert(EPI == kLprPlain || (NM == 2 && NB == 1), "gate/up epilogues are single-vector");
  constexpr int NT = HG ? 1 : NM;  // table sets (64 KB each) and per-lane streams
  constexpr bool SPLIT = HG && NM == 2;  // lanes 0..31 and 32..63 in two matrices
  // x chunks per scalar block (16 SGPRs per chunk and vector).  Chunk loads:
  // a ring of R slots (chunk c in slot c % R), chunk c + DR requested once
  // chunk c's table addresses are formed.  NCH = 0 (chunks per wave known at
  // run time): R = DR = XB, a loop over x blocks; NCH > 0 (the host launches
  // it only when the wave's chunk count is NCH): kLprFirst / kLprAhead, one
  // straight-line sequence.
  constexpr int XB = NCH > 0 ? kLprXBlock : (NT == 1 && NB == 1) ? 4 : 2;
  constexpr int FIRST = HG ? kLprHgFirst : kLprFirst, AHEAD = HG ? kLprHgAhead : kLprAhead;
  constexpr int R = NCH == 0 ? XB : (NCH < FIRST ? NCH : FIRST);
  constexpr int DR = NCH == 0 ? XB : (R < AHEAD ? R : AHEAD);
  constexpr int LO = 16 / S;  // low nibbles of the table entries a thread builds
  typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));
  typedef uint32_t u32x16 __attribute__((ext_vector_type(16)));
  // static LDS: the tables' address is a link-time constant, so a lookup
  // needs no per-read add
  __shared__ uint32_t lds[NT * kLprTableDw + S * NT * NB * 64];
  float* red = reinterpret_cast<float*>(lds + NT * kLprTableDw);

  const uint32_t lane = threadIdx.x & 63;
  const uint32_t w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t N = a.N, K = a.K, NC = K / 32;
  const uint32_t G = a.G;
  const uint32_t c0 = (w * NC) / S, nch = ((w + 1) * NC) / S - c0;
  // The half-group form with NCH > 0 (launched only when every wave has NCH
  // chunks) takes the count as a compile-time constant, so the ring's and
  // the x blocks' range checks fold (the run-time count costs each refill a
  // compare and selects): config 2 13.56-13.61 against 13.65-13.71 us, three
  // alternating rounds on one box.  The one-group form keeps the run-time
  // count: with the constant the hero took 6.82-6.85 against 6.40-6.45 us in
  // the same rounds (its schedule moved), config 4's 8-bit form no faster.
  const uint32_t nchk = (HG && NCH > 0) ? (uint32_t)NCH : nch;
  const uint32_t gbytes = G * 32u + G * (K / 2);
  const uint32_t nbytes = ((N + G - 1) / G) * gbytes;
  // the lane's group, its row in the group and the group's byte offset
  // from the descriptor's base
  uint32_t g, lr, gbase;
  bool live;
  __amdgpu_buffer_rsrc_t ri[NT];  // SPLIT: unused
  if constexpr (!HG) {
    g = blockIdx.x;
    lr = lane;
    live = lane < G;
    gbase = g * gbytes;
#pragma unroll
    for (int m = 0; m < NM; m++)
      ri[m] = __builtin_amdgcn_make_buffer_rsrc((void*)(m == 0 ? a.w : a.w2), (short)0, (int)nbytes, kBufferWord3);
  } else if constexpr (NM == 1) {
    // groups 2 blockIdx.x and 2 blockIdx.x + 1; one past the last group
    // reads zeros (its offsets are past the range) and stores nothing
    g = 2 * blockIdx.x + (lane >> 5);
    lr = lane & 31;
    live = true;
    gbase = g * gbytes;
    ri[0] = __builtin_amdgcn_make_buffer_rsrc((void*)a.w, (short)0, (int)nbytes, kBufferWord3);
  } else {
    // group blockIdx.x of the gate matrix (lanes 0..31) and of the up
    // matrix (lanes 32..63)
    g = blockIdx.x;
    lr = lane & 31;
    live = true;
    gbase = g * gbytes;
  }
  const uint32_t row = g * G + lr;
  // SPLIT: the lane's matrix, addressed per lane
  const uint8_t* const lp = SPLIT ? (lane >= 32 ? a.w2 : a.w) : nullptr;
  // 16-byte load of stream m at offset o (LUT loads: default policy; index
  // chunks: nontemporal)
  auto ld_lut = [&](int m, uint32_t o) -> u32x4v {
    if constexpr (SPLIT)
      return *reinterpret_cast<const u32x4v*>(lp + o);
    else
      return __builtin_amdgcn_raw_buffer_load_b128(ri[m], o, 0u, 0);
  };
  auto ld_idx = [&](int m, uint32_t o) -> u32x4v {
    if constexpr (SPLIT)
      return __builtin_nontemporal_load(reinterpret_cast<const u32x4v*>(lp + o));
    else
      return __builtin_amdgcn_raw_buffer_load_b128(ri[m], o, 0u, kNontemporal);
  };

  // ---- the LUT of the lane's row: 8 dwords, two 16-byte loads and nothing
  // else (the table build waits for them: a separate load of the low-nibble
  // entries a wave needs cost 0.4 us on the hero shape; they are picked out
  // of these registers below).  Lanes past N read the zero LUT slots of the
  // last group's padding rows; lanes past G get an offset past the buffer's
  // range and read zeros.
  uint32_t L[NT][8];
  const uint32_t lo = live ? gbase + lr * 32u : 0x80000000u;
#pragma unroll
  for (int m = 0; m < NT; m++) {
    const u32x4v l0 = ld_lut(m, lo);
    const u32x4v l1 = ld_lut(m, lo + 16u);
    L[m][0] = l0.x; L[m][1] = l0.y; L[m][2] = l0.z; L[m][3] = l0.w;
    L[m][4] = l1.x; L[m][5] = l1.y; L[m][6] = l1.z; L[m][7] = l1.w;
  }

  // ---- index chunks: a ring of P per matrix.  Every load is issued
  // unconditionally, so the wait counts are static; a chunk past the wave's
  // range, and every chunk of a lane past G, gets an offset past the
  // buffer's range, which the range check turns into zeros without a
  // memory access.
  const uint32_t cstride = G * kGiChunk;  // bytes from chunk c to c + 1 of a row
  const uint32_t vbase = live ? gbase + G * 32u + (c0 * G + lr) * kGiChunk : 0x80000000u;
  u32x4v ring[R][NT];
  auto ldc = [&](uint32_t i, u32x4v (&dst)[NT]) {
    const uint32_t vo = i < nchk ? vbase + i * cstride : SPLIT ? vbase : 0x80000000u;
#pragma unroll
    for (int m = 0; m < NT; m++) dst[m] = ld_idx(m, vo);
  };
#pragma unroll
  for (int u = 0; u < R; u++) ldc(u, ring[u]);

  // ---- first x block (scalar loads; x rows are read past the wave's range
  // only inside the row, so no guard is needed for them)
  // (vectors past nb read vector 0; one base pointer and scalar row offsets:
  // two vectors' pointers spilled SGPRs, 7.11 -> 7.05 us at two vectors)
  const u32x16* xw = reinterpret_cast<const u32x16*>(a.x) + c0;
  const uint32_t xrow = K / 32;  // 64-byte x chunks per vector
  u32x16 xs[NB][XB];
  auto ldx = [&](uint32_t i) {
#pragma unroll
    for (int b = 0; b < NB; b++)
#pragma unroll
      for (int u = 0; u < XB; u++)
        xs[b][u] = xw[((uint32_t)b < a.nb ? (uint32_t)b : 0u) * xrow + (i + u < nchk ? i + u : 0)];
  };
  ldx(0);

  // ---- bank-private pair tables.  The wave builds entries e = w + S i:
  // low nibble w + S (i % LO), high nibble i / LO.  Its LO low-nibble fp16
  // values are LUT entries w + S j, selected from L with the wave-uniform w.
  uint32_t hv[NT][LO];
#pragma unroll
  for (int m = 0; m < NT; m++)
#pragma unroll
    for (int j = 0; j < LO; j++) {
      const uint32_t e = w + S * j;
      uint32_t d = L[m][0];
#pragma unroll
      for (int q = 1; q < 8; q++) d = (e >> 1) == (uint32_t)q ? L[m][q] : d;
      hv[m][j] = (e & 1) ? (d >> 16) : (d & 0xFFFFu);
    }
#pragma unroll
  for (int m = 0; m < NT; m++)
#pragma unroll
    for (int i = 0; i < 256 / S; i++) {
      const int hi = i / LO;
      const uint32_t v = __builtin_amdgcn_perm(L[m][hi >> 1], hv[m][i % LO], (hi & 1) ? 0x07060100u : 0x05040100u);
      lds[m * kLprTableDw + (w + S * i) * 64 + lane] = v;
    }
  __syncthreads();
  __builtin_amdgcn_sched_barrier(0);

  // ---- lookups and products.  Chunk c uses ring slot `slot` and x block
  // entry `xu`; with `refill`, chunk c + DR is requested into its slot once
  // chunk c's table addresses are formed.
  const uint32_t lanebase = lane * 4u;
  float acc[NT][NB][2];
#pragma unroll
  for (int m = 0; m < NT; m++)
#pragma unroll
    for (int b = 0; b < NB; b++) acc[m][b][0] = acc[m][b][1] = 0.0f;
  auto chunk = [&](uint32_t c, int slot, int xu, bool refill) {
    uint32_t pr[NT][16];
#pragma unroll
    for (int m = 0; m < NT; m++)
#pragma unroll
      for (int j = 0; j < 16; j++) {
        const uint32_t ad = __builtin_amdgcn_perm(ring[slot][m][j >> 2], lanebase, 0x0C0C0000u | ((4u + (j & 3)) << 8));
        pr[m][j] = *reinterpret_cast<const uint32_t*>(reinterpret_cast<const char*>(lds + m * kLprTableDw) + ad);
      }
    if (refill) ldc(c + DR, ring[(slot + DR) % R]);
#pragma unroll
    for (int m = 0; m < NT; m++)
#pragma unroll
      for (int b = 0; b < NB; b++)
#pragma unroll
        for (int j = 0; j < 16; j++) acc[m][b][j & 1] = dot2(pr[m][j], xs[b][xu][j], acc[m][b][j & 1]);
    __builtin_amdgcn_sched_barrier(0);
  };
  if constexpr (NCH > 0) {
#pragma unroll
    for (int c = 0; c < NCH; c++) {
      if (c % XB == 0 && c != 0) ldx(c);
      chunk(c, c % R, c % XB, c >= R - DR && c + DR < NCH);
    }
  } else {
    // full blocks of XB chunks run without branches; the last partial block
    // skips its missing chunks
    const uint32_t nfull = nch / XB;
    uint32_t i = 0;
    for (uint32_t it = 0; it < nfull; it++, i += XB) {
      if (it != 0) ldx(i);
#pragma unroll
      for (int u = 0; u < XB; u++) chunk(i + u, u, u, true);
    }
    if (i < nch) {
      if (i != 0) ldx(i);
#pragma unroll
      for (int u = 0; u < XB - 1; u++)
        if (i + u < nch) chunk(i + u, u, u, true);
    }
  }

  // ---- wave partials -> LDS -> rows (waves 0 .. NB-1 finish one vector each)
#pragma unroll
  for (int m = 0; m < NT; m++)
#pragma unroll
    for (int b = 0; b < NB; b++) red[((w * NT + m) * NB + b) * 64 + lane] = acc[m][b][0] + acc[m][b][1];
  __syncthreads();
  if (w < (uint32_t)NB) {
    const uint32_t b = w;
    float s[NT];
#pragma unroll
    for (int m = 0; m < NT; m++) {
      s[m] = 0.0f;
#pragma unroll
      for (int v = 0; v < S; v++) s[m] += red[((v * NT + m) * NB + b) * 64 + lane];
    }
    if constexpr (HG && NM == 2) {
      // lane r < 32: the gate row's sum; lane r + 32: the same row's up sum,
      // added in the same wave order
      if constexpr (EPI == kLprSwiglu) {
        float su = 0.0f;
#pragma unroll
        for (int v = 0; v < S; v++) su += red[v * 64 + (lane ^ 32u)];
        if (lane < 32 && row < N) store_out(a.y + row, swiglu_h(s[0], su));
      } else if (row < N) {
        store_out((lane < 32 ? a.y : a.y2) + row, f2h(s[0]));
      }
    } else if (live && row < N && b < a.nb) {
      if constexpr (EPI == kLprSwiglu)
        store_out(a.y + row, swiglu_h(s[0], s[1]));
      else if constexpr (EPI == kLprPair) {
        store_out(a.y + row, f2h(s[0]));
        store_out(a.y2 + row, f2h(s[1]));
      } else
        store_out(a.y + (size_t)b * N + row, f2h(s[0]));
    }
  }
}

template <int S, int NM, int NB, int EPI, int NCH = 0>
__global__ __launch_bounds__(64 * S) void k_gemv_lpr(const uint8_t* w, const uint8_t* w2, const uint16_t* x,
                                                     uint16_t* y, uint16_t* y2, uint32_t N, uint32_t K,
                                                     uint32_t nb, uint32_t G) {
  lpr_body<S, NM, NB, EPI, NCH>(lpr_args(w, w2, x, y, y2, N, K, nb, G));
}

// The half-group form (HG above; G = 32): NM = 2 over ceil(N/32) workgroups,
// NM = 1 over ceil(N/64).
template <int S, int NM, int NB, int EPI, int NCH = 0>
__global__ __launch_bounds__(64 * S) void k_gemv_lpr_hg(const uint8_t* w, const uint8_t* w2, const uint16_t* x,
                                                        uint16_t* y, uint16_t* y2, uint32_t N, uint32_t K,
                                                        uint32_t nb, uint32_t G) {
  lpr_body<S, NM, NB, EPI, NCH, true>(lpr_args(w, w2, x, y, y2, N, K, nb, G));
}

// Chunk loads of k_gemv_lpr8 when the wave's chunk count is a compile-time
// constant: first / ahead as for k_gemv_lpr.  cfg4 shape (14336 x 4096,
// 8-bit, 56-row groups), MI355X, timing copies: (5, 5) with 2-chunk x
// blocks 11.83 us, (4, 4) 11.85, (6, 6) 11.88, (8, 8) with 4-chunk blocks
// 12.14; without the nontemporal hint on the index loads 13.57.
constexpr int kLpr8First = 5;
constexpr int kLpr8Ahead = 5;
// Passes of 4 or more vectors (each chunk's lookups feed 4+ products per
// element, and x takes 8 SGPRs per chunk and vector) prefer a shallower
// ring: config 4 at 4 vectors 13.25 against 13.87-13.91 us with (5, 5) on
// one box, 13.76-13.86 against 14.15-14.24 on another ((2, 2), (3, 2), (4, 3),
// (4, 4), (6, 6) and (8, 8) in between or slower); 1 and 2 vectors keep (5, 5).
constexpr int kLpr8FirstWide = 3;
constexpr int kLpr8AheadWide = 3;

// 8-bit lane-per-row GEMV over GI weights (8-bit GI: [G x 512 B LUTs][K/16
// chunks][G rows][16 B]; a chunk holds 16 elements).  The work layout of
// k_gemv_lpr with S = 8 waves: lane l < G owns row G g + l, wave w a
// contiguous 1/8 of the row's chunks, x in SGPRs.
//  * Table: entry b of lane l's 256-entry LUT sits in the low half of LDS
//    dword 64 b + l (bank-private, 64 KB per matrix); one v_perm builds the
//    address from an index byte, one ds_read_b32 returns the fp16 value,
//    and one v_perm packs two of them for v_dot2.  Per element one and a
//    half VALU ops and one LDS read, plus half a v_dot2 per batch vector.  Wave w builds
//    entries 32 w .. 32 w + 31 of every lane's table from its 64-byte slice
//    of the row's LUT.
//  * NB = 1, 2, 4 or 8 vectors a pass (8 SGPRs per chunk and vector).
//  * NCH > 0: the wave's chunk count as a compile-time constant, one
//    straight-line sequence with kLpr8First / kLpr8Ahead; NCH = 0: a loop
//    over blocks of 4 chunks with the next 4 in flight (chunk counts that are
//    multiples of 4).
// Requires K % 512 == 0, 16-byte aligned x and the weight block below 2 GiB.
template <int S, int NM, int NB, int EPI, int NCH = 0>
__device__ __forceinline__ void lpr8_body(const LprArgs& a) {
  static_assert(S == 8, "eight waves: 32 table entries each");
  static_assert(NM == 1 || NM == 2, "one matrix or gate + up");
  static_assert(NB == 1 || NB == 2 || NB == 4 || NB == 8, "batch vectors per pass");
  static_assert(EPI == kLprPlain || (NM == 2 && NB == 1), "gate/up epilogues are single-vector");
  constexpr int XB = NB >= 4 ? 1 : 2;  // x chunks per scalar block (8 SGPRs per chunk and vector)
  constexpr int LB = 4;                // NCH = 0: chunks per loop trip (ring slots)
  constexpr int F8 = NB >= 4 ? kLpr8FirstWide : kLpr8First, A8 = NB >= 4 ? kLpr8AheadWide : kLpr8Ahead;
  constexpr int R = NCH == 0 ? LB : (NCH < F8 ? NCH : F8);
  constexpr int DR = NCH == 0 ? LB : (R < A8 ? R : A8);
  constexpr int EPW = 256 / S;   // table entries each wave builds
  constexpr int LL = EPW / 8;    // 16-byte LUT loads per lane and matrix
  static_assert(NCH == 0 || NCH % XB == 0, "whole x blocks");
  typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));
  typedef uint32_t u32x8 __attribute__((ext_vector_type(8)));
  __shared__ uint32_t lds[NM * kLprTableDw + S * NM * NB * 64];
  float* red = reinterpret_cast<float*>(lds + NM * kLprTableDw);

  const uint32_t lane = threadIdx.x & 63;
  const uint32_t w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t g = blockIdx.x;
  const uint32_t N = a.N, K = a.K, NC = K / 16;
  const uint32_t G = a.G;
  const uint32_t row = g * G + lane;
  const bool live = lane < G;
  const uint32_t nch = NC / S, c0 = w * nch;
  const uint32_t gbytes = G * 512u + G * K;
  const uint32_t gbase = g * gbytes;
  const uint32_t nbytes = gridDim.x * gbytes;  // one workgroup per group
  __amdgpu_buffer_rsrc_t ri[NM];
#pragma unroll
  for (int m = 0; m < NM; m++)
    ri[m] = __builtin_amdgcn_make_buffer_rsrc((void*)(m == 0 ? a.w : a.w2), (short)0, (int)nbytes, kBufferWord3);

  // ---- this wave's 64-byte slice of the LUT of the lane's row (lanes past
  // G read zeros through the range check; lanes past N the zero LUTs of the
  // last group's padding rows)
  u32x4v L[NM][LL];
  const uint32_t lo = live ? gbase + lane * 512u + w * (EPW * 2u) : 0x80000000u;
#pragma unroll
  for (int m = 0; m < NM; m++)
#pragma unroll
    for (int i = 0; i < LL; i++) L[m][i] = __builtin_amdgcn_raw_buffer_load_b128(ri[m], lo + 16u * i, 0u, 0);

  // ---- index chunks (unconditional loads; past the wave's range the offset
  // is past the buffer's range and reads zeros without a memory access)
  const uint32_t cstride = G * kGiChunk;
  const uint32_t vbase = live ? gbase + G * 512u + (c0 * G + lane) * kGiChunk : 0x80000000u;
  u32x4v ring[R][NM];
  auto ldc = [&](uint32_t i, u32x4v (&dst)[NM]) {
    const uint32_t vo = i < nch ? vbase + i * cstride : 0x80000000u;
#pragma unroll
    for (int m = 0; m < NM; m++) dst[m] = __builtin_amdgcn_raw_buffer_load_b128(ri[m], vo, 0u, kNontemporal);
  };
#pragma unroll
  for (int u = 0; u < R; u++) ldc(u, ring[u]);

  // x of vector b (vectors past nb read vector 0): one base pointer and
  // scalar row offsets, so eight vectors' pointers do not hold 16 SGPRs
  const u32x8* xw = reinterpret_cast<const u32x8*>(a.x) + c0;
  const uint32_t xrow = K / 16;  // 32-byte x chunks per vector
  u32x8 xs[NB][XB];
  auto ldx = [&](uint32_t i) {
#pragma unroll
    for (int b = 0; b < NB; b++)
#pragma unroll
      for (int u = 0; u < XB; u++) xs[b][u] = xw[((uint32_t)b < a.nb ? (uint32_t)b : 0u) * xrow + i + u];
  };
  ldx(0);

  // ---- bank-private tables: entry e at dword 64 e + lane, LUT[e] in the low half
#pragma unroll
  for (int m = 0; m < NM; m++)
#pragma unroll
    for (int i = 0; i < LL; i++)
#pragma unroll
      for (int q = 0; q < 4; q++) {
        const uint32_t d = L[m][i][q];
        const uint32_t e = w * EPW + 8 * i + 2 * q;
        lds[m * kLprTableDw + e * 64 + lane] = d & 0xFFFFu;
        lds[m * kLprTableDw + (e + 1) * 64 + lane] = d >> 16;
      }
  __syncthreads();
  __builtin_amdgcn_sched_barrier(0);

  const uint32_t lanebase = lane * 4u;
  float acc[NM][NB][2];
#pragma unroll
  for (int m = 0; m < NM; m++)
#pragma unroll
    for (int b = 0; b < NB; b++) acc[m][b][0] = acc[m][b][1] = 0.0f;
  auto chunk = [&](uint32_t c, int slot, int xu, bool refill) {
    uint32_t v[NM][16];
#pragma unroll
    for (int m = 0; m < NM; m++)
#pragma unroll
      for (int j = 0; j < 16; j++) {
        const uint32_t ad = __builtin_amdgcn_perm(ring[slot][m][j >> 2], lanebase, 0x0C0C0000u | ((4u + (j & 3)) << 8));
        v[m][j] = *reinterpret_cast<const uint32_t*>(reinterpret_cast<const char*>(lds + m * kLprTableDw) + ad);
      }
    if (refill) ldc(c + DR, ring[(slot + DR) % R]);
#pragma unroll
    for (int m = 0; m < NM; m++)
#pragma unroll
      for (int p = 0; p < 8; p++) {
        const uint32_t pr = __builtin_amdgcn_perm(v[m][2 * p + 1], v[m][2 * p], 0x05040100u);
#pragma unroll
        for (int b = 0; b < NB; b++) acc[m][b][p & 1] = dot2(pr, xs[b][xu][p], acc[m][b][p & 1]);
      }
    __builtin_amdgcn_sched_barrier(0);
  };
  if constexpr (NCH > 0) {
#pragma unroll
    for (int c = 0; c < NCH; c++) {
      if (c % XB == 0 && c != 0) ldx(c);
      chunk(c, c % R, c % XB, c >= R - DR && c + DR < NCH);
    }
  } else {
    for (uint32_t i = 0; i < nch; i += LB) {
#pragma unroll
      for (int u = 0; u < LB; u++) {
        if (u % XB == 0 && (i != 0 || u != 0)) ldx(i + u);
        chunk(i + u, u, u % XB, true);
      }
    }
  }

  // ---- wave partials -> LDS -> rows (waves 0 .. NB-1 finish one vector each)
#pragma unroll
  for (int m = 0; m < NM; m++)
#pragma unroll
    for (int b = 0; b < NB; b++) red[((w * NM + m) * NB + b) * 64 + lane] = acc[m][b][0] + acc[m][b][1];
  __syncthreads();
  if (w < (uint32_t)NB) {
    const uint32_t b = w;
    float s[NM];
#pragma unroll
    for (int m = 0; m < NM; m++) {
      s[m] = 0.0f;
#pragma unroll
      for (int v = 0; v < S; v++) s[m] += red[((v * NM + m) * NB + b) * 64 + lane];
    }
    if (live && row < N && b < a.nb) {
      if constexpr (EPI == kLprSwiglu)
        a.y[row] = swiglu_h(s[0], s[1]);
      else if constexpr (EPI == kLprPair) {
        a.y[row] = f2h(s[0]);
        a.y2[row] = f2h(s[1]);
      } else
        a.y[(size_t)b * N + row] = f2h(s[0]);
    }
  }
}

template <int S, int NM, int NB, int EPI, int NCH = 0>
__global__ __launch_bounds__(64 * S) void k_gemv_lpr8(const uint8_t* w, const uint8_t* w2, const uint16_t* x,
                                                      uint16_t* y, uint16_t* y2, uint32_t N, uint32_t K,
                                                      uint32_t nb, uint32_t G) {
  lpr8_body<S, NM, NB, EPI, NCH>(lpr_args(w, w2, x, y, y2, N, K, nb, G));
}

// k_gemv_lpr8m and k_gemv_lpr4m, the 8- and 4-bit GEMVs of 3..8 vectors
// with these lookups feeding the matrix cores (and k_gemv_lpr4q), are built in their own
// translation unit (gemv_lpr8m.hip) with the max-ilp machine scheduler;
// these launch them on `st`.
hipError_t launch_gemv_lpr8m(dim3 groups, hipStream_t st, const LprArgs& a);
hipError_t launch_gemv_lpr4m(dim3 groups, hipStream_t st, const LprArgs& a);
// k_gemv_lpr4q (the same unit): the 4-bit GEMV of 3..4 vectors with the
// products on the matrix cores' 4 x 4 x 4 blocks.
hipError_t launch_gemv_lpr4q(dim3 groups, hipStream_t st, const LprArgs& a);

// Split-block payload (LUT block then index rows) -> GI with G rows per
// group, 4- or 8-bit.  One thread per 16-byte piece of the GI block, in GI
// order: the writes are contiguous, the reads 16 bytes each.  Rows past N
// get zero LUTs and zero indices.
__global__ __launch_bounds__(256) void k_gi_pack(const uint8_t* __restrict__ src, uint8_t* __restrict__ dst,
                                                 uint32_t N, uint32_t K, uint32_t G, uint32_t bits) {
  const uint32_t lp = gi_lut_bytes(bits) / 16;  // 16-byte pieces of one row's LUT
  const uint32_t rb = K * bits / 8;             // index bytes per row
  const uint32_t NC = rb / kGiChunk;
  const uint32_t per_group = lp * G + NC * G;  // 16-byte pieces per group
  const size_t total = (size_t)((N + G - 1) / G) * per_group;
  const uint8_t* sidx = src + (size_t)N * gi_lut_bytes(bits);
  for (size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x; t < total; t += (size_t)gridDim.x * blockDim.x) {
    const uint32_t g = (uint32_t)(t / per_group), p = (uint32_t)(t % per_group);
    uint4 v = make_uint4(0, 0, 0, 0);
    if (p < lp * G) {  // LUT piece p % lp of row p / lp
      const uint32_t r = g * G + p / lp;
      if (r < N) v = *reinterpret_cast<const uint4*>(src + (size_t)r * gi_lut_bytes(bits) + (p % lp) * 16);
    } else {
      const uint32_t q = p - lp * G, c = q / G, r = g * G + q % G;
      if (r < N) v = *reinterpret_cast<const uint4*>(sidx + (size_t)r * rb + (size_t)c * kGiChunk);
    }
    *reinterpret_cast<uint4*>(dst + t * 16) = v;
  }
}

// GI -> split-block rows: LUTs to dst_lut ([N][32] B), index rows to
// dst_idx ([N][K/2] B), for consumers that keep split-block rows (the
// decode-step model's own weight copies).
__global__ __launch_bounds__(256) void k_gi_unpack(const uint8_t* __restrict__ src, uint8_t* __restrict__ dst_lut,
                                                   uint8_t* __restrict__ dst_idx, uint32_t N, uint32_t K, uint32_t G) {
  const uint32_t NC = K / 32;
  const size_t pieces = (size_t)N * (2 + NC);  // per row: 2 LUT pieces + NC chunks
  for (size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x; t < pieces; t += (size_t)gridDim.x * blockDim.x) {
    const uint32_t r = (uint32_t)(t / (2 + NC)), p = (uint32_t)(t % (2 + NC));
    if (p < 2)
      *reinterpret_cast<uint4*>(dst_lut + (size_t)r * 32 + p * 16) =
          *reinterpret_cast<const uint4*>(src + gi_lut_offset(G, r, K, 4) + p * 16);
    else
      *reinterpret_cast<uint4*>(dst_idx + (size_t)r * (K / 2) + (size_t)(p - 2) * kGiChunk) =
          *reinterpret_cast<const uint4*>(src + gi_chunk_offset(G, r, p - 2, K, 4));
  }
}

}  // namespace prism
