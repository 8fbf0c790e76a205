// gemv_lpr_args.hpp -- the argument block of the lane-per-row GEMVs
// (gemv_lpr.hpp, gemv_lpr8m.hip) and the constants both translation units
// use.  No kernels: it is included by more than one translation unit.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace prism {

constexpr int kLprTableDw = 256 * 64;  // dwords of one workgroup's pair tables (64 KB, one per lane)

struct LprArgs {
  const uint8_t* w;    // GI weights
  const uint8_t* w2;   // NM = 2: up matrix, same shape
  const uint16_t* x;   // [nb][K] fp16
  uint16_t* y;         // [nb][N]
  uint16_t* y2;        // kLprPair: up output [N]
  uint32_t N;
  uint32_t K;
  uint32_t nb;         // live batch vectors (<= NB)
  uint32_t G;          // rows per group (<= 64)
};

// The lane-per-row kernels take these fields as separate scalar arguments
// (14 dwords, in this order) rather than as one struct: the library is built
// with -amdgpu-kernarg-preload-count=16, so scalar arguments arrive in SGPRs
// at wave launch and a wave's first weight requests do not wait for a load
// of its arguments from memory (a struct argument is never preloaded).
// MI355X, hero shape, graph-launched: 6.45 -> 6.40 us; the read floor 5.69
// -> 5.60 us.
__device__ __forceinline__ LprArgs lpr_args(const uint8_t* w, const uint8_t* w2, const uint16_t* x, uint16_t* y,
                                            uint16_t* y2, uint32_t N, uint32_t K, uint32_t nb, uint32_t G) {
  LprArgs a;
  a.w = w;
  a.w2 = w2;
  a.x = x;
  a.y = y;
  a.y2 = y2;
  a.N = N;
  a.K = K;
  a.nb = nb;
  a.G = G;
  return a;
}

// k_gemv_lpr8m (gemv_lpr8m.hip): double steps of index bytes in flight per
// wave, and x's LDS layout (each vector followed by kLpr8mXPad dwords).
constexpr int kLpr8mAhead = 4;
constexpr int kLpr8mXPad = 4;       // dwords after each vector of x in LDS
constexpr int kLpr8mXDw = 16512;  // LDS dwords for x: nb * (K / 2 + kLpr8mXPad) <= kLpr8mXDw

// k_gemv_lpr4q (gemv_lpr8m.hip): chunk loads of a wave whose chunk count is
// a compile-time constant, requested first and kept ahead of the lookups
// (as k_gemv_lpr's kLprFirst / kLprAhead), and the run-time loop's ring
// (blocks of kLpr4qRing chunks, the next block in flight).
constexpr int kLpr4qFirst = 5;
constexpr int kLpr4qAhead = 5;
constexpr int kLpr4qRing = 4;

// Records a launched kernel (by host function) in the launch log of the
// compute call running on this thread, if any (prism_hip.hip).
void note_launch(const void* fn);

}  // namespace prism
