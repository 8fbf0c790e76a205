// gemv_lpr_args.hpp -- the argument block of the lane-per-row GEMVs
// (gemv_lpr.hpp, gemv_lpr8m.hip) and the constants both translation units
// use.  No kernels: it is included by more than one translation unit.
#pragma once
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

// k_gemv_lpr8m (gemv_lpr8m.hip): double steps of index bytes in flight per
// wave, and x's LDS layout (each vector followed by kLpr8mXPad dwords).
constexpr int kLpr8mAhead = 4;
constexpr int kLpr8mXPad = 4;       // dwords after each vector of x in LDS
constexpr int kLpr8mXDw = 16512;  // LDS dwords for x: nb * (K / 2 + kLpr8mXPad) <= kLpr8mXDw

// Records a launched kernel (by host function) in the launch log of the
// compute call running on this thread, if any (prism_hip.hip).
void note_launch(const void* fn);

}  // namespace prism
