// lut_perm.hpp -- register-only decode of a 16-entry fp16 LUT with v_perm_b32.
//
// A row's LUT (16 fp16 = 8 dwords) is held as eight byte planes: the low
// and the high bytes of entries 0-3, 4-7, 8-11 and 12-15.  One index dword
// (8 nibbles, element 2i in the low nibble of byte i) is decoded without
// LDS:
//   * v_perm_b32 selects a byte from an 8-byte window by a 3-bit selector,
//     so each nibble's low 3 bits pick the entry inside the windows
//     {planes 0,1} and {planes 2,3}; bit 3 (spread to a byte mask by one
//     more v_perm) merges the two windows with v_bfi;
//   * that is done for the lo and the hi bytes of the even and the odd
//     nibbles, and two interleaving perms per parity rebuild the fp16
//     values: 25 VALU ops per dword give the pairs (e0,e2) (e4,e6) (e1,e3)
//     (e5,e7); four more perms put them in k order (29 ops).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace prism {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));

struct LutPlanes {
  uint32_t l0, l1, l2, l3, h0, h1, h2, h3;
};

__device__ __forceinline__ uint32_t bsel(uint32_t m, uint32_t a, uint32_t b) { return (a & m) | (b & ~m); }

// ra = LUT dwords 0..3 (entries 0..7), rb = dwords 4..7 (entries 8..15)
__device__ __forceinline__ LutPlanes make_planes(const uint4 ra, const uint4 rb) {
  LutPlanes P;
  P.l0 = __builtin_amdgcn_perm(ra.y, ra.x, 0x06040200u);
  P.h0 = __builtin_amdgcn_perm(ra.y, ra.x, 0x07050301u);
  P.l1 = __builtin_amdgcn_perm(ra.w, ra.z, 0x06040200u);
  P.h1 = __builtin_amdgcn_perm(ra.w, ra.z, 0x07050301u);
  P.l2 = __builtin_amdgcn_perm(rb.y, rb.x, 0x06040200u);
  P.h2 = __builtin_amdgcn_perm(rb.y, rb.x, 0x07050301u);
  P.l3 = __builtin_amdgcn_perm(rb.w, rb.z, 0x06040200u);
  P.h3 = __builtin_amdgcn_perm(rb.w, rb.z, 0x07050301u);
  return P;
}

// 8 nibbles -> fp16 pairs (e0,e2) (e4,e6) (e1,e3) (e5,e7) in o[0..3].
__device__ __forceinline__ void decode_nib8_pairs(uint32_t w, const LutPlanes& P, uint32_t (&o)[4]) {
  const uint32_t se = w & 0x07070707u;
  const uint32_t so = (w >> 4) & 0x07070707u;
  const uint32_t me = __builtin_amdgcn_perm(0xFFFFFFFFu, 0u, (w >> 1) & 0x07070707u);
  const uint32_t mo = __builtin_amdgcn_perm(0xFFFFFFFFu, 0u, (w >> 5) & 0x07070707u);
  const uint32_t le = bsel(me, __builtin_amdgcn_perm(P.l3, P.l2, se), __builtin_amdgcn_perm(P.l1, P.l0, se));
  const uint32_t he = bsel(me, __builtin_amdgcn_perm(P.h3, P.h2, se), __builtin_amdgcn_perm(P.h1, P.h0, se));
  const uint32_t lo = bsel(mo, __builtin_amdgcn_perm(P.l3, P.l2, so), __builtin_amdgcn_perm(P.l1, P.l0, so));
  const uint32_t ho = bsel(mo, __builtin_amdgcn_perm(P.h3, P.h2, so), __builtin_amdgcn_perm(P.h1, P.h0, so));
  o[0] = __builtin_amdgcn_perm(he, le, 0x05010400u);
  o[1] = __builtin_amdgcn_perm(he, le, 0x07030602u);
  o[2] = __builtin_amdgcn_perm(ho, lo, 0x05010400u);
  o[3] = __builtin_amdgcn_perm(ho, lo, 0x07030602u);
}

// 8 nibbles -> one MFMA operand of 8 halves in k order, (e0,e1) (e2,e3)
// (e4,e5) (e6,e7).
__device__ __forceinline__ half8_t decode_nib8_nat(uint32_t w, const LutPlanes& P) {
  uint32_t t[4];
  decode_nib8_pairs(w, P, t);
  typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));
  u32x4v v;
  v.x = __builtin_amdgcn_perm(t[2], t[0], 0x05040100u);
  v.y = __builtin_amdgcn_perm(t[2], t[0], 0x07060302u);
  v.z = __builtin_amdgcn_perm(t[3], t[1], 0x05040100u);
  v.w = __builtin_amdgcn_perm(t[3], t[1], 0x07060302u);
  return __builtin_bit_cast(half8_t, v);
}

}  // namespace prism
