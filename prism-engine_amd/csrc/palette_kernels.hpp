// palette_kernels.hpp -- the palette compiler on the GPU: per-row k-means
// palettization of an fp32 weight matrix into the split-block payload.
//
// Reference: palettize_matrix (src/quantization/palette.rs:230-272) calling
// fit_palette (:75-183) and encode_channel (:198-228) for every row, then
// compile_to_cimage's payload assembly (src/lut/compiler.rs:47-60): per row
// 16 fp16 LUT entries (zero past k), then every row's packed indices,
// (n+1)/2 bytes per row.
//
// One wave per row; the row and its scratch live in LDS (or, for rows too
// long for LDS, in a global workspace).  The result is the reference's byte
// for byte: every fp32 operation happens in the reference's order where the
// order changes the result, and in parallel only where it cannot:
//  * k-means++ picks (from channel[n/2], golden-ratio thresholds): the
//    min-distance update is per element (parallel over lanes); the total is
//    a sequential fp32 fold in element order (a chain of adds handed from
//    lane to lane) that also stores every partial sum; those partial sums are
//    the reference's cumulative scan, and
//    since they never decrease (non-negative terms, monotone rounding) the
//    first one >= the threshold is found by binary search;
//  * Lloyd iterations: the assignment (first strictly smallest squared
//    distance) is per element (parallel); the per-cluster sums are
//    sequential folds in element order, one lane per cluster, adding +0.0
//    for elements of other clusters (an exact no-op: the running sum starts
//    at +0 and never becomes -0); centroid = sum / count; exit once no
//    centroid moved by 0.001 or more;
//  * a stable sort by magnitude, descending; encoding (first strictly
//    nearest entry) per element; fp16 by RNE.
// Arrays are padded to 16 elements (zeros; assignment 0xFF) so the
// sequential folds read whole 16-element blocks; padding adds +0.0 and
// belongs to no cluster.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "gemv_kernels.hpp"

namespace prism {

constexpr int kPaletteMaxK = 16;

// Calibration seeds (compute-core/src/quantization/palette.rs:94-116): the
// first min(n, k) centroids of every row; n == 0 starts from channel[n/2]
// (the root crate's fit_palette).
struct PaletteSeeds {
  float v[kPaletteMaxK];
  uint32_t n;
};

__host__ __device__ constexpr uint32_t palette_pad(uint32_t n) { return (n + 15u) & ~15u; }
// Per row: values, min-distances (reused as byte assignments in the Lloyd
// iterations) and partial sums, palette_pad(n) floats each.
__host__ __device__ constexpr size_t palette_row_bytes(uint32_t n) { return (size_t)palette_pad(n) * 12; }

// Sequential fp32 fold of v[0..np) (np % 16 == 0) in element order,
// storing each partial sum; called by the whole wave.  Lane l holds the 16
// consecutive elements 1024 p + 16 l .. +15 of pass p in registers; the
// running sum passes from lane to lane (readlane), so the chain of adds runs
// in registers instead of waiting on an LDS read every 16 elements.  The
// additions and their order are those of one lane folding v[0], v[1], ...
__device__ __forceinline__ float palette_fold_prefix(const float* v, float* pre, uint32_t np, uint32_t lane) {
#pragma clang fp contract(off)
  float carry = 0.0f;
  for (uint32_t c0 = 0; c0 < np; c0 += 1024) {
    const uint32_t base = c0 + 16 * lane;
    const bool live = base < np;
    float t[16];
#pragma unroll
    for (int q = 0; q < 4; q++) {
      const float4 f = live ? reinterpret_cast<const float4*>(v + base)[q] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      t[4 * q] = f.x;
      t[4 * q + 1] = f.y;
      t[4 * q + 2] = f.z;
      t[4 * q + 3] = f.w;
    }
    const uint32_t lanes = (np - c0) / 16 < 64u ? (np - c0) / 16 : 64u;
    for (uint32_t l = 0; l < lanes; l++) {
      if (lane == l) {
        float s = carry;
#pragma unroll
        for (int j = 0; j < 16; j++) {
          s += t[j];
          t[j] = s;
        }
      }
      carry = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, t[15]), l));
    }
    if (live) {
#pragma unroll
      for (int q = 0; q < 4; q++)
        reinterpret_cast<float4*>(pre + base)[q] = make_float4(t[4 * q], t[4 * q + 1], t[4 * q + 2], t[4 * q + 3]);
    }
  }
  return carry;
}

// Index of the first entry of the non-decreasing pre[0..n) that is >= t,
// or 0 when there is none (the reference's pick when its scan runs out).
__device__ __forceinline__ uint32_t palette_first_at_least(const float* pre, uint32_t n, float t) {
  uint32_t lo = 0, hi = n;
  while (lo < hi) {
    const uint32_t mid = (lo + hi) >> 1;
    if (pre[mid] >= t)
      hi = mid;
    else
      lo = mid + 1;
  }
  return lo < n ? lo : 0u;
}

// First strictly nearest of the k (wave-uniform, <= 16) entries of c.
__device__ __forceinline__ uint32_t palette_nearest(float v, const float (&c)[kPaletteMaxK], uint32_t k) {
  float best = 3.40282347e38f;
  uint32_t bi = 0;
#pragma unroll
  for (uint32_t j = 0; j < (uint32_t)kPaletteMaxK; j++) {
    if (j < k) {
      const float dv = v - c[j];
      const float d = dv * dv;
      if (d < best) {
        best = d;
        bi = j;
      }
    }
  }
  return bi;
}

// Row r = row0 + blockIdx.x.  kLds: the row's arrays in LDS
// (palette_row_bytes(n) dynamic bytes); otherwise in ws, palette_row_bytes(n)
// bytes per row of the launch.  lut_out: 32 bytes per row (16 fp16 entries);
// idx_out: (n+1)/2 bytes per row.
template <bool kLds>
__global__ __launch_bounds__(64) void k_palettize(const float* __restrict__ w, uint32_t n, uint32_t k,
                                                  uint32_t max_iter, PaletteSeeds seeds, uint32_t row0,
                                                  float* __restrict__ ws, uint8_t* __restrict__ lut_out,
                                                  uint8_t* __restrict__ idx_out) {
#pragma clang fp contract(off)
  extern __shared__ float4 sm4[];
  __shared__ float cent[kPaletteMaxK];
  __shared__ float s_new[kPaletteMaxK];
  __shared__ uint32_t s_moved[kPaletteMaxK];

  const uint32_t r = row0 + blockIdx.x, lane = threadIdx.x;
  uint16_t* lut = reinterpret_cast<uint16_t*>(lut_out + (size_t)r * 32);
  if (n == 0) {  // fit_palette returns no entries: an all-zero LUT, no indices
    if (lane < (uint32_t)kPaletteMaxK) lut[lane] = 0;
    return;
  }
  const uint32_t np = palette_pad(n), nb4 = np / 4;
  float* base = kLds ? reinterpret_cast<float*>(sm4) : ws + (size_t)blockIdx.x * (palette_row_bytes(n) / 4);
  float* val = base;
  float* md = base + np;
  float* pre = base + 2 * (size_t)np;
  uint32_t* asg4 = reinterpret_cast<uint32_t*>(md);  // 4 assignment bytes per word
  const float* row = w + (size_t)r * n;
  const float FMAX = 3.40282347e38f;  // f32::MAX
  for (uint32_t i = lane; i < np; i += 64) {
    val[i] = i < n ? row[i] : 0.0f;
    md[i] = i < n ? FMAX : 0.0f;  // padding stays at distance 0
  }
  if (k > n) k = n;
  const uint32_t ns = seeds.n < k ? seeds.n : k;
  if (ns) {
    if (lane < ns) cent[lane] = seeds.v[lane];
  } else if (lane == 0) {
    cent[0] = row[n / 2];
  }
  __syncthreads();

  // ---- k-means++ initialization (its first pass sees only the last seed)
  for (uint32_t nc = ns ? ns : 1; nc < k; nc++) {
    const float last = cent[nc - 1];
    for (uint32_t b = lane; b < nb4; b += 64) {
      const float4 v = reinterpret_cast<const float4*>(val)[b];
      float4 m = reinterpret_cast<const float4*>(md)[b];
      float dv = v.x - last, d = dv * dv;
      if (d < m.x) m.x = d;
      dv = v.y - last, d = dv * dv;
      if (d < m.y) m.y = d;
      dv = v.z - last, d = dv * dv;
      if (d < m.z) m.z = d;
      dv = v.w - last, d = dv * dv;
      if (d < m.w) m.w = d;
      reinterpret_cast<float4*>(md)[b] = m;
    }
    __syncthreads();
    const float total = palette_fold_prefix(md, pre, np, lane);
    __syncthreads();
    if (lane == 0) {
      uint32_t pick;
      if (total <= 0.0f) {
        pick = (uint32_t)(((uint64_t)nc * n / k) % n);
      } else {
        const double x = (double)nc * 0.6180339887498949;
        pick = palette_first_at_least(pre, n, total * (float)(x - trunc(x)));
      }
      cent[nc] = val[pick];
    }
    __syncthreads();
  }

  // ---- Lloyd iterations
  float c[kPaletteMaxK];
  for (uint32_t it = 0; it < max_iter; it++) {
#pragma unroll
    for (int j = 0; j < kPaletteMaxK; j++) c[j] = cent[j];
    for (uint32_t b = lane; b < nb4; b += 64) {
      const float4 v = reinterpret_cast<const float4*>(val)[b];
      uint32_t a = palette_nearest(v.x, c, k) | palette_nearest(v.y, c, k) << 8 |
                   palette_nearest(v.z, c, k) << 16 | palette_nearest(v.w, c, k) << 24;
      const uint32_t i0 = 4 * b;  // padding: no cluster
      if (i0 + 4 > n) a |= 0xFFFFFFFFu << (8 * (n > i0 ? n - i0 : 0));
      asg4[b] = a;
    }
    __syncthreads();
    if (lane < k) {
      float acc = 0.0f;
      uint32_t cnt = 0;
      // block i + 16 is read while block i is folded
      uint4 an = *reinterpret_cast<const uint4*>(asg4);
      float4 tn[4];
#pragma unroll
      for (int q = 0; q < 4; q++) tn[q] = reinterpret_cast<const float4*>(val)[q];
      for (uint32_t i = 0; i < np; i += 16) {
        const uint4 a = an;
        float4 t[4];
#pragma unroll
        for (int q = 0; q < 4; q++) t[q] = tn[q];
        const uint32_t inext = i + 16 < np ? i + 16 : i;  // the last block reads itself again
        an = *reinterpret_cast<const uint4*>(asg4 + inext / 4);
#pragma unroll
        for (int q = 0; q < 4; q++) tn[q] = reinterpret_cast<const float4*>(val + inext)[q];
        const uint32_t aw[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
        for (int q = 0; q < 4; q++) {
          const float tv[4] = {t[q].x, t[q].y, t[q].z, t[q].w};
#pragma unroll
          for (int e = 0; e < 4; e++) {
            const bool mine = ((aw[q] >> (8 * e)) & 0xFFu) == lane;
            acc += mine ? tv[e] : 0.0f;
            cnt += mine ? 1u : 0u;
          }
        }
      }
      // 0: empty cluster (centroid kept); 1: updated; 2: updated and moved
      // by >= 0.001 (a NaN shift counts as not moved, like the max fold).
      s_moved[lane] = 0;
      if (cnt > 0) {
        const float nv = acc / (float)cnt;
        s_new[lane] = nv;
        s_moved[lane] = fabsf(cent[lane] - nv) >= 0.001f ? 2u : 1u;
      }
    }
    __syncthreads();
    bool moved = false;
    for (uint32_t j = 0; j < k; j++) moved |= (s_moved[j] == 2u);
    if (lane < k && s_moved[lane]) cent[lane] = s_new[lane];
    __syncthreads();
    if (!moved) break;  // uniform: every lane read the same flags
  }

  // ---- stable sort by magnitude, descending
  if (lane == 0) {
    for (uint32_t a = 1; a < k; a++) {
      const float v = cent[a];
      uint32_t b = a;
      while (b > 0 && fabsf(cent[b - 1]) < fabsf(v)) {
        cent[b] = cent[b - 1];
        b--;
      }
      cent[b] = v;
    }
  }
  __syncthreads();

  // ---- LUT (fp16, zero past k) and packed indices
#pragma unroll
  for (int j = 0; j < kPaletteMaxK; j++) c[j] = cent[j];
  if (lane < (uint32_t)kPaletteMaxK) lut[lane] = f2h(lane < k ? cent[lane] : 0.0f);
  const uint32_t rb = (n + 1) / 2;
  uint8_t* out = idx_out + (size_t)r * rb;
  for (uint32_t b = lane; b < rb; b += 64) {
    const uint32_t i = 2 * b;
    uint32_t byte = palette_nearest(val[i], c, k);
    if (i + 1 < n) byte |= palette_nearest(val[i + 1], c, k) << 4;
    out[b] = (uint8_t)byte;
  }
}

}  // namespace prism
