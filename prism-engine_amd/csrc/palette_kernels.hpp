// palette_kernels.hpp -- the palette compiler on the GPU: per-row k-means
// palettization of an fp32 weight matrix into the split-block payload.
//
// Reference: palettize_matrix (src/quantization/palette.rs:230-272) calling
// fit_palette (:75-183) and encode_channel (:198-228) for every row, then
// compile_to_cimage's payload assembly (src/lut/compiler.rs:47-60): per row
// 16 fp16 LUT entries (zero past k), then every row's packed indices,
// (n+1)/2 bytes per row.
//
// One wave per row; the row and its scratch live in LDS.  The result is the
// reference's byte for byte: every fp32 operation happens in the
// reference's order where the order changes the result, and in parallel
// only where it cannot:
//  * k-means++ picks (from channel[n/2], golden-ratio thresholds): the
//    min-distance update is per element (parallel over lanes); the total and
//    the cumulative scan that picks the next centroid are sequential fp32
//    folds in element order (lane 0);
//  * Lloyd iterations: the assignment (first strictly smallest squared
//    distance) is per element (parallel); the per-cluster sums are
//    sequential folds in element order, one lane per cluster, adding +0.0
//    for elements of other clusters (an exact no-op: the running sum starts
//    at +0 and never becomes -0); centroid = sum / count; exit once no
//    centroid moved by 0.001 or more;
//  * a stable sort by magnitude, descending; encoding (first strictly
//    nearest entry) per element; fp16 by RNE.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "gemv_kernels.hpp"

namespace prism {

constexpr int kPaletteMaxK = 16;

// Dynamic LDS bytes of the LDS-resident variant for rows of n elements:
// values, then min-distances (initialization) reused as byte assignments
// (Lloyd iterations).
__host__ __device__ constexpr size_t palette_lds_bytes(uint32_t n) { return (size_t)n * 8; }

// One wave per row r = row0 + blockIdx.x.  kLds: the row and its scratch in
// LDS (palette_lds_bytes(n) dynamic bytes); otherwise values are read from w
// and the scratch is ws[blockIdx.x * n ..] (n floats per row of the launch).
// lut_out: 32 bytes per row (16 fp16 entries); idx_out: (n+1)/2 bytes per row.
template <bool kLds>
__global__ __launch_bounds__(64) void k_palettize(const float* __restrict__ w, uint32_t n, uint32_t k,
                                                  uint32_t max_iter, uint32_t row0, float* __restrict__ ws,
                                                  uint8_t* __restrict__ lut_out, uint8_t* __restrict__ idx_out) {
#pragma clang fp contract(off)
  extern __shared__ float sm[];
  __shared__ float cent[kPaletteMaxK];
  __shared__ float s_new[kPaletteMaxK];
  __shared__ uint32_t s_moved[kPaletteMaxK];

  const uint32_t r = row0 + blockIdx.x, lane = threadIdx.x;
  uint16_t* lut = reinterpret_cast<uint16_t*>(lut_out + (size_t)r * 32);
  if (n == 0) {  // fit_palette returns no entries: an all-zero LUT, no indices
    if (lane < (uint32_t)kPaletteMaxK) lut[lane] = 0;
    return;
  }
  const float* row = w + (size_t)r * n;
  const float FMAX = 3.40282347e38f;  // f32::MAX
  const float* val;
  float* md;
  if constexpr (kLds) {
    float* v = sm;
    md = sm + n;
    for (uint32_t i = lane; i < n; i += 64) v[i] = row[i];
    val = v;
  } else {
    val = row;
    md = ws + (size_t)blockIdx.x * n;
  }
  uint8_t* asg = reinterpret_cast<uint8_t*>(md);
  for (uint32_t i = lane; i < n; i += 64) md[i] = FMAX;
  if (k > n) k = n;
  if (lane == 0) cent[0] = row[n / 2];
  __syncthreads();

  // ---- k-means++ initialization
  for (uint32_t nc = 1; nc < k; nc++) {
    const float last = cent[nc - 1];
    for (uint32_t i = lane; i < n; i += 64) {
      const float dv = val[i] - last;
      const float d = dv * dv;
      if (d < md[i]) md[i] = d;
    }
    __syncthreads();
    if (lane == 0) {
      float total = 0.0f;
      for (uint32_t i = 0; i < n; i++) total += md[i];
      if (total <= 0.0f) {
        cent[nc] = val[(uint32_t)(((uint64_t)nc * n / k) % n)];
      } else {
        const double x = (double)nc * 0.6180339887498949;
        const float target = total * (float)(x - trunc(x));
        float cum = 0.0f;
        uint32_t picked = 0;
        for (uint32_t i = 0; i < n; i++) {
          cum += md[i];
          if (cum >= target) {
            picked = i;
            break;
          }
        }
        cent[nc] = val[picked];
      }
    }
    __syncthreads();
  }

  // ---- Lloyd iterations
  for (uint32_t it = 0; it < max_iter; it++) {
    for (uint32_t i = lane; i < n; i += 64) {
      float best = FMAX;
      uint32_t bc = 0;
      for (uint32_t j = 0; j < k; j++) {
        const float dv = val[i] - cent[j];
        const float d = dv * dv;
        if (d < best) {
          best = d;
          bc = j;
        }
      }
      asg[i] = (uint8_t)bc;
    }
    __syncthreads();
    if (lane < k) {
      float acc = 0.0f;
      uint32_t cnt = 0;
      for (uint32_t i = 0; i < n; i++) {
        const bool mine = asg[i] == lane;
        acc += mine ? val[i] : 0.0f;
        cnt += mine ? 1u : 0u;
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
  if (lane < (uint32_t)kPaletteMaxK) lut[lane] = f2h(lane < k ? cent[lane] : 0.0f);
  const uint32_t rb = (n + 1) / 2;
  for (uint32_t b = lane; b < rb; b += 64) {
    uint32_t byte = 0;
    for (uint32_t h = 0; h < 2; h++) {
      const uint32_t i = 2 * b + h;
      if (i >= n) break;
      float best = FMAX;
      uint32_t bi = 0;
      for (uint32_t j = 0; j < k; j++) {
        const float dv = val[i] - cent[j];
        const float d = dv * dv;
        if (d < best) {
          best = d;
          bi = j;
        }
      }
      byte |= bi << (4 * h);
    }
    idx_out[(size_t)r * rb + b] = (uint8_t)byte;
  }
}

}  // namespace prism
