/*
 * prism_cpuref_palette.c -- CPU oracle for the palette compiler (per-row
 * k-means palettization that produces the split-block weights).
 *
 * TEST INFRASTRUCTURE ONLY, like prism_cpuref.c.
 *
 * Reference behaviour restated here (Tribunus-dev/prism-engine):
 *   cpuref_fit_palette        fit_palette, src/quantization/palette.rs:75-183
 *                             (k-means++ init from channel[n/2] with the
 *                             golden-ratio threshold of :186-191, Lloyd
 *                             iterations with a 0.001 shift exit, centroids
 *                             sorted by magnitude, descending, stably).
 *                             With seeds: compute-core's fit_palette
 *                             (compute-core/src/quantization/palette.rs:
 *                             94-201): the first min(len, k) centroids are
 *                             the seeds and k-means++ continues from them
 *                             (its first distance pass sees only the last
 *                             seed, as there); the rest is unchanged (its
 *                             transposed assignment loop picks the same
 *                             first strictly nearest centroid).
 *   cpuref_encode_channel     encode_channel, palette.rs:198-228
 *   cpuref_palettize_payload  palettize_matrix (palette.rs:230-272) followed
 *                             by compile_to_cimage's payload assembly
 *                             (src/lut/compiler.rs:47-60): per row 16 fp16
 *                             entries (zero past k), then every row's packed
 *                             indices, (n+1)/2 bytes per row.
 * Arithmetic: fp32, sequential folds in element order, no contraction.
 */
#include <math.h>
#include <stddef.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

uint16_t cpuref_f32_to_f16(float f);

/* weighted_threshold: total * frac(seed * 0.6180339887498949) (f64 frac). */
static float weighted_threshold(float total, size_t seed) {
  double x = (double)seed * 0.6180339887498949;
  double frac = x - trunc(x);
  return total * (float)frac;
}

/* Returns the number of centroids written to out (min(k, n); 0 for n == 0).
 * seeds may be NULL (root crate fit_palette); otherwise nseeds >= 1. */
size_t cpuref_fit_palette_seeded(const float* ch, size_t n, size_t k, size_t max_iter, const float* seeds,
                                 size_t nseeds, float* out) {
  if (n == 0 || k == 0) return 0;
  if (seeds && nseeds == 0) return 0; /* the reference panics (centroids[-1]); callers reject it */
  if (k > n) k = n;
  float* c = out;
  size_t nc = 0;
  if (seeds) {
    for (size_t j = 0; j < nseeds && j < k; j++) c[nc++] = seeds[j];
  } else {
    c[nc++] = ch[n / 2];
  }
  float* min_d = (float*)malloc(sizeof(float) * n);
  size_t* asg = (size_t*)malloc(sizeof(size_t) * n);
  for (size_t i = 0; i < n; i++) min_d[i] = 3.40282347e38f; /* f32::MAX */
  while (nc < k) {
    const float last = c[nc - 1];
    float total = 0.0f;
    for (size_t i = 0; i < n; i++) {
      const float dv = ch[i] - last;
      const float d = dv * dv;
      if (d < min_d[i]) min_d[i] = d;
      total += min_d[i];
    }
    if (total <= 0.0f) {
      c[nc] = ch[(nc * n / k) % n];
      nc++;
      continue;
    }
    const float target = weighted_threshold(total, nc);
    float cum = 0.0f;
    size_t picked = 0;
    for (size_t i = 0; i < n; i++) {
      cum += min_d[i];
      if (cum >= target) {
        picked = i;
        break;
      }
    }
    c[nc++] = ch[picked];
  }
  float sums[256];
  uint64_t counts[256];
  for (size_t it = 0; it < max_iter; it++) {
    for (size_t i = 0; i < n; i++) {
      float best = 3.40282347e38f;
      size_t bc = 0;
      for (size_t j = 0; j < k; j++) {
        const float dv = ch[i] - c[j];
        const float d = dv * dv;
        if (d < best) {
          best = d;
          bc = j;
        }
      }
      asg[i] = bc;
    }
    for (size_t j = 0; j < k; j++) {
      sums[j] = 0.0f;
      counts[j] = 0;
    }
    for (size_t i = 0; i < n; i++) {
      sums[asg[i]] += ch[i];
      counts[asg[i]] += 1;
    }
    float max_shift = 0.0f;
    for (size_t j = 0; j < k; j++) {
      if (counts[j] > 0) {
        const float nv = sums[j] / (float)counts[j];
        const float sh = fabsf(c[j] - nv);
        if (sh > max_shift) max_shift = sh;
        c[j] = nv;
      }
    }
    if (max_shift < 0.001f) break;
  }
  /* stable sort by |c| descending (insertion sort keeps equal keys in order) */
  for (size_t a = 1; a < k; a++) {
    const float v = c[a];
    size_t b = a;
    while (b > 0 && fabsf(c[b - 1]) < fabsf(v)) {
      c[b] = c[b - 1];
      b--;
    }
    c[b] = v;
  }
  free(min_d);
  free(asg);
  return k;
}

size_t cpuref_fit_palette(const float* ch, size_t n, size_t k, size_t max_iter, float* out) {
  return cpuref_fit_palette_seeded(ch, n, k, max_iter, NULL, 0, out);
}

/* Packs (n+1)/2 bytes into packed (element 2i low nibble); returns the MSE. */
float cpuref_encode_channel(const float* ch, size_t n, const float* cb, size_t kc, uint8_t* packed) {
  float mse = 0.0f;
  if (kc > 16) kc = 16;
  memset(packed, 0, (n + 1) / 2);
  for (size_t i = 0; i < n; i++) {
    uint8_t bi = 0;
    float best = 3.40282347e38f;
    for (size_t j = 0; j < kc; j++) {
      const float dv = ch[i] - cb[j];
      const float d = dv * dv;
      if (d < best) {
        best = d;
        bi = (uint8_t)j;
      }
    }
    mse += best;
    if ((i & 1) == 0)
      packed[i / 2] = bi;
    else
      packed[i / 2] |= (uint8_t)(bi << 4);
  }
  return n ? mse / (float)n : 0.0f;
}

/* The compiler's split-block payload for a [out_dim x in_dim] f32 matrix:
 * out_dim*32 LUT bytes then out_dim*((in_dim+1)/2) index bytes.  mse (may be
 * NULL) receives each row's encode MSE. */
int cpuref_palettize_payload_seeded(const float* w, size_t out_dim, size_t in_dim, size_t k, size_t max_iter,
                                    const float* seeds, size_t nseeds, uint8_t* payload, float* mse) {
  if (k == 0 || k > 16) return -1;
  if (seeds && nseeds == 0) return -1; /* the reference indexes centroids[-1] */
  const size_t rb = (in_dim + 1) / 2;
  uint8_t* idx = payload + out_dim * 32;
  for (size_t r = 0; r < out_dim; r++) {
    float cb[16] = {0};
    const size_t kc = cpuref_fit_palette_seeded(w + r * in_dim, in_dim, k, max_iter, seeds, nseeds, cb);
    const float e = cpuref_encode_channel(w + r * in_dim, in_dim, cb, kc, idx + r * rb);
    if (mse) mse[r] = e;
    for (size_t j = 0; j < 16; j++) {
      const uint16_t h = cpuref_f32_to_f16(j < kc ? cb[j] : 0.0f);
      payload[r * 32 + 2 * j] = (uint8_t)(h & 0xFF);
      payload[r * 32 + 2 * j + 1] = (uint8_t)(h >> 8);
    }
  }
  return 0;
}

int cpuref_palettize_payload(const float* w, size_t out_dim, size_t in_dim, size_t k, size_t max_iter,
                             uint8_t* payload, float* mse) {
  return cpuref_palettize_payload_seeded(w, out_dim, in_dim, k, max_iter, NULL, 0, payload, mse);
}
