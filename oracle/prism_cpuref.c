/*
 * prism_cpuref.c -- CPU oracle for the palettized-LUT weight contraction.
 *
 * TEST INFRASTRUCTURE ONLY.  This file restates the reference's CPU path so
 * that tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg can
 * check the HIP library against it.  Nothing in the product links, loads or
 * calls it; the product has no CPU fallback.
 *
 * Reference behaviour restated here (Tribunus-dev/prism-engine):
 *   cpuref_lut_gemv4     compute-core/src/lut/evaluator.rs:21-44 (lut_gemv_cpu)
 *                        twins: compute-core/src/lut/engine.rs:623-644,
 *                               src/lut/cpu_fallback.rs:12-35
 *   cpuref_silu_inplace  compute-core/src/lut/evaluator.rs:78-83
 *   cpuref_swiglu        compute-core/src/lut/evaluator.rs:209-225
 *                        (evaluate_activations(Silu, gate, Some(up)))
 *   cpuref_gateup_swiglu the engine's unfused CPU sequence for an MLP:
 *                        src/lut/engine_impl.rs:1120-1127 (two gemv calls)
 *                        then :1349-1374 (silu + gate*up)
 *   cpuref_lut_embed     compute-core/src/lut/evaluator.rs:176-197
 *   f16 <-> f32          the `half` crate v2.7.1 (Cargo.lock:1600-1602):
 *                        f16->f32 is exact; f32->f16 is IEEE-754
 *                        round-to-nearest-even with overflow to inf.
 *
 * Build extensions (the reference has no implementation of these; each is
 * the direct generalisation of lut_gemv_cpu, declared as such):
 *   cpuref_lut_gemv8     byte indices, 256-entry per-row LUT.  Format from
 *                        compute-core/tests/palettized_vs_direct.rs:108-135
 *                        (per-row 256-entry LUT, 1-byte indices row-major),
 *                        laid out split-block like the 4-bit payload.
 *   cpuref_gemv_batch    B independent GEMVs (B rows of x).
 *   cpuref_gemm          M independent GEMV rows (the reference's GEMM
 *                        template, templates/palettized_gemm.metal, is never
 *                        dispatched and accumulates in half; the CPU
 *                        semantics are M calls of lut_gemv_cpu).
 *
 * Arithmetic: a sequential fp32 left fold in element order, no contraction
 * (build with -ffp-contract=off).  Every product of two fp16 values is exact
 * in fp32, so contraction could not change the result anyway.
 */
#include <math.h>
#include <stddef.h>
#include <stdint.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ---- binary16 <-> binary32 (half crate semantics) ---------------------- */

float cpuref_f16_to_f32(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 0x1Fu;
  uint32_t man = h & 0x3FFu;
  uint32_t bits;
  if (exp == 0) {
    if (man == 0) {
      bits = sign;
    } else { /* subnormal: normalise */
      int e = -1;
      do {
        man <<= 1;
        e++;
      } while ((man & 0x400u) == 0);
      man &= 0x3FFu;
      bits = sign | ((uint32_t)(127 - 15 - e) << 23) | (man << 13);
    }
  } else if (exp == 0x1F) {
    bits = sign | 0x7F800000u | (man << 13) | (man ? 0x00400000u : 0u);
  } else {
    bits = sign | ((exp + 127 - 15) << 23) | (man << 13);
  }
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

uint16_t cpuref_f32_to_f16(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  uint32_t sign = (x >> 16) & 0x8000u;
  uint32_t exp = (x >> 23) & 0xFFu;
  uint32_t man = x & 0x7FFFFFu;
  if (exp == 0xFF) { /* inf / nan (nan keeps quiet bit + top payload) */
    if (man == 0) return (uint16_t)(sign | 0x7C00u);
    return (uint16_t)(sign | 0x7E00u | (man >> 13));
  }
  int e = (int)exp - 127 + 15;
  if (e >= 0x1F) return (uint16_t)(sign | 0x7C00u); /* overflow -> inf */
  if (e <= 0) {                                       /* subnormal or zero */
    if (e < -10) return (uint16_t)sign;               /* below half of min subnormal */
    uint32_t m = man | 0x800000u;                     /* implicit bit */
    int shift = 14 - e;                               /* 14..24 */
    uint32_t half_m = m >> shift;
    uint32_t rem = m & ((1u << shift) - 1u);
    uint32_t halfway = 1u << (shift - 1);
    if (rem > halfway || (rem == halfway && (half_m & 1u))) half_m++;
    return (uint16_t)(sign | half_m);
  }
  uint32_t half_m = man >> 13;
  uint32_t rem = man & 0x1FFFu;
  uint32_t out = sign | ((uint32_t)e << 10) | half_m;
  if (rem > 0x1000u || (rem == 0x1000u && (half_m & 1u))) out++; /* may carry into exp: correct */
  return (uint16_t)out;
}

/* ---- summation order (test support) -------------------------------------
 * Mode 0 (the default) is the reference's sequential left fold, which every
 * function in this file restates.  Mode 1 is an order-perturbed variant used
 * only by tests/test_step_order.py to measure how far an equally valid fp32
 * summation order moves the decode step's outputs: each long sum (the GEMV
 * rows, the RMS norm's sum of squares, the softmax denominator and the
 * attention's value sums) is cut into blocks of 64 consecutive terms, each
 * block folded sequentially, and the block sums added as a binary tree --
 * the shape of a GPU reduction.  It is not a restatement of anything. */
int cpuref_fold_mode = 0;
void cpuref_set_fold_mode(int mode) { cpuref_fold_mode = mode; }

/* Set when a blocked sum had more than 2048 blocks (131072 terms): mode 1
 * then refuses to give a result rather than drop terms; the caller reads
 * and clears it (cpuref_fold_overflowed). */
static volatile int cpuref_fold_overflow = 0;
int cpuref_fold_overflowed(void) {
  const int v = cpuref_fold_overflow;
  cpuref_fold_overflow = 0;
  return v;
}

/* Blocked accumulator for mode 1: add terms in order, close a block every
 * 64 terms, and finish with a pairwise tree over the block sums. */
typedef struct {
  float part[2048];
  size_t nparts, cnt;
  float acc;
} cpuref_blocked;
void cpuref_blocked_init(cpuref_blocked* b) {
  b->nparts = 0;
  b->cnt = 0;
  b->acc = 0.0f;
}
void cpuref_blocked_add(cpuref_blocked* b, float v) {
  b->acc += v;
  if (++b->cnt == 64) {
    if (b->nparts < 2048)
      b->part[b->nparts++] = b->acc;
    else
      cpuref_fold_overflow = 1;
    b->acc = 0.0f;
    b->cnt = 0;
  }
}
float cpuref_blocked_sum(cpuref_blocked* b) {
  if (b->cnt) {
    if (b->nparts < 2048)
      b->part[b->nparts++] = b->acc;
    else
      cpuref_fold_overflow = 1;
  }
  size_t n = b->nparts;
  if (n == 0) return 0.0f;
  while (n > 1) {
    const size_t h = n / 2;
    for (size_t i = 0; i < h; i++) b->part[i] = b->part[2 * i] + b->part[2 * i + 1];
    if (n & 1) b->part[h] = b->part[n - 1];
    n = h + (n & 1);
  }
  return b->part[0];
}

/* ---- palettized GEMV ---------------------------------------------------- */

static inline uint16_t rd16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }
static inline uint32_t rd32(const uint8_t* p) {
  return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}

/* One row of lut_gemv_cpu (evaluator.rs:26-42). */
static uint16_t gemv4_row(const uint16_t* inp, const uint8_t* p, uint32_t dm, uint32_t dn, uint32_t r) {
  const size_t cbb = (size_t)dm * 16 * 2;
  float cb[16];
  for (int i = 0; i < 16; i++) cb[i] = cpuref_f16_to_f32(rd16(p + (size_t)r * 32 + (size_t)i * 2));
  const size_t io = cbb + (size_t)r * (dn / 2);
  if (cpuref_fold_mode == 1) {
    cpuref_blocked b;
    cpuref_blocked_init(&b);
    for (uint32_t wi = 0; wi < dn / 8; wi++) {
      uint32_t pw = rd32(p + io + (size_t)wi * 4);
      for (uint32_t j = 0; j < 8; j++) cpuref_blocked_add(&b, cpuref_f16_to_f32(inp[wi * 8 + j]) * cb[(pw >> (j * 4)) & 0x0Fu]);
    }
    return cpuref_f32_to_f16(cpuref_blocked_sum(&b));
  }
  float acc = 0.0f;
  for (uint32_t wi = 0; wi < dn / 8; wi++) {
    uint32_t pw = rd32(p + io + (size_t)wi * 4);
    for (uint32_t j = 0; j < 8; j++) {
      acc += cpuref_f16_to_f32(inp[wi * 8 + j]) * cb[(pw >> (j * 4)) & 0x0Fu];
    }
  }
  return cpuref_f32_to_f16(acc);
}

/* lut_gemv_cpu: o[r] = f16(sum_k f32(x[k]) * f32(LUT_r[nib(r,k)])).
 * Elements beyond the last whole 8-element word are dropped, as in the
 * reference (evaluator.rs:33 iterates dn/8 words). */
void cpuref_lut_gemv4(const uint16_t* inp, const uint8_t* p, uint32_t dm, uint32_t dn, uint16_t* out) {
  for (uint32_t r = 0; r < dm; r++) out[r] = gemv4_row(inp, p, dm, dn, r);
}

/* Row-parallel variant (informational CPU baseline): same per-row order,
 * so bit-identical to cpuref_lut_gemv4. */
void cpuref_lut_gemv4_mt(const uint16_t* inp, const uint8_t* p, uint32_t dm, uint32_t dn, uint16_t* out,
                         int nthreads) {
#ifdef _OPENMP
#pragma omp parallel for schedule(static) num_threads(nthreads)
#endif
  for (long r = 0; r < (long)dm; r++) out[r] = gemv4_row(inp, p, dm, dn, (uint32_t)r);
  (void)nthreads;
}

/* 8-bit extension: payload = [dm x 256 fp16 LUT][dm x dn index bytes]. */
static uint16_t gemv8_row(const uint16_t* inp, const uint8_t* p, uint32_t dm, uint32_t dn, uint32_t r) {
  const size_t cbb = (size_t)dm * 256 * 2;
  const uint8_t* lut = p + (size_t)r * 512;
  const uint8_t* idx = p + cbb + (size_t)r * dn;
  if (cpuref_fold_mode == 1) {
    cpuref_blocked b;
    cpuref_blocked_init(&b);
    for (uint32_t k = 0; k < dn; k++)
      cpuref_blocked_add(&b, cpuref_f16_to_f32(inp[k]) * cpuref_f16_to_f32(rd16(lut + (size_t)idx[k] * 2)));
    return cpuref_f32_to_f16(cpuref_blocked_sum(&b));
  }
  float acc = 0.0f;
  for (uint32_t k = 0; k < dn; k++) {
    acc += cpuref_f16_to_f32(inp[k]) * cpuref_f16_to_f32(rd16(lut + (size_t)idx[k] * 2));
  }
  return cpuref_f32_to_f16(acc);
}

void cpuref_lut_gemv8(const uint16_t* inp, const uint8_t* p, uint32_t dm, uint32_t dn, uint16_t* out) {
  for (uint32_t r = 0; r < dm; r++) out[r] = gemv8_row(inp, p, dm, dn, r);
}

void cpuref_lut_gemv8_mt(const uint16_t* inp, const uint8_t* p, uint32_t dm, uint32_t dn, uint16_t* out,
                         int nthreads) {
#ifdef _OPENMP
#pragma omp parallel for schedule(static) num_threads(nthreads)
#endif
  for (long r = 0; r < (long)dm; r++) out[r] = gemv8_row(inp, p, dm, dn, (uint32_t)r);
  (void)nthreads;
}

/* B independent GEMVs: x is [B x dn], y is [B x dm]. bits in {4, 8}. */
int cpuref_gemv_batch(const uint16_t* x, uint32_t batch, const uint8_t* p, uint32_t dm, uint32_t dn,
                      uint32_t bits, uint16_t* y) {
  for (uint32_t b = 0; b < batch; b++) {
    if (bits == 4)
      cpuref_lut_gemv4(x + (size_t)b * dn, p, dm, dn, y + (size_t)b * dm);
    else if (bits == 8)
      cpuref_lut_gemv8(x + (size_t)b * dn, p, dm, dn, y + (size_t)b * dm);
    else
      return -1;
  }
  return 0;
}

/* GEMM: Y[M x dm] = X[M x dn] . W^T, as M independent GEMV rows. Row-parallel
 * across M when threads > 1 (bit-identical). */
int cpuref_gemm(const uint16_t* X, uint32_t M, const uint8_t* p, uint32_t dm, uint32_t dn, uint32_t bits,
                uint16_t* Y, int nthreads) {
  if (bits != 4 && bits != 8) return -1;
#ifdef _OPENMP
#pragma omp parallel for schedule(dynamic, 1) num_threads(nthreads)
#endif
  for (long m = 0; m < (long)M; m++) {
    for (uint32_t r = 0; r < dm; r++) {
      Y[(size_t)m * dm + r] = bits == 4 ? gemv4_row(X + (size_t)m * dn, p, dm, dn, r)
                                        : gemv8_row(X + (size_t)m * dn, p, dm, dn, r);
    }
  }
  (void)nthreads;
  return 0;
}

/* ---- activations -------------------------------------------------------- */

/* silu_inplace (evaluator.rs:78-83): f16(f / (1 + exp(-f))) in f32. */
void cpuref_silu_inplace(uint16_t* x, size_t n) {
  for (size_t i = 0; i < n; i++) {
    float f = cpuref_f16_to_f32(x[i]);
    x[i] = cpuref_f32_to_f16(f / (1.0f + expf(-f)));
  }
}

/* evaluate_activations(Silu, gate, Some(up)) (evaluator.rs:209-225):
 * gate <- silu(gate); gate[i] <- f16(f32(gate[i]) * f32(up[i])). */
void cpuref_swiglu(uint16_t* gate, const uint16_t* up, size_t n) {
  cpuref_silu_inplace(gate, n);
  for (size_t i = 0; i < n; i++) {
    float a = cpuref_f16_to_f32(gate[i]);
    float b = cpuref_f16_to_f32(up[i]);
    gate[i] = cpuref_f32_to_f16(a * b);
  }
}

/* The MLP's CPU sequence: gate = gemv(x, Wg); up = gemv(x, Wu);
 * y = swiglu(gate, up).  y must hold dm values; scratch `up_tmp` dm values. */
int cpuref_gateup_swiglu(const uint16_t* x, const uint8_t* pg, const uint8_t* pu, uint32_t dm, uint32_t dn,
                         uint32_t bits, uint16_t* y, uint16_t* up_tmp, int nthreads) {
  if (bits == 4) {
    cpuref_lut_gemv4_mt(x, pg, dm, dn, y, nthreads);
    cpuref_lut_gemv4_mt(x, pu, dm, dn, up_tmp, nthreads);
  } else if (bits == 8) {
    cpuref_lut_gemv8_mt(x, pg, dm, dn, y, nthreads);
    cpuref_lut_gemv8_mt(x, pu, dm, dn, up_tmp, nthreads);
  } else {
    return -1;
  }
  cpuref_swiglu(y, up_tmp, dm);
  return 0;
}

/* ---- LUT decode --------------------------------------------------------- */

/* lut_embed (evaluator.rs:176-197): the fp16 bits of one decoded row;
 * an out-of-range token gives zeros. out holds hidden_dim values. */
void cpuref_lut_embed(uint32_t token, const uint8_t* payload, uint32_t vocab_size, uint32_t hidden_dim,
                      uint16_t* out) {
  if (token >= vocab_size) {
    memset(out, 0, (size_t)hidden_dim * 2);
    return;
  }
  const size_t cb = (size_t)vocab_size * 16 * 2;
  const size_t io = cb + (size_t)token * (hidden_dim / 2);
  uint32_t n = 0;
  for (uint32_t wi = 0; wi < hidden_dim / 8; wi++) {
    uint32_t pw = rd32(payload + io + (size_t)wi * 4);
    for (uint32_t j = 0; j < 8; j++) out[n++] = rd16(payload + (size_t)token * 32 + ((pw >> (j * 4)) & 0xFu) * 2);
  }
  for (; n < hidden_dim; n++) out[n] = 0; /* the reference returns a shorter vector */
}

/* Dense decode of rows [r0, r0+nrows) for either bit width (the per-row
 * form of lut_embed, used to check a decoder bit for bit). */
int cpuref_decode_rows(const uint8_t* p, uint32_t dm, uint32_t dn, uint32_t bits, uint32_t r0, uint32_t nrows,
                       uint16_t* out) {
  if (bits != 4 && bits != 8) return -1;
  for (uint32_t i = 0; i < nrows; i++) {
    uint32_t r = r0 + i;
    uint16_t* o = out + (size_t)i * dn;
    if (bits == 4) {
      /* lut_embed's word loop: only (dn/8)*8 elements decode; the rest of
       * the dense row is zero. */
      const size_t io = (size_t)dm * 32 + (size_t)r * (dn / 2);
      const uint32_t keff = (dn / 8) * 8;
      for (uint32_t k = 0; k < dn; k++) {
        if (k >= keff) {
          o[k] = 0;
          continue;
        }
        uint8_t b = p[io + k / 2];
        uint32_t nib = (k & 1) ? (b >> 4) : (b & 0xFu);
        o[k] = rd16(p + (size_t)r * 32 + nib * 2);
      }
    } else {
      const size_t io = (size_t)dm * 512 + (size_t)r * dn;
      for (uint32_t k = 0; k < dn; k++) o[k] = rd16(p + (size_t)r * 512 + (size_t)p[io + k] * 2);
    }
  }
  return 0;
}
