/*
 * prism_cpuref_step.c -- CPU oracle for one decode step of a palettized
 * transformer (the Qwen2 graph of the reference engine).
 *
 * TEST INFRASTRUCTURE ONLY, like prism_cpuref.c: tests/, smoke() and
 * bench.py's cpu_baseline leg use it to check the HIP decode step.
 *
 * Reference behaviour restated here (Tribunus-dev/prism-engine):
 *   cpuref_rms_norm_inplace  compute-core/src/lut/evaluator.rs:49-64
 *                            (no gamma: the engine's CPU norm ignores the
 *                            norm weight, src/lut/engine_impl.rs:1056-1065)
 *   cpuref_vec_add_inplace   evaluator.rs:67-73
 *   cpuref_rope_inplace      evaluator.rs:154-166 (base 10000 whatever the
 *                            configured theta; engine_impl.rs:1068-1075)
 *   cpuref_kv_quant          KVCache::append's q() (engine_impl.rs:532-556)
 *                            and the VProj branch (:1134-1157)
 *   cpuref_kv_dequant        dequant_inline (engine_impl.rs:569-584)
 *   cpuref_attention         attention_cpu (evaluator.rs:104-146)
 *   cpuref_decode_step       PrismEngine::step (engine_impl.rs:1076-1405)
 *                            over the node order ModelGraph::build gives a
 *                            Qwen2 config (src/lut/graph.rs:304-530):
 *                            embed; per layer Norm, Q, K, V, RoPE(Q only),
 *                            SDPA, O (+ residual), Norm, gate, up, SiLU*up,
 *                            down (+ residual); final Norm; tied LM head
 *                            (the embedding matrix, :1384-1403).
 * Transcendentals are the C library's expf / sinf / cosf / powf, the same
 * functions the reference's f32 methods call on Linux.
 */
#include <math.h>
#include <stddef.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

float cpuref_f16_to_f32(uint16_t h);
uint16_t cpuref_f32_to_f16(float f);
void cpuref_lut_gemv4_mt(const uint16_t* inp, const uint8_t* p, uint32_t dm, uint32_t dn, uint16_t* out,
                         int nthreads);
void cpuref_lut_gemv8_mt(const uint16_t* inp, const uint8_t* p, uint32_t dm, uint32_t dn, uint16_t* out,
                         int nthreads);
void cpuref_silu_inplace(uint16_t* x, size_t n);
void cpuref_swiglu(uint16_t* gate, const uint16_t* up, size_t n);
void cpuref_lut_embed(uint32_t token, const uint8_t* payload, uint32_t vocab_size, uint32_t hidden_dim,
                      uint16_t* out);

#define F(h) cpuref_f16_to_f32(h)
#define H(f) cpuref_f32_to_f16(f)

/* Summation order switch and blocked accumulator (prism_cpuref.c). */
extern int cpuref_fold_mode;
typedef struct {
  float part[2048];
  size_t nparts, cnt;
  float acc;
} cpuref_blocked;
void cpuref_blocked_init(cpuref_blocked* b);
void cpuref_blocked_add(cpuref_blocked* b, float v);
float cpuref_blocked_sum(cpuref_blocked* b);

/* rms_norm_inplace: inv = 1 / sqrt(sum(f*f) / n + eps), sequential fp32
 * sum; x <- f16(x * inv). */
void cpuref_rms_norm_inplace(uint16_t* x, size_t n, float eps) {
  float sum = 0.0f;
  if (cpuref_fold_mode == 1) {
    cpuref_blocked b;
    cpuref_blocked_init(&b);
    for (size_t i = 0; i < n; i++) cpuref_blocked_add(&b, F(x[i]) * F(x[i]));
    sum = cpuref_blocked_sum(&b);
  } else {
    for (size_t i = 0; i < n; i++) {
      float f = F(x[i]);
      sum += f * f;
    }
  }
  float inv = 1.0f / sqrtf(sum / (float)n + eps);
  for (size_t i = 0; i < n; i++) x[i] = H(F(x[i]) * inv);
}

/* vec_add_inplace: a <- f16(a + b). */
void cpuref_vec_add_inplace(uint16_t* a, const uint16_t* b, size_t n) {
  for (size_t i = 0; i < n; i++) a[i] = H(F(a[i]) + F(b[i]));
}

/* The rotation angle of pair j at position pos: pos * 10000^(-2j/hd). */
float cpuref_rope_angle(int64_t pos, size_t j, size_t hd) {
  return (float)pos * powf(10000.0f, (-2.0f * (float)j) / (float)hd);
}

/* rope_inplace: every hd-wide head, pairs (j, j + hd/2). */
void cpuref_rope_inplace(uint16_t* x, size_t n, int64_t pos, size_t hd) {
  const size_t h = hd / 2;
  for (size_t i = 0; i < n; i += hd) {
    for (size_t j = 0; j < h; j++) {
      float a = F(x[i + j]);
      float b = F(x[i + j + h]);
      float ang = cpuref_rope_angle(pos, j, hd);
      float sa = sinf(ang), ca = cosf(ang);
      x[i + j] = H(a * ca - b * sa);
      x[i + j + h] = H(a * sa + b * ca);
    }
  }
}

/* One token block of the INT8 KV cache: [scale f32 LE][n x i8].  Returns
 * the bytes written (0 for an empty slice, which writes nothing). */
size_t cpuref_kv_quant(const uint16_t* data, size_t n, uint8_t* out) {
  if (n == 0) return 0;
  float max_abs = 0.0f;
  for (size_t i = 0; i < n; i++) max_abs = fmaxf(max_abs, fabsf(F(data[i])));
  float scale = max_abs > 1e-10f ? 127.0f / max_abs : 1.0f;
  memcpy(out, &scale, 4); /* little-endian host */
  for (size_t i = 0; i < n; i++) {
    float q = roundf(F(data[i]) * scale); /* half away from zero, like f32::round */
    if (q < -128.0f) q = -128.0f;
    if (q > 127.0f) q = 127.0f;
    out[4 + i] = (uint8_t)(int8_t)q;
  }
  return 4 + n;
}

/* dequant_inline over ntok blocks of kv_dim values: f16(i8 * (1 / s)). */
void cpuref_kv_dequant(const uint8_t* data, size_t ntok, size_t kv_dim, uint16_t* out) {
  const size_t ts = kv_dim + 4;
  for (size_t t = 0; t < ntok; t++) {
    float s;
    memcpy(&s, data + t * ts, 4);
    const float rs = 1.0f / s;
    for (size_t j = 0; j < kv_dim; j++) out[t * kv_dim + j] = H((float)(int8_t)data[t * ts + 4 + j] * rs);
  }
}

/* attention_cpu: grouped-query softmax(q k^T / sqrt(hd)) v per head.
 * kc, vc: [sl x nkv x hd] fp16; out [nh x hd]. */
void cpuref_attention(const uint16_t* q, const uint16_t* kc, const uint16_t* vc, size_t nh, size_t nkv, size_t hd,
                      size_t sl, uint16_t* out) {
  const size_t g = nh / (nkv ? nkv : 1);
  const size_t kvd = nkv * hd;
  float* sc = (float*)malloc(sizeof(float) * (sl ? sl : 1));
  float* ex = (float*)malloc(sizeof(float) * (sl ? sl : 1));
  const float den = sqrtf((float)hd);
  for (size_t h = 0; h < nh; h++) {
    const size_t kh = h / g, qb = h * hd;
    for (size_t p = 0; p < sl; p++) {
      const size_t kb = p * kvd + kh * hd;
      float s = 0.0f;
      for (size_t d = 0; d < hd; d++) s += F(q[qb + d]) * F(kc[kb + d]);
      sc[p] = s / den;
    }
    float mx = -INFINITY;
    for (size_t p = 0; p < sl; p++) mx = fmaxf(mx, sc[p]);
    float es = 0.0f;
    for (size_t p = 0; p < sl; p++) ex[p] = expf(sc[p] - mx);
    if (cpuref_fold_mode == 1) {
      cpuref_blocked b;
      cpuref_blocked_init(&b);
      for (size_t p = 0; p < sl; p++) cpuref_blocked_add(&b, ex[p]);
      es = cpuref_blocked_sum(&b);
    } else {
      for (size_t p = 0; p < sl; p++) es += ex[p];
    }
    const float inv = 1.0f / (es + 1e-10f);
    for (size_t d = 0; d < hd; d++) {
      float ac = 0.0f;
      if (cpuref_fold_mode == 1) {
        cpuref_blocked b;
        cpuref_blocked_init(&b);
        for (size_t p = 0; p < sl; p++) cpuref_blocked_add(&b, ex[p] * F(vc[p * kvd + kh * hd + d]) * inv);
        ac = cpuref_blocked_sum(&b);
      } else {
        for (size_t p = 0; p < sl; p++) ac += ex[p] * F(vc[p * kvd + kh * hd + d]) * inv;
      }
      out[qb + d] = H(ac);
    }
  }
  free(sc);
  free(ex);
}

/* ---- the decode step ----------------------------------------------------- */

/* dims: n_layers, hidden, n_heads, n_kv_heads, head_dim, intermediate,
 *       vocab, bits (4 or 8).
 * w:    n_layers * 7 split-block payloads in the order q, k, v, o, gate,
 *       up, down; embed: the [vocab x hidden] embedding, also the tied LM
 *       head (always 4-bit: lut_embed decodes nibbles).
 * kv:   per layer k[l], v[l]: byte buffers holding kv_len[l] token blocks
 *       of (4 + kv_dim) bytes each, with room for one more; kv_len[l] is
 *       advanced by one (KVCache::append + the VProj branch).
 * logits: vocab fp16 values. */
static void gemv(const uint16_t* x, const uint8_t* p, uint32_t dm, uint32_t dn, uint32_t bits, uint16_t* y,
                 int nthreads) {
  if (bits == 8)
    cpuref_lut_gemv8_mt(x, p, dm, dn, y, nthreads);
  else
    cpuref_lut_gemv4_mt(x, p, dm, dn, y, nthreads);
}

int cpuref_decode_step(const uint32_t* dims, float eps, const uint8_t* embed, const uint8_t* const* w,
                       uint8_t* const* kbuf, uint8_t* const* vbuf, size_t* kv_len, uint32_t token, int64_t pos,
                       uint16_t* logits, int nthreads) {
  const uint32_t L = dims[0], D = dims[1], NH = dims[2], NKV = dims[3], HD = dims[4], I = dims[5], V = dims[6],
                 bits = dims[7];
  if (bits != 4 && bits != 8) return -1;
  const uint32_t QD = NH * HD, KVD = NKV * HD;
  const size_t mx = (D > QD ? D : QD) > I ? (D > QD ? D : QD) : I;
  uint16_t* h = (uint16_t*)malloc(2 * mx);
  uint16_t* hr = (uint16_t*)malloc(2 * mx);
  uint16_t* q = (uint16_t*)malloc(2 * QD);
  uint16_t* kv = (uint16_t*)malloc(2 * KVD);
  uint16_t* gate = (uint16_t*)malloc(2 * I);
  uint16_t* up = (uint16_t*)malloc(2 * I);
  uint16_t* o = (uint16_t*)malloc(2 * D);
  if (!h || !hr || !q || !kv || !gate || !up || !o) return -2;

  cpuref_lut_embed(token, embed, V, D, h);
  memcpy(hr, h, 2 * D);
  for (uint32_t l = 0; l < L; l++) {
    const uint8_t* const* lw = w + (size_t)l * 7;
    cpuref_rms_norm_inplace(h, D, eps);
    gemv(h, lw[0], QD, D, bits, q, nthreads);
    gemv(h, lw[1], KVD, D, bits, kv, nthreads);
    const size_t ts = 4 + KVD;
    cpuref_kv_quant(kv, KVD, kbuf[l] + kv_len[l] * ts);
    gemv(h, lw[2], KVD, D, bits, kv, nthreads);
    cpuref_kv_quant(kv, KVD, vbuf[l] + kv_len[l] * ts);
    kv_len[l] += 1;
    cpuref_rope_inplace(q, QD, pos, HD); /* Q only */
    const size_t sl = kv_len[l];
    uint16_t* kc = (uint16_t*)malloc(2 * sl * KVD);
    uint16_t* vc = (uint16_t*)malloc(2 * sl * KVD);
    if (!kc || !vc) return -2;
    cpuref_kv_dequant(kbuf[l], sl, KVD, kc);
    cpuref_kv_dequant(vbuf[l], sl, KVD, vc);
    cpuref_attention(q, kc, vc, NH, NKV, HD, sl, h);
    free(kc);
    free(vc);
    gemv(h, lw[3], D, QD, bits, o, nthreads); /* o_proj */
    memcpy(h, o, 2 * D);
    cpuref_vec_add_inplace(h, hr, D);
    memcpy(hr, h, 2 * D);
    cpuref_rms_norm_inplace(h, D, eps);
    gemv(h, lw[4], I, D, bits, gate, nthreads);
    gemv(h, lw[5], I, D, bits, up, nthreads);
    cpuref_swiglu(gate, up, I);
    gemv(gate, lw[6], D, I, bits, h, nthreads);
    cpuref_vec_add_inplace(h, hr, D);
    memcpy(hr, h, 2 * D);
  }
  cpuref_rms_norm_inplace(h, D, eps);
  cpuref_lut_gemv4_mt(h, embed, V, D, logits, nthreads);
  free(h);
  free(hr);
  free(q);
  free(kv);
  free(gate);
  free(up);
  free(o);
  return 0;
}
