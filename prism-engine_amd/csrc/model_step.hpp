// model_step.hpp -- prism_hip_model: the GPU-resident decode step.
// Included once, at the end of prism_hip.hip (it uses that file's
// validation helpers and GEMV launcher).  Declarations and contract:
// include/prism_hip.h.
//
// HBM layout per model (all model-owned):
//   embed            [vocab x hidden] 4-bit split-block (also the LM head)
//   per layer        qkv: q, k and v fused into one [(nh+2*nkv)*64 x hidden]
//                    split-block matrix (LUT rows q|k|v, then index rows
//                    q|k|v), o, gate, up, down as given
//   KV cache         int8 K and V planes [layer][max_seq][kv_dim] and fp32
//                    scales [layer][max_seq]
//   RoPE table       (cos, sin) [max_seq][32], built on the host with the C
//                    library's powf / sinf / cosf -- the functions the
//                    reference's rope_inplace calls -- so the device
//                    rotation uses the reference's angles bit for bit
//   activations      residual stream h [hidden], q|k|v [nqkv], attention
//                    split partials [nh][kAttnSplits][66] fp32, SwiGLU output
//                    [intermediate], logits [vocab] fp16; StepParams
// One step = k_step_begin (token, pos, KV lengths by value: stores them and
// the token's embedding row) + one graph replay of the fixed launch
// sequence (captured once per weight set).
#pragma once
#include <cmath>
#include <vector>

struct prism_hip_model {
  prism_hip_ctx* ctx = nullptr;
  int device = 0;
  prism_hip_model_config cfg{};
  uint32_t qd = 0, kvd = 0, nqkv = 0;
  uint8_t* embed = nullptr;
  bool embed_set = false;
  std::vector<uint8_t*> qkv, o, gate, up, down;
  std::vector<bool> layer_set;
  int8_t* kq = nullptr;
  int8_t* vq = nullptr;
  float* ks = nullptr;
  float* vs = nullptr;
  float2* rope = nullptr;
  uint16_t* hres = nullptr;
  uint16_t* qkv_out = nullptr;
  uint16_t* act = nullptr;
  uint16_t* logits = nullptr;
  prism::StepParams* d_params = nullptr;
  float* attn_part = nullptr;     // k_step_attention split partials
  std::vector<uint32_t> kv_len;
  hipStream_t cap_stream = nullptr;
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
  std::vector<void*> allocs;
};

static void model_detach(prism_hip_model* m) { m->ctx = nullptr; }

namespace {

size_t payload4(uint32_t rows, uint32_t k) { return (size_t)rows * 32 + (size_t)rows * (k / 2); }

void model_release(prism_hip_model* m) {
  DeviceGuard g(m->device);
  if (m->exec) (void)hipGraphExecDestroy(m->exec);
  if (m->graph) (void)hipGraphDestroy(m->graph);
  if (m->cap_stream) (void)hipStreamDestroy(m->cap_stream);
  for (void* p : m->allocs) (void)hipFree(p);
  m->allocs.clear();
  m->exec = nullptr;
  m->graph = nullptr;
  m->cap_stream = nullptr;
}

template <class T>
int model_alloc(prism_hip_model* m, T** p, size_t bytes) {
  void* d = nullptr;
  HIP_TRY(m->ctx, hipMalloc(&d, bytes ? bytes : 16));
  m->allocs.push_back(d);
  *p = reinterpret_cast<T*>(d);
  return PRISM_HIP_OK;
}

void model_invalidate(prism_hip_model* m) {
  if (m->exec) (void)hipGraphExecDestroy(m->exec);
  if (m->graph) (void)hipGraphDestroy(m->graph);
  m->exec = nullptr;
  m->graph = nullptr;
}

int model_check(prism_hip_model* m) {
  if (!m) return PRISM_HIP_ERR_NULL;
  if (!m->ctx) return PRISM_HIP_ERR_CONTEXT;
  return PRISM_HIP_OK;
}

int check_w4(prism_hip_ctx* ctx, const prism_hip_weight* w, const char* what, uint32_t rows, uint32_t k) {
  int rc = check_weight(ctx, w);
  if (rc) return rc;
  if (w->bits != 4) return fail(ctx, PRISM_HIP_ERR_BITS, "%s: the decode step takes 4-bit weights", what);
  if (w->dim_m != rows || w->dim_n != k)
    return fail(ctx, PRISM_HIP_ERR_SHAPE, "%s is %ux%u, the config needs %ux%u", what, w->dim_m, w->dim_n, rows, k);
  return PRISM_HIP_OK;
}

// The fixed per-token launch sequence (captured into the model's graph).
int model_enqueue(prism_hip_model* m, hipStream_t st) {
  prism_hip_ctx* ctx = m->ctx;
  const prism_hip_model_config& c = m->cfg;
  const uint32_t D = c.hidden, I = c.intermediate, V = c.vocab;
  const float eps = c.rms_eps;
  int rc;
  for (uint32_t l = 0; l < c.n_layers; l++) {
    const uint8_t* wq = m->qkv[l];
    if ((rc = launch_gemv_raw(ctx, 4, m->nqkv, D, wq, wq + (size_t)m->nqkv * 32, nullptr, nullptr, m->hres, 1,
                              m->qkv_out, st, prism::kEpiNorm, eps)))
      return rc;
    prism::AttnArgs aa;
    aa.qkv = m->qkv_out;
    aa.kq = m->kq + (size_t)l * c.max_seq * m->kvd;
    aa.ks = m->ks + (size_t)l * c.max_seq;
    aa.vq = m->vq + (size_t)l * c.max_seq * m->kvd;
    aa.vs = m->vs + (size_t)l * c.max_seq;
    aa.rope = m->rope;
    aa.sp = m->d_params;
    aa.part = m->attn_part;
    aa.layer = l;
    aa.nh = c.n_heads;
    aa.nkv = c.n_kv_heads;
    hipLaunchKernelGGL(prism::k_step_attention, dim3(c.n_heads * prism::kAttnSplits), dim3(prism::kAttnThreads), 0,
                       st, aa);
    HIP_TRY(ctx, hipGetLastError());
    // O projection: x = the attention output, combined from the split
    // partials in the GEMV's prologue; residual add in its epilogue
    const uint8_t* wo = m->o[l];
    if ((rc = launch_gemv_raw(ctx, 4, D, m->qd, wo, wo + (size_t)D * 32, nullptr, nullptr, nullptr, 1, m->hres, st,
                              prism::kEpiAttnIn | prism::kEpiResid, 0.0f, m->attn_part)))
      return rc;
    const uint8_t* wg = m->gate[l];
    const uint8_t* wu = m->up[l];
    if ((rc = launch_gemv_raw(ctx, 4, I, D, wg, wg + (size_t)I * 32, wu, wu + (size_t)I * 32, m->hres, 1, m->act,
                              st, prism::kEpiNorm, eps)))
      return rc;
    const uint8_t* wd = m->down[l];
    if ((rc = launch_gemv_raw(ctx, 4, D, I, wd, wd + (size_t)D * 32, nullptr, nullptr, m->act, 1, m->hres, st,
                              prism::kEpiResid)))
      return rc;
  }
  return launch_gemv_raw(ctx, 4, V, D, m->embed, m->embed + (size_t)V * 32, nullptr, nullptr, m->hres, 1, m->logits,
                         st, prism::kEpiNorm, eps);
}

int model_ready(prism_hip_model* m) {
  if (!m->embed_set) return fail(m->ctx, PRISM_HIP_ERR_SHAPE, "model has no embedding");
  for (uint32_t l = 0; l < m->cfg.n_layers; l++)
    if (!m->layer_set[l]) return fail(m->ctx, PRISM_HIP_ERR_SHAPE, "model layer %u has no weights", l);
  return PRISM_HIP_OK;
}

}  // namespace

extern "C" {

prism_hip_model* prism_hip_model_create(prism_hip_ctx* ctx, const prism_hip_model_config* cfg) {
  if (!ctx) return nullptr;
  if (!cfg) {
    fail(ctx, PRISM_HIP_ERR_NULL, "config is NULL");
    return nullptr;
  }
  const prism_hip_model_config& c = *cfg;
  if (c.head_dim != 64 || c.n_heads == 0 || c.n_kv_heads == 0 || c.n_heads % c.n_kv_heads != 0 ||
      c.n_kv_heads * 64 > 256 || c.hidden == 0 || c.hidden % 8 != 0 || c.intermediate == 0 ||
      c.intermediate % 8 != 0 || c.vocab == 0 || c.n_layers > (uint32_t)prism::kMaxLayers || c.max_seq == 0 ||
      c.max_seq > (uint32_t)prism::kAttnMaxSeq - 1) {
    fail(ctx, PRISM_HIP_ERR_SHAPE,
         "unsupported config: head_dim %u (64), heads %u/%u (kv heads*64 <= 256), hidden %u, intermediate %u "
         "(multiples of 8), vocab %u, layers %u (<= %d), max_seq %u (1..%d)",
         c.head_dim, c.n_heads, c.n_kv_heads, c.hidden, c.intermediate, c.vocab, c.n_layers, prism::kMaxLayers,
         c.max_seq, prism::kAttnMaxSeq - 1);
    return nullptr;
  }
  DeviceGuard g(ctx->device);
  auto* m = new prism_hip_model;
  m->ctx = ctx;
  m->device = ctx->device;
  m->cfg = c;
  m->qd = c.n_heads * 64;
  m->kvd = c.n_kv_heads * 64;
  m->nqkv = m->qd + 2 * m->kvd;
  const uint32_t L = c.n_layers, D = c.hidden, I = c.intermediate;
  m->qkv.assign(L, nullptr);
  m->o.assign(L, nullptr);
  m->gate.assign(L, nullptr);
  m->up.assign(L, nullptr);
  m->down.assign(L, nullptr);
  m->layer_set.assign(L, false);
  m->kv_len.assign(L, 0);
  int rc = PRISM_HIP_OK;
  for (uint32_t l = 0; l < L && !rc; l++) {
    rc = model_alloc(m, &m->qkv[l], payload4(m->nqkv, D));
    if (!rc) rc = model_alloc(m, &m->o[l], payload4(D, m->qd));
    if (!rc) rc = model_alloc(m, &m->gate[l], payload4(I, D));
    if (!rc) rc = model_alloc(m, &m->up[l], payload4(I, D));
    if (!rc) rc = model_alloc(m, &m->down[l], payload4(D, I));
  }
  const size_t kvn = (size_t)(L ? L : 1) * c.max_seq;
  if (!rc) rc = model_alloc(m, &m->embed, payload4(c.vocab, D));
  if (!rc) rc = model_alloc(m, &m->kq, kvn * m->kvd);
  if (!rc) rc = model_alloc(m, &m->vq, kvn * m->kvd);
  if (!rc) rc = model_alloc(m, &m->ks, kvn * 4);
  if (!rc) rc = model_alloc(m, &m->vs, kvn * 4);
  if (!rc) rc = model_alloc(m, &m->rope, (size_t)c.max_seq * 32 * sizeof(float2));
  if (!rc) rc = model_alloc(m, &m->hres, (size_t)D * 2);
  if (!rc) rc = model_alloc(m, &m->qkv_out, (size_t)m->nqkv * 2);
  if (!rc) rc = model_alloc(m, &m->act, (size_t)I * 2);
  if (!rc) rc = model_alloc(m, &m->logits, (size_t)c.vocab * 2);
  if (!rc) rc = model_alloc(m, &m->d_params, sizeof(prism::StepParams));
  if (!rc) rc = model_alloc(m, &m->attn_part, (size_t)c.n_heads * prism::kAttnSplits * (2 + 64) * 4);

  if (!rc) {
    // RoPE angles pos * 10000^(-2j/64) with the C library's powf/sinf/cosf,
    // exactly as rope_inplace computes them (evaluator.rs:154-166).
    std::vector<float2> tab((size_t)c.max_seq * 32);
    for (uint32_t p = 0; p < c.max_seq; p++)
      for (uint32_t j = 0; j < 32; j++) {
        const float ang = (float)p * powf(10000.0f, (-2.0f * (float)j) / 64.0f);
        tab[(size_t)p * 32 + j] = make_float2(cosf(ang), sinf(ang));
      }
    hipError_t e = hipMemcpy(m->rope, tab.data(), tab.size() * sizeof(float2), hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipStreamCreateWithFlags(&m->cap_stream, hipStreamNonBlocking);
    if (e != hipSuccess) rc = fail(ctx, PRISM_HIP_ERR_DEVICE, "model setup: %s", hipGetErrorString(e));
  }
  if (rc) {
    model_release(m);
    delete m;
    return nullptr;
  }
  ctx->models.insert(m);
  ctx->err.clear();
  return m;
}

void prism_hip_model_free(prism_hip_model* m) {
  if (!m) return;
  if (m->ctx) m->ctx->models.erase(m);
  model_release(m);
  delete m;
}

int prism_hip_model_set_embedding(prism_hip_model* m, const prism_hip_weight* embed) {
  int rc = model_check(m);
  if (rc) return rc;
  prism_hip_ctx* ctx = m->ctx;
  if ((rc = check_w4(ctx, embed, "embedding", m->cfg.vocab, m->cfg.hidden))) return rc;
  DeviceGuard g(m->device);
  if ((rc = copy_split_rows(ctx, embed, m->embed, m->embed + (size_t)m->cfg.vocab * 32, ctx->stream))) return rc;
  HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
  m->embed_set = true;
  model_invalidate(m);
  ctx->err.clear();
  return PRISM_HIP_OK;
}

int prism_hip_model_set_layer(prism_hip_model* m, uint32_t layer, const prism_hip_weight* q_proj,
                              const prism_hip_weight* k_proj, const prism_hip_weight* v_proj,
                              const prism_hip_weight* o_proj, const prism_hip_weight* gate_proj,
                              const prism_hip_weight* up_proj, const prism_hip_weight* down_proj) {
  int rc = model_check(m);
  if (rc) return rc;
  prism_hip_ctx* ctx = m->ctx;
  const prism_hip_model_config& c = m->cfg;
  if (layer >= c.n_layers) return fail(ctx, PRISM_HIP_ERR_SHAPE, "layer %u of %u", layer, c.n_layers);
  const uint32_t D = c.hidden, I = c.intermediate;
  if ((rc = check_w4(ctx, q_proj, "q_proj", m->qd, D)) || (rc = check_w4(ctx, k_proj, "k_proj", m->kvd, D)) ||
      (rc = check_w4(ctx, v_proj, "v_proj", m->kvd, D)) || (rc = check_w4(ctx, o_proj, "o_proj", D, m->qd)) ||
      (rc = check_w4(ctx, gate_proj, "gate_proj", I, D)) || (rc = check_w4(ctx, up_proj, "up_proj", I, D)) ||
      (rc = check_w4(ctx, down_proj, "down_proj", D, I)))
    return rc;
  DeviceGuard g(m->device);
  hipStream_t st = ctx->stream;
  // fused QKV: LUT rows q|k|v, then index rows q|k|v
  uint8_t* f = m->qkv[layer];
  const prism_hip_weight* parts[3] = {q_proj, k_proj, v_proj};
  size_t lut_off = 0, idx_off = (size_t)m->nqkv * 32;
  for (const prism_hip_weight* w : parts) {
    const size_t lb = (size_t)w->dim_m * 32, ib = (size_t)w->dim_m * (D / 2);
    if ((rc = copy_split_rows(ctx, w, f + lut_off, f + idx_off, st))) return rc;
    lut_off += lb;
    idx_off += ib;
  }
  // the other projections keep their own split-block buffers
  const prism_hip_weight* own[4] = {o_proj, gate_proj, up_proj, down_proj};
  uint8_t* dst[4] = {m->o[layer], m->gate[layer], m->up[layer], m->down[layer]};
  for (int i = 0; i < 4; i++)
    if ((rc = copy_split_rows(ctx, own[i], dst[i], dst[i] + (size_t)own[i]->dim_m * 32, st))) return rc;
  HIP_TRY(ctx, hipStreamSynchronize(st));
  m->layer_set[layer] = true;
  model_invalidate(m);
  ctx->err.clear();
  return PRISM_HIP_OK;
}

int prism_hip_model_kv_append(prism_hip_model* m, uint32_t layer, const uint16_t* k, const uint16_t* v,
                              uint32_t ntokens) {
  int rc = model_check(m);
  if (rc) return rc;
  prism_hip_ctx* ctx = m->ctx;
  const prism_hip_model_config& c = m->cfg;
  if (layer >= c.n_layers) return fail(ctx, PRISM_HIP_ERR_SHAPE, "layer %u of %u", layer, c.n_layers);
  if (ntokens == 0) return PRISM_HIP_OK;
  if (!k || !v) return fail(ctx, PRISM_HIP_ERR_NULL, "k or v is NULL");
  if ((uint64_t)m->kv_len[layer] + ntokens > c.max_seq)
    return fail(ctx, PRISM_HIP_ERR_SIZE, "layer %u: %u + %u tokens exceed max_seq %u", layer, m->kv_len[layer],
                ntokens, c.max_seq);
  DeviceGuard g(m->device);
  const size_t rb = (size_t)ntokens * m->kvd * 2;
  if ((rc = ensure_stage(ctx, 2 * rb))) return rc;
  hipStream_t st = ctx->stream;
  uint16_t* dk = reinterpret_cast<uint16_t*>(ctx->d_stage);
  uint16_t* dv = dk + (size_t)ntokens * m->kvd;
  HIP_TRY(ctx, hipMemcpyAsync(dk, k, rb, hipMemcpyHostToDevice, st));
  HIP_TRY(ctx, hipMemcpyAsync(dv, v, rb, hipMemcpyHostToDevice, st));
  const size_t po = (size_t)layer * c.max_seq;
  hipLaunchKernelGGL(prism::k_kv_quant_rows, dim3(ntokens), dim3(256), 0, st, dk, ntokens, m->kvd,
                     m->kq + po * m->kvd, m->ks + po, m->kv_len[layer]);
  HIP_TRY(ctx, hipGetLastError());
  hipLaunchKernelGGL(prism::k_kv_quant_rows, dim3(ntokens), dim3(256), 0, st, dv, ntokens, m->kvd,
                     m->vq + po * m->kvd, m->vs + po, m->kv_len[layer]);
  HIP_TRY(ctx, hipGetLastError());
  HIP_TRY(ctx, hipStreamSynchronize(st));
  m->kv_len[layer] += ntokens;
  ctx->err.clear();
  return PRISM_HIP_OK;
}

int prism_hip_model_kv_len(const prism_hip_model* m, uint32_t layer, uint32_t* len) {
  if (!m || !len) return PRISM_HIP_ERR_NULL;
  if (layer >= m->cfg.n_layers) return PRISM_HIP_ERR_SHAPE;
  *len = m->kv_len[layer];
  return PRISM_HIP_OK;
}

int prism_hip_model_kv_read(prism_hip_model* m, uint32_t layer, uint8_t* k_blocks, uint8_t* v_blocks) {
  int rc = model_check(m);
  if (rc) return rc;
  prism_hip_ctx* ctx = m->ctx;
  if (layer >= m->cfg.n_layers) return fail(ctx, PRISM_HIP_ERR_SHAPE, "layer %u of %u", layer, m->cfg.n_layers);
  if (!k_blocks || !v_blocks) return fail(ctx, PRISM_HIP_ERR_NULL, "output is NULL");
  const uint32_t n = m->kv_len[layer], kvd = m->kvd;
  if (n == 0) return PRISM_HIP_OK;
  DeviceGuard g(m->device);
  // steps enqueued on the context stream finish first (other streams are
  // the caller's to synchronize)
  HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
  std::vector<int8_t> q((size_t)n * kvd);
  std::vector<float> s(n);
  const size_t po = (size_t)layer * m->cfg.max_seq;
  for (int which = 0; which < 2; which++) {
    const int8_t* dq = (which ? m->vq : m->kq) + po * kvd;
    const float* ds = (which ? m->vs : m->ks) + po;
    HIP_TRY(ctx, hipMemcpy(q.data(), dq, q.size(), hipMemcpyDeviceToHost));
    HIP_TRY(ctx, hipMemcpy(s.data(), ds, s.size() * 4, hipMemcpyDeviceToHost));
    uint8_t* out = which ? v_blocks : k_blocks;
    for (uint32_t t = 0; t < n; t++) {
      std::memcpy(out + (size_t)t * (kvd + 4), &s[t], 4);
      std::memcpy(out + (size_t)t * (kvd + 4) + 4, q.data() + (size_t)t * kvd, kvd);
    }
  }
  ctx->err.clear();
  return PRISM_HIP_OK;
}

int prism_hip_model_kv_reset(prism_hip_model* m) {
  int rc = model_check(m);
  if (rc) return rc;
  for (auto& n : m->kv_len) n = 0;
  return PRISM_HIP_OK;
}

int prism_hip_model_kv_truncate(prism_hip_model* m, uint32_t len) {
  int rc = model_check(m);
  if (rc) return rc;
  for (auto& n : m->kv_len) n = n < len ? n : len;
  return PRISM_HIP_OK;
}

int prism_hip_model_step_dev(prism_hip_model* m, uint32_t token, int64_t pos, void* stream) {
  int rc = model_check(m);
  if (rc) return rc;
  prism_hip_ctx* ctx = m->ctx;
  const prism_hip_model_config& c = m->cfg;
  if ((rc = model_ready(m))) return rc;
  if (pos < 0 || pos >= (int64_t)c.max_seq)
    return fail(ctx, PRISM_HIP_ERR_SHAPE, "pos %lld outside 0..%u", (long long)pos, c.max_seq - 1);
  prism::StepParams p;
  std::memset(&p, 0, sizeof p);
  p.token = token;
  p.pos = (uint32_t)pos;
  for (uint32_t l = 0; l < c.n_layers; l++) {
    if (m->kv_len[l] >= c.max_seq)
      return fail(ctx, PRISM_HIP_ERR_SIZE, "layer %u KV cache is full (%u tokens)", l, c.max_seq);
    p.kv_len[l] = m->kv_len[l];
  }
  DeviceGuard g(m->device);
  hipStream_t st = pick_stream(ctx, stream);
  if (!m->exec) {
    HIP_TRY(ctx, hipStreamBeginCapture(m->cap_stream, hipStreamCaptureModeThreadLocal));
    rc = model_enqueue(m, m->cap_stream);
    hipGraph_t gr = nullptr;
    hipError_t e = hipStreamEndCapture(m->cap_stream, &gr);
    if (rc) {
      if (gr) (void)hipGraphDestroy(gr);
      return rc;
    }
    if (e != hipSuccess) return fail(ctx, PRISM_HIP_ERR_DEVICE, "step capture: %s", hipGetErrorString(e));
    m->graph = gr;
    HIP_TRY(ctx, hipGraphInstantiate(&m->exec, m->graph, nullptr, nullptr, 0));
  }
  hipLaunchKernelGGL(prism::k_step_begin, dim3(1), dim3(256), 0, st, p, m->d_params, m->embed, c.vocab, c.hidden,
                     m->hres);
  HIP_TRY(ctx, hipGetLastError());
  HIP_TRY(ctx, hipGraphLaunch(m->exec, st));
  for (uint32_t l = 0; l < c.n_layers; l++) m->kv_len[l] += 1;
  ctx->err.clear();
  return PRISM_HIP_OK;
}

int prism_hip_model_step(prism_hip_model* m, uint32_t token, int64_t pos, uint16_t* logits) {
  int rc = model_check(m);
  if (rc) return rc;
  prism_hip_ctx* ctx = m->ctx;
  if (!logits) return fail(ctx, PRISM_HIP_ERR_NULL, "logits is NULL");
  if ((rc = prism_hip_model_step_dev(m, token, pos, nullptr))) return rc;
  DeviceGuard g(m->device);
  HIP_TRY(ctx, hipMemcpyAsync(logits, m->logits, (size_t)m->cfg.vocab * 2, hipMemcpyDeviceToHost, ctx->stream));
  HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
  return PRISM_HIP_OK;
}

const void* prism_hip_model_logits_dev(const prism_hip_model* m) { return m ? m->logits : nullptr; }

}  // extern "C"
