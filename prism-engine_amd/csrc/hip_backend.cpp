// hip_backend.cpp -- HipBackend (see hip_backend.hpp) and its C ABI
// (prism_hip_backend_* in include/prism_hip.h).
#include "hip_backend.hpp"

#include <string>

namespace prism {

std::unique_ptr<HipBackend> HipBackend::create(int device, std::string* err) {
  prism_hip_ctx* ctx = prism_hip_ctx_create(device);
  if (!ctx) {
    if (err) *err = prism_hip_last_error(nullptr);
    return nullptr;
  }
  return std::unique_ptr<HipBackend>(new HipBackend(ctx));
}

HipBackend::~HipBackend() {
  for (auto& kv : weights_) prism_hip_weight_free(kv.second);
  weights_.clear();
  prism_hip_ctx_destroy(ctx_);
}

std::string HipBackend::hip_err(int rc) const {
  std::string s = prism_hip_last_error(ctx_);
  if (s.empty()) s = "prism_hip error " + std::to_string(rc);
  return s;
}

const prism_hip_weight* HipBackend::find(const std::string& key) const {
  auto it = weights_.find(key);
  return it == weights_.end() ? nullptr : it->second;
}

std::string HipBackend::add_tensor(const std::string& key, const uint8_t* payload, size_t bytes, uint32_t dim_m,
                                   uint32_t dim_n, uint32_t bits) {
  // asynchronous: every other call of the backend runs on the same stream,
  // after the copy; synchronize() waits for all of them
  prism_hip_weight* w =
      prism_hip_weight_upload_async(ctx_, payload, bytes, dim_m, dim_n, bits, PRISM_HIP_LAYOUT_SPLIT_BLOCK);
  if (!w) return key + ": " + prism_hip_last_error(ctx_);
  auto it = weights_.find(key);
  if (it != weights_.end()) {
    prism_hip_weight_free(it->second);
    it->second = w;
  } else {
    weights_.emplace(key, w);
  }
  return "";
}

std::string HipBackend::synchronize() {
  const int rc = prism_hip_ctx_synchronize(ctx_);
  return rc == PRISM_HIP_OK ? "" : hip_err(rc);
}

std::string HipBackend::gemv(const std::string& key, const uint16_t* inp, size_t inp_len, uint16_t* out,
                             size_t out_len) {
  const prism_hip_weight* w = find(key);
  if (!w) return "miss " + key;  // engine_impl.rs:156-159
  uint32_t dm = 0, dn = 0;
  prism_hip_weight_info(w, &dm, &dn, nullptr, nullptr);
  if (inp_len == 0 || inp_len % dn != 0)
    return key + ": input has " + std::to_string(inp_len) + " values, dim_n is " + std::to_string(dn);
  const size_t batch = inp_len / dn;
  if (out_len != batch * dm)
    return key + ": output has " + std::to_string(out_len) + " values, needs " + std::to_string(batch * dm);
  const int rc = prism_hip_gemv(ctx_, w, inp, (uint32_t)batch, out);
  return rc == PRISM_HIP_OK ? "" : hip_err(rc);
}

std::string HipBackend::fused_gate_up(const std::string& gate_key, const std::string& up_key, const uint16_t* input,
                                      size_t in_len, uint16_t* output, size_t out_len) {
  const prism_hip_weight* g = find(gate_key);
  if (!g) return "miss " + gate_key;  // engine_impl.rs:450-453
  const prism_hip_weight* u = find(up_key);
  if (!u) return "miss " + up_key;  // engine_impl.rs:454-457
  uint32_t dm = 0, dn = 0;
  prism_hip_weight_info(g, &dm, &dn, nullptr, nullptr);
  if (in_len != dn) return gate_key + ": input has " + std::to_string(in_len) + " values, dim_n is " + std::to_string(dn);
  if (out_len != dm)
    return gate_key + ": output has " + std::to_string(out_len) + " values, dim_m is " + std::to_string(dm);
  const int rc = prism_hip_gateup_swiglu(ctx_, g, u, input, output);
  return rc == PRISM_HIP_OK ? "" : hip_err(rc);
}

std::string HipBackend::gemm(const std::string& key, const uint16_t* X, uint32_t M, uint16_t* Y) {
  const prism_hip_weight* w = find(key);
  if (!w) return "miss " + key;
  const int rc = prism_hip_gemm(ctx_, w, X, M, Y);
  return rc == PRISM_HIP_OK ? "" : hip_err(rc);
}

std::string HipBackend::embed(const std::string& key, uint32_t token, uint16_t* out, size_t out_len) {
  const prism_hip_weight* w = find(key);
  if (!w) return "miss " + key;
  uint32_t dn = 0;
  prism_hip_weight_info(w, nullptr, &dn, nullptr, nullptr);
  if (out_len != dn) return key + ": output has " + std::to_string(out_len) + " values, dim_n is " + std::to_string(dn);
  const int rc = prism_hip_lut_embed(ctx_, w, token, out);
  return rc == PRISM_HIP_OK ? "" : hip_err(rc);
}

}  // namespace prism

// ---- C ABI ---------------------------------------------------------------

struct prism_hip_backend {
  std::unique_ptr<prism::HipBackend> impl;
  std::string err;
};

namespace {
thread_local std::string g_backend_create_err;

int finish(prism_hip_backend* b, const std::string& e, int code_on_err) {
  b->err = e;
  return e.empty() ? PRISM_HIP_OK : code_on_err;
}

// Map an error string to its code: "miss <key>" -> ERR_KEY, else the
// context's code class (shape/device) as reported.
int code_for(const std::string& e) {
  if (e.rfind("miss ", 0) == 0) return PRISM_HIP_ERR_KEY;
  if (e.find("values") != std::string::npos) return PRISM_HIP_ERR_SHAPE;
  if (e.find("payload is") != std::string::npos) return PRISM_HIP_ERR_SIZE;
  if (e.find("bits must") != std::string::npos) return PRISM_HIP_ERR_BITS;
  if (e.find("differ") != std::string::npos) return PRISM_HIP_ERR_MISMATCH;
  if (e.find("empty shape") != std::string::npos) return PRISM_HIP_ERR_SHAPE;
  return PRISM_HIP_ERR_DEVICE;
}
}  // namespace

extern "C" {

prism_hip_backend* prism_hip_backend_new(int device) {
  std::string err;
  auto impl = prism::HipBackend::create(device, &err);
  if (!impl) {
    g_backend_create_err = err;
    return nullptr;
  }
  auto* b = new prism_hip_backend;
  b->impl = std::move(impl);
  return b;
}

void prism_hip_backend_free(prism_hip_backend* b) { delete b; }

const char* prism_hip_backend_last_error(const prism_hip_backend* b) {
  return b ? b->err.c_str() : g_backend_create_err.c_str();
}

int prism_hip_backend_add_tensor(prism_hip_backend* b, const char* key, const uint8_t* payload, size_t bytes,
                                 uint32_t dim_m, uint32_t dim_n, uint32_t bits) {
  if (!b) return PRISM_HIP_ERR_NULL;
  if (!key || !payload) return finish(b, "key or payload is NULL", PRISM_HIP_ERR_NULL);
  const std::string e = b->impl->add_tensor(key, payload, bytes, dim_m, dim_n, bits);
  return finish(b, e, code_for(e));
}

int prism_hip_backend_gemv(prism_hip_backend* b, const char* key, const uint16_t* inp, size_t inp_len, uint16_t* out,
                           size_t out_len) {
  if (!b) return PRISM_HIP_ERR_NULL;
  if (!key || !inp || !out) return finish(b, "key, input or output is NULL", PRISM_HIP_ERR_NULL);
  const std::string e = b->impl->gemv(key, inp, inp_len, out, out_len);
  return finish(b, e, code_for(e));
}

int prism_hip_backend_fused_gate_up(prism_hip_backend* b, const char* gate_key, const char* up_key,
                                    const uint16_t* input, size_t in_len, uint16_t* output, size_t out_len) {
  if (!b) return PRISM_HIP_ERR_NULL;
  if (!gate_key || !up_key || !input || !output) return finish(b, "a key or buffer is NULL", PRISM_HIP_ERR_NULL);
  const std::string e = b->impl->fused_gate_up(gate_key, up_key, input, in_len, output, out_len);
  return finish(b, e, code_for(e));
}

int prism_hip_backend_gemm(prism_hip_backend* b, const char* key, const uint16_t* X, uint32_t M, uint16_t* Y) {
  if (!b) return PRISM_HIP_ERR_NULL;
  if (!key || !X || !Y) return finish(b, "key, X or Y is NULL", PRISM_HIP_ERR_NULL);
  const std::string e = b->impl->gemm(key, X, M, Y);
  return finish(b, e, code_for(e));
}

int prism_hip_backend_embed(prism_hip_backend* b, const char* key, uint32_t token, uint16_t* out, size_t out_len) {
  if (!b) return PRISM_HIP_ERR_NULL;
  if (!key || !out) return finish(b, "key or output is NULL", PRISM_HIP_ERR_NULL);
  const std::string e = b->impl->embed(key, token, out, out_len);
  return finish(b, e, code_for(e));
}

size_t prism_hip_backend_len(const prism_hip_backend* b) { return b ? b->impl->len() : 0; }

int prism_hip_backend_synchronize(prism_hip_backend* b) {
  if (!b) return PRISM_HIP_ERR_NULL;
  const std::string e = b->impl->synchronize();
  return finish(b, e, e.empty() ? PRISM_HIP_OK : PRISM_HIP_ERR_DEVICE);
}

}  // extern "C"
