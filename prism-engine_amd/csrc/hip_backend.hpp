// hip_backend.hpp -- C++ HipBackend, the MI355X counterpart of the
// reference's MetalBackend (src/lut/engine_impl.rs:31-490).
//
// Same surface and meaning:
//   MetalBackend::new(tensors, ...)          -> HipBackend::create + add_tensor
//   MetalBackend::gemv(key, inp, out)        -> HipBackend::gemv
//   MetalBackend::fused_gate_up(g, u, x, y)  -> HipBackend::fused_gate_up
// Errors are the reference's `Result<(), String>`: an empty string is Ok,
// anything else is the Err text ("miss <key>" for an unknown tensor, as at
// engine_impl.rs:156-159).  Every compute method is synchronous on the
// backend's stream, like the reference's commit + wait_until_completed;
// add_tensor only enqueues its device copy (synchronize() waits for them).
// Unlike the reference's caller (PrismEngine::gemv, engine_impl.rs:1489-1504)
// nothing here falls back to the CPU: an Err is the caller's to handle.
#pragma once
#include <cstddef>
#include <cstdint>
#include <memory>
#include <string>
#include <unordered_map>

#include "prism_hip.h"

namespace prism {

class HipBackend {
 public:
  // Returns nullptr and sets *err on failure.
  static std::unique_ptr<HipBackend> create(int device, std::string* err);
  ~HipBackend();
  HipBackend(const HipBackend&) = delete;
  HipBackend& operator=(const HipBackend&) = delete;

  // One CompiledTensor {key, dim_m, dim_n, payload} (src/lut/compiler.rs:14-20).
  std::string add_tensor(const std::string& key, const uint8_t* payload, size_t bytes, uint32_t dim_m,
                         uint32_t dim_n, uint32_t bits);
  std::string gemv(const std::string& key, const uint16_t* inp, size_t inp_len, uint16_t* out, size_t out_len);
  std::string fused_gate_up(const std::string& gate_key, const std::string& up_key, const uint16_t* input,
                            size_t in_len, uint16_t* output, size_t out_len);
  std::string gemm(const std::string& key, const uint16_t* X, uint32_t M, uint16_t* Y);
  std::string embed(const std::string& key, uint32_t token, uint16_t* out, size_t out_len);
  // Waits for every add_tensor upload (they are asynchronous on the stream).
  std::string synchronize();

  size_t len() const { return weights_.size(); }
  const prism_hip_weight* find(const std::string& key) const;
  prism_hip_ctx* ctx() const { return ctx_; }

 private:
  explicit HipBackend(prism_hip_ctx* ctx) : ctx_(ctx) {}
  std::string hip_err(int rc) const;
  prism_hip_ctx* ctx_;
  std::unordered_map<std::string, prism_hip_weight*> weights_;
};

}  // namespace prism
