/*
 * prism_hip.h -- C ABI of the MI355X (gfx950) palettized-LUT contraction.
 *
 * This is the `extern "C"` layer the reference's `prism-ffi` crate would
 * bind (prism-ffi/src/lib.rs:28-90 sets the conventions: opaque handles,
 * constructors that return NULL on failure, `*_free` that accepts NULL,
 * `int` results with 0 = OK and a distinct negative code per failure, -2 =
 * backend not linked).  Plain pointers and sizes only.
 *
 * Weight payloads use the reference's split-block `.cimage` layout
 * (src/lut/compiler.rs:50-61, read by compute-core/src/lut/evaluator.rs:14-31):
 *
 *   4-bit: [dim_m x 16 fp16 LUT, LE][dim_m x (dim_n/2) packed nibbles]
 *          element 2i = low nibble of byte i, 2i+1 = high nibble
 *          (src/quantization/palette.rs:207-212)
 *   8-bit: [dim_m x 256 fp16 LUT, LE][dim_m x dim_n index bytes]
 *          (build extension; format of compute-core/tests/
 *           palettized_vs_direct.rs:108-135 laid out split-block)
 *
 * Semantics follow lut_gemv_cpu (compute-core/src/lut/evaluator.rs:21-44):
 * fp32 accumulation, fp16 (round-to-nearest-even) output.  For 4-bit
 * weights only the first (dim_n/8)*8 elements of a row contribute and rows
 * are dim_n/2 bytes apart, exactly as in the reference.
 *
 * Thread model: a context owns one HIP stream and is not reentrant; callers
 * serialise calls on one context (one context per thread is fine).  Entry
 * points that take host pointers are synchronous, like
 * MetalBackend::gemv (src/lut/engine_impl.rs:155-190).  `*_dev` entry points
 * take device pointers and a hipStream_t (passed as void*, NULL = the
 * context's stream) and are asynchronous.
 */
#ifndef PRISM_HIP_H
#define PRISM_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- result codes (compute-core/src/ffi.rs:28-43 style) ---------------- */
#define PRISM_HIP_OK 0
#define PRISM_HIP_ERR_NULL (-1)       /* a required pointer is NULL                 */
#define PRISM_HIP_ERR_NOT_LINKED (-2) /* backend not linked (prism-ffi/src/lib.rs:52-56) */
#define PRISM_HIP_ERR_SHAPE (-3)      /* dim/batch out of range or inconsistent     */
#define PRISM_HIP_ERR_BITS (-4)       /* bits not in {4, 8}                          */
#define PRISM_HIP_ERR_SIZE (-5)       /* payload bytes != expected for the shape     */
#define PRISM_HIP_ERR_LAYOUT (-6)     /* unknown layout code                          */
#define PRISM_HIP_ERR_DEVICE (-7)     /* HIP runtime error (see last_error)          */
#define PRISM_HIP_ERR_MISMATCH (-8)   /* gate/up weights disagree in shape or bits  */
#define PRISM_HIP_ERR_KEY (-9)        /* backend: no tensor under that key          */
#define PRISM_HIP_ERR_CONTEXT (-10)   /* weight belongs to another context/device   */

#define PRISM_HIP_LAYOUT_SPLIT_BLOCK 0u

typedef struct prism_hip_ctx prism_hip_ctx;
typedef struct prism_hip_weight prism_hip_weight;
typedef struct prism_hip_backend prism_hip_backend;

/* ---- context ------------------------------------------------------------ */

/* Replaces the device/queue half of MetalBackend::new
 * (src/lut/engine_impl.rs:51-57,106-107): selects `device`, creates the
 * context's stream and its staging buffers.  NULL on failure. */
prism_hip_ctx* prism_hip_ctx_create(int device);
void prism_hip_ctx_destroy(prism_hip_ctx* ctx); /* accepts NULL */

/* Last error text of this context ("" when none).  The pointer stays valid
 * until the next call on the context.  NULL ctx -> text of the last failed
 * ctx_create on this thread. */
const char* prism_hip_last_error(const prism_hip_ctx* ctx);

/* Library version string (static). */
const char* prism_hip_version(void);

/* ---- weights ------------------------------------------------------------ */

/* Replaces the weight upload of MetalBackend::new
 * (src/lut/engine_impl.rs:124-133: one device copy per CompiledTensor).
 * Copies `bytes` of host payload to device memory owned by the library.
 * bytes must equal dim_m*2^bits*2 + dim_m*(bits==4 ? dim_n/2 : dim_n).
 * NULL on failure (reason in prism_hip_last_error(ctx)). */
prism_hip_weight* prism_hip_weight_upload(prism_hip_ctx* ctx, const uint8_t* payload, size_t bytes,
                                          uint32_t dim_m, uint32_t dim_n, uint32_t bits, uint32_t layout);
/* prism_hip_weight_upload without the final wait, for uploading a whole
 * model (MetalBackend::new's loop, engine_impl.rs:124-133) with one wait at
 * the end.  The payload is consumed (copied into the context's pinned
 * staging ring) before the call returns; the device copy completes in order
 * on the context stream, so every later call on this context sees it.  Call
 * prism_hip_ctx_synchronize before using the weight on another stream. */
prism_hip_weight* prism_hip_weight_upload_async(prism_hip_ctx* ctx, const uint8_t* payload, size_t bytes,
                                                uint32_t dim_m, uint32_t dim_n, uint32_t bits, uint32_t layout);
/* Wait for everything enqueued on the context stream (uploads included). */
int prism_hip_ctx_synchronize(prism_hip_ctx* ctx);
/* Same, from a payload already in device memory (copied device-to-device). */
prism_hip_weight* prism_hip_weight_upload_dev(prism_hip_ctx* ctx, const void* d_payload, size_t bytes,
                                              uint32_t dim_m, uint32_t dim_n, uint32_t bits, uint32_t layout);
void prism_hip_weight_free(prism_hip_weight* w); /* accepts NULL */
/* Shape query; any out pointer may be NULL.  Returns 0 or ERR_NULL. */
int prism_hip_weight_info(const prism_hip_weight* w, uint32_t* dim_m, uint32_t* dim_n, uint32_t* bits,
                          size_t* bytes);

/* ---- palettized GEMV (decode) ------------------------------------------- */

/* y[b, r] = f16( sum_k f32(x[b, k]) * f32(LUT_r[idx(r, k)]) ), b < batch.
 * x: [batch x dim_n] fp16 bits, y: [batch x dim_m] fp16 bits, host memory.
 * Replaces MetalBackend::gemv (src/lut/engine_impl.rs:155-190) and
 * lut_gemv_cpu (compute-core/src/lut/evaluator.rs:21-44) for batch 1; a
 * batch of B is B independent GEMVs. Synchronous. */
int prism_hip_gemv(prism_hip_ctx* ctx, const prism_hip_weight* w, const uint16_t* x, uint32_t batch,
                   uint16_t* y);
/* Device-pointer form; asynchronous on `stream` (NULL = context stream). */
int prism_hip_gemv_dev(prism_hip_ctx* ctx, const prism_hip_weight* w, const void* d_x, uint32_t batch,
                       void* d_y, void* stream);

/* ---- fused gate_up + SwiGLU GEMV ---------------------------------------- */

/* y[r] = f16( f32(f16(silu(f32(g16[r])))) * f32(u16[r]) ) with
 * g16 = gemv(x, gate), u16 = gemv(x, up): the CPU path's roundings
 * (compute-core/src/lut/evaluator.rs:78-83,209-225).  Replaces
 * MetalBackend::fused_gate_up (src/lut/engine_impl.rs:443-490) with the
 * split-block layout and out_dim = dim_m.  x: [dim_n], y: [dim_m]. */
int prism_hip_gateup_swiglu(prism_hip_ctx* ctx, const prism_hip_weight* gate, const prism_hip_weight* up,
                            const uint16_t* x, uint16_t* y);
int prism_hip_gateup_swiglu_dev(prism_hip_ctx* ctx, const prism_hip_weight* gate, const prism_hip_weight* up,
                                const void* d_x, void* d_y, void* stream);

/* ---- gate and up GEMVs without activation (two outputs) ---------------- */

/* gate_out[r] = gemv(x, gate)[r], up_out[r] = gemv(x, up)[r] (fp16 bits),
 * in one pass over both matrices: the two raw outputs of
 * templates/fused_gate_up.metal:16-97 (output_gate, output_up; a kernel the
 * reference compiles but never dispatches), with the split-block layout and
 * out_dim = dim_m.  Each output equals prism_hip_gemv of that matrix bit for
 * bit.  For callers that apply an activation other than SiLU (for example
 * gelu_inplace, compute-core/src/lut/evaluator.rs:86-95).  Shapes must
 * match (ERR_MISMATCH).  x: [dim_n]; outputs: [dim_m]. */
int prism_hip_gate_up(prism_hip_ctx* ctx, const prism_hip_weight* gate, const prism_hip_weight* up,
                      const uint16_t* x, uint16_t* gate_out, uint16_t* up_out);
int prism_hip_gate_up_dev(prism_hip_ctx* ctx, const prism_hip_weight* gate, const prism_hip_weight* up,
                          const void* d_x, void* d_gate_out, void* d_up_out, void* stream);

/* ---- palettized GEMM (prefill) ------------------------------------------ */

/* Y[M x dim_m] = X[M x dim_n] . W^T, fp32 accumulation, fp16 out: M
 * independent lut_gemv_cpu rows.  Replaces templates/palettized_gemm.metal
 * (never dispatched by the reference; kernel_provider.rs:233-237).
 * Prefills of 33..256 rows (4-bit; 49..256 for 8-bit) split K: their
 * fp32 partials (up to 4 * M * dim_m * 4 bytes) come from a stream-ordered
 * pool the context creates on first use and frees on the call's stream,
 * so calls on different streams do not share them. */
int prism_hip_gemm(prism_hip_ctx* ctx, const prism_hip_weight* w, const uint16_t* X, uint32_t M, uint16_t* Y);
int prism_hip_gemm_dev(prism_hip_ctx* ctx, const prism_hip_weight* w, const void* d_X, uint32_t M, void* d_Y,
                       void* stream);
/* prism_hip_gemm_dev without any allocation.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code
 * under HIP graph capture, serving loops, harnesses that forbid hipMalloc).
 * Same kernels and results as prism_hip_gemm_dev; the split-K partials live
 * in a static 64 MiB array on each GPU instead of the context's pool, and a
 * call whose partials would exceed it returns PRISM_HIP_ERR_SIZE (none does
 * on a 256-CU MI355X).  All calls on one GPU share that array: calls that
 * overlap on one GPU (other streams, other contexts) race. */
int prism_hip_gemm_dev_noalloc(prism_hip_ctx* ctx, const prism_hip_weight* w, const void* d_X, uint32_t M,
                               void* d_Y, void* stream);

/* ---- LUT decode ---------------------------------------------------------- */

/* lut_embed (compute-core/src/lut/evaluator.rs:176-197): out[0..dim_n) =
 * fp16 bits of row `token` decoded through its LUT; token >= dim_m gives
 * zeros.  Host memory, synchronous. */
int prism_hip_lut_embed(prism_hip_ctx* ctx, const prism_hip_weight* w, uint32_t token, uint16_t* out);
/* Dense decode of rows [row0, row0+nrows) into d_out [nrows x dim_n] fp16
 * (device memory, asynchronous). */
int prism_hip_decode_rows_dev(prism_hip_ctx* ctx, const prism_hip_weight* w, uint32_t row0, uint32_t nrows,
                              void* d_out, void* stream);

/* ---- palette compiler ---------------------------------------------------- */

/* k-means palettization of an fp32 [out_dim x in_dim] row-major matrix into
 * the split-block payload: out_dim x 16 fp16 LUT entries (zero past k),
 * then every row's packed 4-bit indices, (in_dim+1)/2 bytes per row
 * (prism_hip_palettize_bytes in all).  Replaces palettize_matrix
 * (src/quantization/palette.rs:230-272: fit_palette :75-183 with the
 * threshold of :186-191, encode_channel :198-228) plus compile_to_cimage's
 * payload assembly (src/lut/compiler.rs:47-60, called with k=16,
 * max_iter=50); the payload is byte-identical to the reference's.
 * k must be 1..16 (PRISM_HIP_ERR_SHAPE otherwise).  seeds (host memory, may
 * be NULL) are the calibration seeds of compute-core's
 * palettize_matrix_phased (compute-core/src/quantization/palette.rs:
 * 94-116, 409-431): the first min(nseeds, k) centroids of every row, with
 * k-means++ continuing from them; NULL starts every row from channel[n/2]
 * as the root crate does.  Non-NULL seeds need nseeds >= 1 (the reference
 * panics on an empty list); entries past 16 are never used. */
size_t prism_hip_palettize_bytes(uint32_t out_dim, uint32_t in_dim);
int prism_hip_palettize(prism_hip_ctx* ctx, const float* w, uint32_t out_dim, uint32_t in_dim, uint32_t k,
                        uint32_t max_iter, const float* seeds, uint32_t nseeds, uint8_t* payload);
int prism_hip_palettize_dev(prism_hip_ctx* ctx, const void* d_w, uint32_t out_dim, uint32_t in_dim, uint32_t k,
                            uint32_t max_iter, const float* seeds, uint32_t nseeds, void* d_payload,
                            void* stream);

/* ---- keyed backend (MetalBackend's surface) ------------------------------ */

/* A name -> weight map over one context, mirroring MetalBackend
 * (src/lut/engine_impl.rs:31-154): `weight_bufs: HashMap<String,(Buffer,
 * dim_m, dim_n)>`.  Errors are returned as codes; the text (the
 * reference's `Err(String)`, e.g. "miss <key>") is in
 * prism_hip_backend_last_error. */
prism_hip_backend* prism_hip_backend_new(int device);
void prism_hip_backend_free(prism_hip_backend* b); /* accepts NULL */
const char* prism_hip_backend_last_error(const prism_hip_backend* b);
/* Upload one CompiledTensor (src/lut/compiler.rs:14-20) under `key`;
 * replaces an existing entry of the same key. */
int prism_hip_backend_add_tensor(prism_hip_backend* b, const char* key, const uint8_t* payload, size_t bytes,
                                 uint32_t dim_m, uint32_t dim_n, uint32_t bits);
/* MetalBackend::gemv(key, inp, out) (src/lut/engine_impl.rs:155):
 * inp_len must be dim_n (or a multiple of it: a batch), out_len dim_m
 * times the batch. */
int prism_hip_backend_gemv(prism_hip_backend* b, const char* key, const uint16_t* inp, size_t inp_len,
                           uint16_t* out, size_t out_len);
/* MetalBackend::fused_gate_up(gate_key, up_key, input, output)
 * (src/lut/engine_impl.rs:443-449). */
int prism_hip_backend_fused_gate_up(prism_hip_backend* b, const char* gate_key, const char* up_key,
                                    const uint16_t* input, size_t in_len, uint16_t* output, size_t out_len);
/* Prefill GEMM over a keyed tensor. */
int prism_hip_backend_gemm(prism_hip_backend* b, const char* key, const uint16_t* X, uint32_t M, uint16_t* Y);
/* The engine's embed of one token through a keyed tensor
 * (src/lut/engine_impl.rs:1407-1446 via lut_embed). */
int prism_hip_backend_embed(prism_hip_backend* b, const char* key, uint32_t token, uint16_t* out,
                            size_t out_len);
/* Number of registered tensors. */
size_t prism_hip_backend_len(const prism_hip_backend* b);
/* add_tensor uploads asynchronously on the backend's own stream (its other
 * calls are ordered after them); this waits for every upload to finish. */
int prism_hip_backend_synchronize(prism_hip_backend* b);

/* ---- GPU-resident decode step ----------------------------------------------
 * Replaces PrismEngine::step (src/lut/engine_impl.rs:1076-1405) for the
 * Qwen2 graph ModelGraph::build produces (src/lut/graph.rs:304-530), with
 * the engine's INT8 KV cache (KVCache, engine_impl.rs:514-584) resident in
 * HBM.  The engine's per-node CPU/GPU round trips (:160-188) become one HIP
 * graph per token.  Semantics are the reference CPU path's: RMS norms
 * without a norm weight (:1056-1065), RoPE on Q only with base 10000
 * whatever rope_theta says (:1068-1075, :1211-1218), residual adds after
 * o_proj and down_proj, silu(gate)*up, tied LM head = the embedding
 * matrix (:1384-1403).  All projections are 4-bit split-block weights. */
typedef struct prism_hip_model prism_hip_model;

typedef struct prism_hip_model_config {
  uint32_t n_layers;     /* num_hidden_layers                       */
  uint32_t hidden;       /* hidden_size (multiple of 8)             */
  uint32_t n_heads;      /* num_attention_heads                     */
  uint32_t n_kv_heads;   /* num_key_value_heads (divides n_heads)   */
  uint32_t head_dim;     /* 64                                      */
  uint32_t intermediate; /* intermediate_size (multiple of 8)       */
  uint32_t vocab;        /* vocab_size                              */
  uint32_t max_seq;      /* KV capacity in tokens per layer         */
  float rms_eps;         /* rms_norm_eps                            */
  float rope_theta;      /* recorded; the CPU path rotates with 10000 */
} prism_hip_model_config;

/* Allocates the KV cache, activations and the RoPE table (generate()'s
 * KVCache::new, engine_impl.rs:933-953).  NULL on error (context text). */
prism_hip_model* prism_hip_model_create(prism_hip_ctx* ctx, const prism_hip_model_config* cfg);
void prism_hip_model_free(prism_hip_model* m);

/* Weights are copied into the model (QKV fused into one matrix), so the
 * handles may be freed afterwards.  embed: [vocab x hidden] 4-bit, the
 * TokenEmbedding tensor and the tied LM head (engine_impl.rs:1407-1446,
 * :1384-1403).  Layer tensors in ModelGraph order (graph.rs:380-490). */
int prism_hip_model_set_embedding(prism_hip_model* m, const prism_hip_weight* embed);
int prism_hip_model_set_layer(prism_hip_model* m, uint32_t layer, const prism_hip_weight* q_proj,
                              const prism_hip_weight* k_proj, const prism_hip_weight* v_proj,
                              const prism_hip_weight* o_proj, const prism_hip_weight* gate_proj,
                              const prism_hip_weight* up_proj, const prism_hip_weight* down_proj);

/* KVCache::append(layer, k, v) for `ntokens` rows of kv_dim fp16 values
 * each (host memory); every row becomes one INT8 block (engine_impl.rs:532-556). */
int prism_hip_model_kv_append(prism_hip_model* m, uint32_t layer, const uint16_t* k, const uint16_t* v,
                              uint32_t ntokens);
/* Tokens cached in `layer` (KVCache::seq_len, engine_impl.rs:564-566). */
int prism_hip_model_kv_len(const prism_hip_model* m, uint32_t layer, uint32_t* len);
/* The layer's cache in the reference's byte format: len blocks of
 * [scale f32 LE][kv_dim x i8] for K and for V (each len*(kv_dim+4) bytes). */
int prism_hip_model_kv_read(prism_hip_model* m, uint32_t layer, uint8_t* k_blocks, uint8_t* v_blocks);
int prism_hip_model_kv_reset(prism_hip_model* m);
/* Forget every layer's tokens past `len` (a rollback; no device work).  The
 * reference's KVCache only grows; this serves fixed-length benchmarks and
 * callers that discard rejected tokens. */
int prism_hip_model_kv_truncate(prism_hip_model* m, uint32_t len);

/* One decode step: PrismEngine::step(token, pos) -> logits [vocab] fp16.
 * Appends one KV token per layer.  pos < max_seq and every layer's KV
 * length < max_seq.  _step copies the logits to host memory and waits;
 * _step_dev only enqueues on `stream` (NULL: the context stream) and leaves
 * the logits in the model's device buffer (prism_hip_model_logits_dev). */
int prism_hip_model_step(prism_hip_model* m, uint32_t token, int64_t pos, uint16_t* logits);
int prism_hip_model_step_dev(prism_hip_model* m, uint32_t token, int64_t pos, void* stream);
const void* prism_hip_model_logits_dev(const prism_hip_model* m);

/* The read floor.  No counterpart in the reference: a measuring stick for the
 * GEMV kernels above.  Reads each of `bytes` (< 2 GiB) bytes of d_buf once
 * with the fastest single-launch streaming shape found on MI355X and writes
 * (almost surely) nothing to d_sink (>= 1 KB of device memory).  Enqueues on
 * `stream` (NULL: the context stream) and returns. */
int prism_hip_stream_read_dev(prism_hip_ctx* ctx, const void* d_buf, size_t bytes, void* d_sink, void* stream);

/* Two more measuring sticks, no counterpart in the reference either.
 * prism_hip_launch_empty_dev enqueues one launch of an empty one-wave kernel
 * (the cost of a dependent launch, which bounds chains of small kernels such
 * as the decode step).  prism_hip_mfma_probe_dev enqueues `groups` workgroups
 * of four waves, each wave running `iters` rounds of 16
 * v_mfma_f32_32x32x16_f16 on registers (524 288 flop per wave and round);
 * d_sink (>= 1 KB of device memory) is (almost surely) not written.  Both
 * enqueue on `stream` (NULL: the context stream) and return. */
int prism_hip_launch_empty_dev(prism_hip_ctx* ctx, void* stream);
int prism_hip_mfma_probe_dev(prism_hip_ctx* ctx, uint32_t groups, uint32_t iters, void* d_sink, void* stream);

/* Issue-rate probe, no counterpart in the reference: `groups` workgroups of
 * 256 * waves_per_simd threads (1, 2 or 4 waves on each SIMD), each wave
 * running `iters` rounds of 8 independent instructions of kind `op`: 0
 * v_fma_f32, 1 v_dot2_f32_f16, 2 v_perm_b32, 3 v_mfma_f32_4x4x4f16.  d_sink
 * (>= 1 KB of device memory) is (almost surely) not written.  Enqueues on
 * `stream` (NULL: the context stream) and returns. */
int prism_hip_issue_probe_dev(prism_hip_ctx* ctx, uint32_t op, uint32_t groups, uint32_t waves_per_simd,
                              uint32_t iters, void* d_sink, void* stream);

/* The kernels the dispatch launched in the context's most recent compute
 * call (GEMV, gate/up, GEMM, row decode, palettize, read floor), by their
 * device names in launch order, joined by " + ", e.g.
 * "k_gemv_lpr<8, 1, 1, 0, 16>"; a kernel launched n > 1 times in a row
 * appears once followed by " x<n>" ("k_gemv_mfma<4, true> x3").  "" before the
 * first such call.  No counterpart in the reference: measurement and tests
 * read it to label what ran.  The pointer stays valid until the next call
 * on the context. */
const char* prism_hip_last_kernels(prism_hip_ctx* ctx);

#ifdef __cplusplus
}
#endif
#endif /* PRISM_HIP_H */
