// prism-ffi/src/hip.rs -- the extern block of libprism_hip, one declaration
// per function of include/prism_hip.h (tests/test_rust_binding.py checks the
// names, argument types and return types against the header).  Declared in
// prism-ffi/src/lib.rs as `#[cfg(feature = "hip-dispatch")] pub mod hip;`;
// error codes follow prism-ffi's convention (-2: not linked,
// prism-ffi/src/lib.rs:52-56).
#![allow(non_camel_case_types)]
use std::os::raw::{c_char, c_int, c_void};

#[repr(C)] pub struct prism_hip_ctx { _p: [u8; 0] }
#[repr(C)] pub struct prism_hip_weight { _p: [u8; 0] }
#[repr(C)] pub struct prism_hip_backend { _p: [u8; 0] }

pub const PRISM_HIP_OK: c_int = 0;
pub const PRISM_HIP_ERR_NULL: c_int = -1;
pub const PRISM_HIP_ERR_NOT_LINKED: c_int = -2; // prism-ffi/src/lib.rs:52-56
pub const PRISM_HIP_ERR_SHAPE: c_int = -3;
pub const PRISM_HIP_ERR_BITS: c_int = -4;
pub const PRISM_HIP_ERR_SIZE: c_int = -5;
pub const PRISM_HIP_ERR_LAYOUT: c_int = -6;
pub const PRISM_HIP_ERR_DEVICE: c_int = -7;
pub const PRISM_HIP_ERR_MISMATCH: c_int = -8;
pub const PRISM_HIP_ERR_KEY: c_int = -9;
pub const PRISM_HIP_ERR_CONTEXT: c_int = -10;

#[link(name = "prism_hip")]
extern "C" {
    pub fn prism_hip_ctx_create(device: c_int) -> *mut prism_hip_ctx;
    pub fn prism_hip_ctx_destroy(ctx: *mut prism_hip_ctx);
    pub fn prism_hip_last_error(ctx: *const prism_hip_ctx) -> *const c_char;
    pub fn prism_hip_version() -> *const c_char;
    pub fn prism_hip_weight_upload(ctx: *mut prism_hip_ctx, payload: *const u8, bytes: usize,
        dim_m: u32, dim_n: u32, bits: u32, layout: u32) -> *mut prism_hip_weight;
    pub fn prism_hip_weight_upload_async(ctx: *mut prism_hip_ctx, payload: *const u8, bytes: usize,
        dim_m: u32, dim_n: u32, bits: u32, layout: u32) -> *mut prism_hip_weight;
    pub fn prism_hip_ctx_synchronize(ctx: *mut prism_hip_ctx) -> c_int;
    pub fn prism_hip_weight_upload_dev(ctx: *mut prism_hip_ctx, d_payload: *const c_void, bytes: usize,
        dim_m: u32, dim_n: u32, bits: u32, layout: u32) -> *mut prism_hip_weight;
    pub fn prism_hip_weight_free(w: *mut prism_hip_weight);
    pub fn prism_hip_weight_info(w: *const prism_hip_weight, dim_m: *mut u32, dim_n: *mut u32,
        bits: *mut u32, bytes: *mut usize) -> c_int;
    pub fn prism_hip_gemv(ctx: *mut prism_hip_ctx, w: *const prism_hip_weight, x: *const u16,
        batch: u32, y: *mut u16) -> c_int;
    pub fn prism_hip_gemv_dev(ctx: *mut prism_hip_ctx, w: *const prism_hip_weight, d_x: *const c_void,
        batch: u32, d_y: *mut c_void, stream: *mut c_void) -> c_int;
    pub fn prism_hip_gateup_swiglu(ctx: *mut prism_hip_ctx, gate: *const prism_hip_weight,
        up: *const prism_hip_weight, x: *const u16, y: *mut u16) -> c_int;
    pub fn prism_hip_gateup_swiglu_dev(ctx: *mut prism_hip_ctx, gate: *const prism_hip_weight,
        up: *const prism_hip_weight, d_x: *const c_void, d_y: *mut c_void, stream: *mut c_void) -> c_int;
    // fused_gate_up.metal's two raw outputs (no activation), each equal to prism_hip_gemv's
    pub fn prism_hip_gate_up(ctx: *mut prism_hip_ctx, gate: *const prism_hip_weight,
        up: *const prism_hip_weight, x: *const u16, gate_out: *mut u16, up_out: *mut u16) -> c_int;
    pub fn prism_hip_gate_up_dev(ctx: *mut prism_hip_ctx, gate: *const prism_hip_weight,
        up: *const prism_hip_weight, d_x: *const c_void, d_gate: *mut c_void, d_up: *mut c_void,
        stream: *mut c_void) -> c_int;
    pub fn prism_hip_gemm(ctx: *mut prism_hip_ctx, w: *const prism_hip_weight, x: *const u16, m: u32,
        y: *mut u16) -> c_int;
    pub fn prism_hip_gemm_dev(ctx: *mut prism_hip_ctx, w: *const prism_hip_weight, d_x: *const c_void,
        m: u32, d_y: *mut c_void, stream: *mut c_void) -> c_int;
    // No reference counterpart: the GEMM for callers that cannot allocate (static per-GPU scratch)
    pub fn prism_hip_gemm_dev_noalloc(ctx: *mut prism_hip_ctx, w: *const prism_hip_weight,
        d_x: *const c_void, m: u32, d_y: *mut c_void, stream: *mut c_void) -> c_int;
    pub fn prism_hip_lut_embed(ctx: *mut prism_hip_ctx, w: *const prism_hip_weight, token: u32,
        out: *mut u16) -> c_int;
    pub fn prism_hip_decode_rows_dev(ctx: *mut prism_hip_ctx, w: *const prism_hip_weight, row0: u32,
        nrows: u32, d_out: *mut c_void, stream: *mut c_void) -> c_int;

    // Palette compiler (palettize_matrix + compile_to_cimage's payload, compiler.rs:47-60)
    pub fn prism_hip_palettize_bytes(out_dim: u32, in_dim: u32) -> usize;
    pub fn prism_hip_palettize(ctx: *mut prism_hip_ctx, w: *const f32, out_dim: u32, in_dim: u32, k: u32,
        max_iter: u32, seeds: *const f32, nseeds: u32, payload: *mut u8) -> c_int;
    pub fn prism_hip_palettize_dev(ctx: *mut prism_hip_ctx, d_w: *const c_void, out_dim: u32, in_dim: u32,
        k: u32, max_iter: u32, seeds: *const f32, nseeds: u32, d_payload: *mut c_void,
        stream: *mut c_void) -> c_int;
    pub fn prism_hip_backend_new(device: c_int) -> *mut prism_hip_backend;
    pub fn prism_hip_backend_free(b: *mut prism_hip_backend);
    pub fn prism_hip_backend_last_error(b: *const prism_hip_backend) -> *const c_char;
    pub fn prism_hip_backend_add_tensor(b: *mut prism_hip_backend, key: *const c_char, payload: *const u8,
        bytes: usize, dim_m: u32, dim_n: u32, bits: u32) -> c_int;
    pub fn prism_hip_backend_gemv(b: *mut prism_hip_backend, key: *const c_char, inp: *const u16,
        inp_len: usize, out: *mut u16, out_len: usize) -> c_int;
    pub fn prism_hip_backend_fused_gate_up(b: *mut prism_hip_backend, gate_key: *const c_char,
        up_key: *const c_char, input: *const u16, in_len: usize, output: *mut u16, out_len: usize) -> c_int;
    pub fn prism_hip_backend_gemm(b: *mut prism_hip_backend, key: *const c_char, x: *const u16, m: u32,
        y: *mut u16) -> c_int;
    pub fn prism_hip_backend_embed(b: *mut prism_hip_backend, key: *const c_char, token: u32,
        out: *mut u16, out_len: usize) -> c_int;
    pub fn prism_hip_backend_len(b: *const prism_hip_backend) -> usize;
    pub fn prism_hip_backend_synchronize(b: *mut prism_hip_backend) -> c_int;

    // GPU-resident decode step (PrismEngine::step, engine_impl.rs:1076-1405)
    pub fn prism_hip_model_create(ctx: *mut prism_hip_ctx, cfg: *const prism_hip_model_config)
        -> *mut prism_hip_model;
    pub fn prism_hip_model_free(m: *mut prism_hip_model);
    pub fn prism_hip_model_set_embedding(m: *mut prism_hip_model, embed: *const prism_hip_weight) -> c_int;
    pub fn prism_hip_model_set_layer(m: *mut prism_hip_model, layer: u32, q: *const prism_hip_weight,
        k: *const prism_hip_weight, v: *const prism_hip_weight, o: *const prism_hip_weight,
        gate: *const prism_hip_weight, up: *const prism_hip_weight, down: *const prism_hip_weight) -> c_int;
    pub fn prism_hip_model_kv_append(m: *mut prism_hip_model, layer: u32, k: *const u16, v: *const u16,
        ntokens: u32) -> c_int;
    pub fn prism_hip_model_kv_len(m: *const prism_hip_model, layer: u32, len: *mut u32) -> c_int;
    pub fn prism_hip_model_kv_read(m: *mut prism_hip_model, layer: u32, k_blocks: *mut u8,
        v_blocks: *mut u8) -> c_int;
    pub fn prism_hip_model_kv_reset(m: *mut prism_hip_model) -> c_int;
    pub fn prism_hip_model_kv_truncate(m: *mut prism_hip_model, len: u32) -> c_int;
    pub fn prism_hip_model_step(m: *mut prism_hip_model, token: u32, pos: i64, logits: *mut u16) -> c_int;
    pub fn prism_hip_model_step_dev(m: *mut prism_hip_model, token: u32, pos: i64, stream: *mut c_void)
        -> c_int;
    pub fn prism_hip_model_logits_dev(m: *const prism_hip_model) -> *const c_void;

    // No reference counterpart: the read floor the GEMVs are measured against
    pub fn prism_hip_stream_read_dev(ctx: *mut prism_hip_ctx, d_buf: *const c_void, bytes: usize,
        d_sink: *mut c_void, stream: *mut c_void) -> c_int;
    // No reference counterpart: one dependent launch, the matrix cores' rate
    pub fn prism_hip_launch_empty_dev(ctx: *mut prism_hip_ctx, stream: *mut c_void) -> c_int;
    pub fn prism_hip_mfma_probe_dev(ctx: *mut prism_hip_ctx, groups: u32, iters: u32, d_sink: *mut c_void,
        stream: *mut c_void) -> c_int;
    // No reference counterpart: one instruction kind's issue rate
    pub fn prism_hip_issue_probe_dev(ctx: *mut prism_hip_ctx, op: u32, groups: u32, waves_per_simd: u32,
        iters: u32, d_sink: *mut c_void, stream: *mut c_void) -> c_int;
    // No reference counterpart: the kernels the last compute call launched
    pub fn prism_hip_last_kernels(ctx: *mut prism_hip_ctx) -> *const c_char;
}

#[repr(C)] pub struct prism_hip_model { _p: [u8; 0] }
#[repr(C)]
pub struct prism_hip_model_config {
    pub n_layers: u32, pub hidden: u32, pub n_heads: u32, pub n_kv_heads: u32, pub head_dim: u32,
    pub intermediate: u32, pub vocab: u32, pub max_seq: u32, pub rms_eps: f32, pub rope_theta: f32,
}
