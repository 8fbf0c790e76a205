// src/backend/hip.rs -- HipBackend: MetalBackend's keyed GEMV surface
// (src/lut/engine_impl.rs:51-190,443-490) over libprism_hip.  Wiring:
// `#[cfg(feature = "hip-dispatch")] pub mod hip;` in src/backend/mod.rs, and
// `pub mod backend;` in src/lib.rs (src/lib.rs:1-13 does not declare the
// backend directory today); the engine crate's `hip-dispatch` feature enables
// prism-ffi's (`hip-dispatch = ["dep:prism-ffi", "prism-ffi/hip-dispatch"]`).
// Written for a maintainer: no Rust toolchain was available to compile it.
use std::collections::HashMap;
use std::ffi::{CStr, CString};

use prism_ffi::hip::*;

use crate::lut::compiler::CompiledTensor;

pub struct HipBackend { raw: *mut prism_hip_backend }
unsafe impl Send for HipBackend {} // engine is driven from one thread at a time (prism-bridge/src/lib.rs:548-551)

impl HipBackend {
    pub fn new(tensors: &HashMap<String, CompiledTensor>, _mh: u64, _mi: u64,
               _num_layers: u32, _kv_stride: u64) -> Result<Self, String> {
        let raw = unsafe { prism_hip_backend_new(0) };
        if raw.is_null() { return Err(last(std::ptr::null())); }
        let b = HipBackend { raw };
        for (k, ct) in tensors {
            let key = CString::new(k.as_str()).unwrap();
            let rc = unsafe { prism_hip_backend_add_tensor(raw, key.as_ptr(), ct.payload.as_ptr(),
                ct.payload.len(), ct.dim_m, ct.dim_n, 4) };
            if rc != PRISM_HIP_OK { return Err(last(raw)); }
        }
        // add_tensor only enqueues each copy (pinned staging ring); wait once for all of them
        if unsafe { prism_hip_backend_synchronize(raw) } != PRISM_HIP_OK { return Err(last(raw)); }
        Ok(b)
    }
    pub fn gemv(&self, key: &str, inp: &[u16], out: &mut [u16]) -> Result<(), String> {
        let k = CString::new(key).unwrap();
        let rc = unsafe { prism_hip_backend_gemv(self.raw, k.as_ptr(), inp.as_ptr(), inp.len(),
            out.as_mut_ptr(), out.len()) };
        if rc == PRISM_HIP_OK { Ok(()) } else { Err(last(self.raw)) } // "miss <key>" etc.
    }
    pub fn fused_gate_up(&self, gate_key: &str, up_key: &str, input: &[u16],
                         output: &mut [u16]) -> Result<(), String> {
        let (g, u) = (CString::new(gate_key).unwrap(), CString::new(up_key).unwrap());
        let rc = unsafe { prism_hip_backend_fused_gate_up(self.raw, g.as_ptr(), u.as_ptr(),
            input.as_ptr(), input.len(), output.as_mut_ptr(), output.len()) };
        if rc == PRISM_HIP_OK { Ok(()) } else { Err(last(self.raw)) }
    }
}
impl Drop for HipBackend { fn drop(&mut self) { unsafe { prism_hip_backend_free(self.raw) } } }

fn last(b: *const prism_hip_backend) -> String {
    unsafe { CStr::from_ptr(prism_hip_backend_last_error(b)).to_string_lossy().into_owned() }
}
