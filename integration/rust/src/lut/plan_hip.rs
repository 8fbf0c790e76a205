// src/lut/plan_hip.rs -- the plan-level selector with an MI355X device: which
// backend runs each node of a ModelGraph when libprism_hip is linked.
// Wiring: `pub mod plan_hip;` in src/lut/mod.rs; in src/lut/graph.rs add the
// three variants below to `BackendAssignment` (:566-576) and `HipKernel` to
// `AttentionBackend` (:587-590), and let `generate_plan` (:592-640) delegate:
//
//     pub fn generate_plan(graph: &ModelGraph, has_metal: bool, has_ane: bool) -> ExecutionPlan {
//         crate::lut::plan_hip::plan_for(graph, PlanDevice::pick(crate::lut::plan_hip::has_hip(), has_metal), has_ane)
//     }
//
// compile_to_cimage (src/lut/compiler.rs:30) then records "HipGemm" etc. in
// the .cimage header when it runs on an MI355X host.  Variants to add:
//
//     HipGemm,      // palettized GEMV / gate_up / GEMM on the GPU (prism_hip_gemv, _gateup_swiglu, _gemm)
//     HipAttention, // decode attention on the GPU, INT8 KV blocks (prism_hip_model_step)
//     HipFused,     // norm, RoPE or activation fused into the GPU decode step
//
// Written for a maintainer: no Rust toolchain was available to compile it.
use crate::lut::graph::{AttentionBackend, BackendAssignment, ComputeNode, ExecutionPlan, KVCacheConfig, ModelGraph};

/// The device a plan puts the palettized contractions on.
#[derive(Clone, Copy, Debug, PartialEq, Eq)]
pub enum PlanDevice {
    Hip,
    Metal,
    Cpu,
}

impl PlanDevice {
    /// HIP when libprism_hip found a gfx950 device, else Metal, else the CPU.
    pub fn pick(has_hip: bool, has_metal: bool) -> Self {
        if has_hip {
            PlanDevice::Hip
        } else if has_metal {
            PlanDevice::Metal
        } else {
            PlanDevice::Cpu
        }
    }

    fn contraction(self) -> BackendAssignment {
        match self {
            PlanDevice::Hip => BackendAssignment::HipGemm,
            PlanDevice::Metal => BackendAssignment::MetalGemm,
            PlanDevice::Cpu => BackendAssignment::CpuGemm,
        }
    }

    fn attention(self) -> BackendAssignment {
        match self {
            PlanDevice::Hip => BackendAssignment::HipAttention,
            PlanDevice::Metal => BackendAssignment::MetalAttention,
            PlanDevice::Cpu => BackendAssignment::CpuSoftmaxAttn,
        }
    }

    /// Norm, RoPE and activation nodes: inside the GPU decode step on HIP,
    /// on the CPU otherwise (the Metal engine runs them on the CPU too).
    fn elementwise(self, cpu: BackendAssignment) -> BackendAssignment {
        if self == PlanDevice::Hip { BackendAssignment::HipFused } else { cpu }
    }
}

/// The execution plan of `graph` with the contractions on `dev`.
pub fn plan_for(graph: &ModelGraph, dev: PlanDevice, _has_ane: bool) -> ExecutionPlan {
    let node_backends = graph
        .nodes
        .iter()
        .map(|node| match node {
            ComputeNode::TokenEmbedding { .. } => BackendAssignment::Skip,
            ComputeNode::Norm { .. } => dev.elementwise(BackendAssignment::CpuNorm),
            ComputeNode::RotaryEmbedding { .. } | ComputeNode::MRoPE { .. } => {
                dev.elementwise(BackendAssignment::CpuRope)
            }
            ComputeNode::Activation { .. } => dev.elementwise(BackendAssignment::CpuActivation),
            ComputeNode::ScaledDotProductAttention { .. } | ComputeNode::LinearAttention { .. } => dev.attention(),
            ComputeNode::PalettizedMatmul { .. }
            | ComputeNode::AttentionOutputGate { .. }
            | ComputeNode::SharedKVProjection { .. }
            | ComputeNode::LanguageModelHead { .. }
            | ComputeNode::MultiTokenPredictionHead { .. } => dev.contraction(),
        })
        .collect();
    ExecutionPlan {
        version: 1,
        architecture: "prism-engine".into(),
        num_layers: graph.num_layers,
        node_backends,
        // the HIP decode step keeps the CPU path's INT8 blocks (KVCache::append)
        kv_cache: if dev == PlanDevice::Metal { KVCacheConfig::Fp16 } else { KVCacheConfig::Int8 },
        attention_strategy: match dev {
            PlanDevice::Hip => AttentionBackend::HipKernel,
            PlanDevice::Metal => AttentionBackend::MetalKernel,
            PlanDevice::Cpu => AttentionBackend::CpuSoftmax,
        },
        lm_head_backend: match dev {
            PlanDevice::Hip => "hip",
            PlanDevice::Metal => "metal",
            PlanDevice::Cpu => "cpu",
        }
        .into(),
    }
}

/// True when libprism_hip is linked and finds a gfx950 device.
pub fn has_hip() -> bool {
    #[cfg(feature = "hip-dispatch")]
    {
        let ctx = unsafe { prism_ffi::hip::prism_hip_ctx_create(0) };
        if ctx.is_null() {
            return false;
        }
        unsafe { prism_ffi::hip::prism_hip_ctx_destroy(ctx) };
        true
    }
    #[cfg(not(feature = "hip-dispatch"))]
    {
        false
    }
}
