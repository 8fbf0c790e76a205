"""The execution plan a .cimage header records, with the MI355X device.

The reference's compile step stores a per-node backend assignment in the
.cimage header (src/lut/compiler.rs:30-34; ExecutionPlan, BackendAssignment
and generate_plan in src/lut/graph.rs:549-640).  This module restates the
node sequence ModelGraph::build emits for a standard-attention decoder
(graph.rs:304-530) and the assignment with a HIP device added: palettized
contractions go to HipGemm, attention to HipAttention, and the norms, RoPE
and activations, which the HIP decode step fuses, to HipFused.  Without a HIP
device the assignment is the reference's (Metal or CPU).  The Rust side of
the same selector is integration/rust/src/lut/plan_hip.rs.
"""
from __future__ import annotations

import json

# ComputeNode variants (graph.rs:52-112) that a plan assigns
CONTRACTIONS = ("PalettizedMatmul", "AttentionOutputGate", "SharedKVProjection", "LanguageModelHead",
                "MultiTokenPredictionHead")
ATTENTION = ("ScaledDotProductAttention", "LinearAttention")
ELEMENTWISE = {"Norm": "CpuNorm", "RotaryEmbedding": "CpuRope", "MRoPE": "CpuRope", "Activation": "CpuActivation"}


def graph_nodes(n_layers: int, tie_word_embeddings: bool = True) -> list[str]:
    """ComputeNode kinds of ModelGraph::build for a standard-attention
    decoder without M-RoPE, shared K/V or multi-token prediction (Qwen2,
    Llama): the embedding, per layer input norm, q/k/v, RoPE, attention, o,
    post-attention norm, gate, up, activation, down; the final norm; an LM
    head node only when the head is not tied to the embedding."""
    layer = ["Norm", "PalettizedMatmul", "PalettizedMatmul", "PalettizedMatmul", "RotaryEmbedding",
             "ScaledDotProductAttention", "PalettizedMatmul", "Norm", "PalettizedMatmul", "PalettizedMatmul",
             "Activation", "PalettizedMatmul"]
    nodes = ["TokenEmbedding"] + layer * n_layers + ["Norm"]
    if not tie_word_embeddings:
        nodes.append("LanguageModelHead")
    return nodes


def device(has_hip: bool, has_metal: bool) -> str:
    """The device the contractions run on: HIP first, then Metal, then CPU."""
    return "hip" if has_hip else "metal" if has_metal else "cpu"


def assign(node: str, dev: str) -> str:
    """BackendAssignment of one node on `dev`."""
    if node == "TokenEmbedding":
        return "Skip"
    if node in CONTRACTIONS:
        return {"hip": "HipGemm", "metal": "MetalGemm", "cpu": "CpuGemm"}[dev]
    if node in ATTENTION:
        return {"hip": "HipAttention", "metal": "MetalAttention", "cpu": "CpuSoftmaxAttn"}[dev]
    if node in ELEMENTWISE:
        return "HipFused" if dev == "hip" else ELEMENTWISE[node]
    raise ValueError(f"unknown node kind {node!r}")


def generate_plan(nodes: list[str], num_layers: int, has_hip: bool, has_metal: bool = False) -> dict:
    """ExecutionPlan (graph.rs:551-561) as serde writes it."""
    dev = device(has_hip, has_metal)
    return {
        "version": 1,
        "architecture": "prism-engine",
        "num_layers": num_layers,
        "node_backends": [assign(n, dev) for n in nodes],
        "kv_cache": "Fp16" if dev == "metal" else "Int8",
        "attention_strategy": {"hip": "HipKernel", "metal": "MetalKernel", "cpu": "CpuSoftmax"}[dev],
        "lm_head_backend": dev,
    }


def plan_json(plan: dict) -> str:
    """serde_json::to_string of the plan: compact, fields in declaration order."""
    return json.dumps(plan, separators=(",", ":"))
