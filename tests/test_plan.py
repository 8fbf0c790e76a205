"""The execution plan with the MI355X device (prism-engine_amd/plan.py and
integration/rust/src/lut/plan_hip.rs) against the reference's ModelGraph
facts and its own generate_plan (src/lut/graph.rs:549-640).

No Rust toolchain is available, so the Rust selector is parsed: every arm of
its match over ComputeNode, per device, must give the assignment the Python
mirror gives.  The Qwen2.5-0.5B graph has 1 + 24 x 12 + 1 nodes and 168
palettized tensors (graph.rs test_qwen2_graph)."""
import importlib
import json
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
RUST = os.path.join(ROOT, "integration", "rust", "src", "lut", "plan_hip.rs")
plan = importlib.import_module("prism-engine_amd.plan")
pe = importlib.import_module("prism-engine_amd")

# ComputeNode variants (graph.rs:52-112)
NODES = ("TokenEmbedding", "Norm", "PalettizedMatmul", "RotaryEmbedding", "ScaledDotProductAttention",
         "LinearAttention", "AttentionOutputGate", "MRoPE", "SharedKVProjection", "MultiTokenPredictionHead",
         "Activation", "LanguageModelHead")
# what the reference's generate_plan assigns with and without Metal (graph.rs:596-633)
REF_METAL = {"TokenEmbedding": "Skip", "Norm": "CpuNorm", "PalettizedMatmul": "MetalGemm",
             "RotaryEmbedding": "CpuRope", "MRoPE": "CpuRope", "ScaledDotProductAttention": "MetalAttention",
             "LinearAttention": "MetalAttention", "AttentionOutputGate": "MetalGemm",
             "SharedKVProjection": "MetalGemm", "Activation": "CpuActivation", "LanguageModelHead": "MetalGemm",
             "MultiTokenPredictionHead": "MetalGemm"}
REF_CPU = {k: v.replace("MetalGemm", "CpuGemm").replace("MetalAttention", "CpuSoftmaxAttn")
           for k, v in REF_METAL.items()}


def test_qwen2_graph_node_counts():
    cfg = pe.Qwen2Config()
    nodes = plan.graph_nodes(cfg.n_layers)
    assert len(nodes) == 1 + 24 * 12 + 1
    assert sum(n == "PalettizedMatmul" for n in nodes) == 168
    assert len(plan.graph_nodes(2, tie_word_embeddings=False)) == 1 + 2 * 12 + 2


@pytest.mark.parametrize("has_metal,ref", [(True, REF_METAL), (False, REF_CPU)])
def test_without_hip_the_plan_is_the_references(has_metal, ref):
    p = plan.generate_plan(list(NODES), 24, has_hip=False, has_metal=has_metal)
    assert dict(zip(NODES, p["node_backends"])) == ref
    assert p["kv_cache"] == ("Fp16" if has_metal else "Int8")
    assert p["attention_strategy"] == ("MetalKernel" if has_metal else "CpuSoftmax")
    assert p["lm_head_backend"] == ("metal" if has_metal else "cpu")


def test_hip_takes_the_contractions_and_the_fused_step():
    cfg = pe.Qwen2Config()
    nodes = plan.graph_nodes(cfg.n_layers)
    for has_metal in (False, True):
        p = plan.generate_plan(nodes, cfg.n_layers, has_hip=True, has_metal=has_metal)
        got = dict(zip(nodes, p["node_backends"]))
        assert got == {"TokenEmbedding": "Skip", "Norm": "HipFused", "PalettizedMatmul": "HipGemm",
                       "RotaryEmbedding": "HipFused", "ScaledDotProductAttention": "HipAttention",
                       "Activation": "HipFused"}
        assert (p["kv_cache"], p["attention_strategy"], p["lm_head_backend"]) == ("Int8", "HipKernel", "hip")
    assert list(json.loads(plan.plan_json(p))) == ["version", "architecture", "num_layers", "node_backends",
                                                   "kv_cache", "attention_strategy", "lm_head_backend"]


def _rust_arms():
    """node kind -> {device: assignment} from plan_hip.rs's match arms."""
    src = open(RUST).read()
    body = src[src.index("pub fn plan_for"):]
    body = body[:body.index(".collect()")]
    helpers = {
        "dev.contraction()": {"hip": "HipGemm", "metal": "MetalGemm", "cpu": "CpuGemm"},
        "dev.attention()": {"hip": "HipAttention", "metal": "MetalAttention", "cpu": "CpuSoftmaxAttn"},
    }
    # check the helpers' own match arms
    for fn, want in (("fn contraction", helpers["dev.contraction()"]), ("fn attention", helpers["dev.attention()"])):
        seg = src[src.index(fn):]
        seg = seg[:seg.index("\n    }\n")]
        arms = dict(re.findall(r"PlanDevice::(\w+) => BackendAssignment::(\w+)", seg))
        assert {k.lower(): v for k, v in arms.items()} == want, fn
    out = {}
    body = " ".join(body[body.index("match node {") + len("match node {"):].split())
    pats = list(re.finditer(r"((?:\|?\s*ComputeNode::\w+ \{ \.\. \}\s*)+)=>", body))
    for i, m in enumerate(pats):
        kinds = re.findall(r"ComputeNode::(\w+)", m.group(1))
        end = pats[i + 1].start() if i + 1 < len(pats) else len(body)
        rhs = body[m.end():end].strip().rstrip(",").strip()
        if rhs.startswith("{"):
            rhs = rhs[1:rhs.rindex("}")].strip()
        rhs = re.match(r"dev\.\w+\((?:BackendAssignment::\w+)?\)|BackendAssignment::\w+", rhs).group(0)
        if rhs == "BackendAssignment::Skip":
            res = {d: "Skip" for d in ("hip", "metal", "cpu")}
        elif rhs in helpers:
            res = helpers[rhs]
        else:
            em = re.fullmatch(r"dev\.elementwise\(BackendAssignment::(\w+)\)", rhs)
            assert em, rhs
            res = {"hip": "HipFused", "metal": em.group(1), "cpu": em.group(1)}
        for k in kinds:
            assert k not in out, k
            out[k] = res
    return out


def test_rust_selector_matches_the_python_mirror():
    arms = _rust_arms()
    assert set(arms) == set(NODES), sorted(set(NODES) ^ set(arms))
    for node in NODES:
        for dev, (has_hip, has_metal) in (("hip", (True, False)), ("metal", (False, True)), ("cpu", (False, False))):
            assert plan.device(has_hip, has_metal) == dev
            assert arms[node][dev] == plan.assign(node, dev), (node, dev)


def test_plan_rides_in_the_cimage_header(tmp_path):
    import numpy as np
    cfg = pe.Qwen2Config(n_layers=2)
    p = plan.generate_plan(plan.graph_nodes(cfg.n_layers), cfg.n_layers, has_hip=True)
    path = str(tmp_path / "m.cimage")
    w = pe.CImageWriter(path)
    w.set_execution_plan(plan.plan_json(p))
    w.append_palettized("t", np.zeros(64 * 32 + 64 * 64, np.uint8), 64, 128, 4)
    w.finalize()
    r = pe.CImageReader(path)
    assert json.loads(r.execution_plan) == p
    r.close()
