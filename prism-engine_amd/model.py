"""Qwen2-architecture palettized decoder: configuration, the reference's
tensor names, and seeded synthetic weights / KV cache for tests and the
decode-step benchmark.

The configuration mirrors what ModelGraph::build reads from a Hugging Face
config (src/lut/graph.rs:240-285) for the Qwen2 family; tensor names follow
the nodes it emits (graph.rs:304-530): embed_tokens, per layer
self_attn.{q,k,v,o}_proj and mlp.{gate,up,down}_proj, with the LM head tied
to the embedding (tie_word_embeddings).
"""
from __future__ import annotations

import json
from dataclasses import dataclass

import numpy as np

from .palette import PalettizedTensor, synth_tensor

LAYER_ROLES = ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj")


@dataclass(frozen=True)
class Qwen2Config:
    """Decoder shape; defaults are Qwen2.5-0.5B (tests/fixtures/lut_graph/
    qwen2_config.json in the reference)."""
    n_layers: int = 24
    hidden: int = 896
    n_heads: int = 14
    n_kv_heads: int = 2
    head_dim: int = 64
    intermediate: int = 4864
    vocab: int = 151936
    rms_eps: float = 1e-6
    rope_theta: float = 1000000.0

    @classmethod
    def from_hf(cls, d: dict | str) -> "Qwen2Config":
        """From a config.json dict (or its path): the keys graph.rs reads."""
        if isinstance(d, str):
            with open(d) as f:
                d = json.load(f)
        heads = int(d["num_attention_heads"])
        hidden = int(d["hidden_size"])
        return cls(n_layers=int(d["num_hidden_layers"]), hidden=hidden, n_heads=heads,
                   n_kv_heads=int(d.get("num_key_value_heads", heads)),
                   head_dim=int(d.get("head_dim", hidden // heads)),
                   intermediate=int(d["intermediate_size"]), vocab=int(d["vocab_size"]),
                   rms_eps=float(d.get("rms_norm_eps", 1e-6)), rope_theta=float(d.get("rope_theta", 10000.0)))

    @property
    def q_dim(self) -> int:
        return self.n_heads * self.head_dim

    @property
    def kv_dim(self) -> int:
        return self.n_kv_heads * self.head_dim

    def shapes(self) -> dict[str, tuple[int, int]]:
        """[dim_m, dim_n] of each layer tensor, by role."""
        D, I, Q, KV = self.hidden, self.intermediate, self.q_dim, self.kv_dim
        return {"q_proj": (Q, D), "k_proj": (KV, D), "v_proj": (KV, D), "o_proj": (D, Q),
                "gate_proj": (I, D), "up_proj": (I, D), "down_proj": (D, I)}

    def oracle_dims(self, bits: int = 4) -> tuple[int, ...]:
        return (self.n_layers, self.hidden, self.n_heads, self.n_kv_heads, self.head_dim, self.intermediate,
                self.vocab, bits)

    def weight_bytes(self, bits: int = 4) -> int:
        """Palettized bytes read per decode step (every layer tensor + the
        tied embedding / LM head)."""
        t = 2 << bits

        def pb(m, n):
            return m * t + m * n * bits // 8

        per_layer = sum(pb(m, n) for m, n in self.shapes().values())
        return self.n_layers * per_layer + pb(self.vocab, self.hidden)

    def kv_bytes(self, n_tokens: int) -> int:
        """INT8 KV bytes one step reads: K and V blocks (scale + kv_dim) for
        n_tokens tokens in every layer."""
        return self.n_layers * 2 * n_tokens * (self.kv_dim + 4)


def tensor_names(cfg: Qwen2Config, prefix: str = "model") -> dict:
    """The reference's keys: {"embed": ..., "layers": [{role: key}]}."""
    layers = []
    for l in range(cfg.n_layers):
        p = f"{prefix}.layers.{l}"
        layers.append({r: f"{p}.{'self_attn' if r[0] in 'qkvo' else 'mlp'}.{r}.weight" for r in LAYER_ROLES})
    return {"embed": f"{prefix}.embed_tokens.weight", "layers": layers}


def synth_weights(cfg: Qwen2Config, seed: int, bits: int = 4):
    """Random-init palettized weights (per-row LUT: sorted N(0, 0.02) fp16;
    uniform indices): returns (embed, [per-layer tuple in LAYER_ROLES order])."""
    names = tensor_names(cfg)
    shapes = cfg.shapes()
    embed = synth_tensor(cfg.vocab, cfg.hidden, 4, seed, key=names["embed"])
    layers = []
    for l in range(cfg.n_layers):
        ts = []
        for j, r in enumerate(LAYER_ROLES):
            m, n = shapes[r]
            ts.append(synth_tensor(m, n, bits, seed * 1000 + 17 * l + j + 1, key=names["layers"][l][r]))
        layers.append(tuple(ts))
    return embed, layers


def synth_kv(cfg: Qwen2Config, n_tokens: int, seed: int):
    """Per layer (K, V), each [n_tokens x kv_dim] fp16 bits drawn from N(0, 1)."""
    rng = np.random.Generator(np.random.PCG64(seed + 104729))
    out = []
    for _ in range(cfg.n_layers):
        k = rng.standard_normal(size=(n_tokens, cfg.kv_dim)).astype(np.float32).astype(np.float16).view(np.uint16)
        v = rng.standard_normal(size=(n_tokens, cfg.kv_dim)).astype(np.float32).astype(np.float16).view(np.uint16)
        out.append((k, v))
    return out


def payloads(embed: PalettizedTensor, layers) -> tuple:
    """(embed payload, [tuple of 7 payloads]) for the oracle."""
    return embed.payload, [tuple(t.payload for t in lw) for lw in layers]
