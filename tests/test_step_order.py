"""How far an equally valid fp32 summation order moves the decode step.

The reference sums every GEMV row, RMS norm and softmax sequentially in
fp32 and rounds each vector to fp16 (compute-core/src/lut/evaluator.rs:21-64,
104-146).  Any other order is as faithful to that arithmetic, and the GPU
necessarily uses another (wave reductions).  The oracle's fold mode 1
(oracle/prism_cpuref.c) re-runs the same step with every long sum cut into
64-term blocks added as a tree.  Measured on the Qwen2.5-0.5B step (seed
1003, 512 cached tokens), mode 1 against mode 0: 5.1e-4 (1 layer), 9.3e-4
(2), 1.2e-3 (4), 2.0e-3 (8), 3.1e-3 (16), 4.6e-3 (24): the last-ulp
differences of each layer travel the residual stream and grow smoothly
with depth.  The GPU's 24-layer logits sit inside that spread
(tests/test_gpu_step.py::test_step_depth_sweep); a 2e-3 bound on them would
also reject a second, correct CPU implementation.
"""
import importlib

import numpy as np
import pytest

import oracle

pe = importlib.import_module("prism-engine_amd")


def _rel(a, b):
    a = a.view(np.float16).astype(np.float64)
    b = b.view(np.float16).astype(np.float64)
    return float(np.max(np.abs(a - b)) / np.max(np.abs(b)))


def test_fold_mode_is_a_real_perturbation_within_gemv_tolerance():
    """One GEMV: the blocked fold changes some outputs' last bits and stays
    within the per-vector bound; mode 0 stays the reference's bytes."""
    t = pe.synth_tensor(512, 4096, 4, seed=5)
    x = pe.synth_x(1, 4096, seed=6)
    ref = oracle.gemv(x, t.payload, 512, 4096, 4)
    lib = oracle.lib()
    lib.cpuref_set_fold_mode(1)
    try:
        alt = oracle.gemv(x, t.payload, 512, 4096, 4)
    finally:
        lib.cpuref_set_fold_mode(0)
    assert np.array_equal(oracle.gemv(x, t.payload, 512, 4096, 4), ref)
    assert not np.array_equal(alt, ref)
    assert _rel(alt, ref) <= 2e-3


def step_drift(cfg, depths, seed=1003, n_cached=512, token=42):
    """Logits of the sequential and the blocked oracle for the first L
    layers of the same weights and cache, for each L in depths."""
    embed, layers = pe.synth_weights(cfg, seed)
    emb_p, lay_p = pe.model.payloads(embed, layers)
    kvs = pe.synth_kv(cfg, n_cached, seed)
    out = {}
    for L in depths:
        dims = (L,) + tuple(cfg.oracle_dims()[1:])
        res = []
        for fold in (0, 1):
            kv = oracle.KVState(L, cfg.kv_dim, n_cached + 1)
            for l in range(L):
                k, v = kvs[l]
                for t in range(n_cached):
                    kv.append(l, k[t], v[t])
            res.append(oracle.decode_step(dims, cfg.rms_eps, emb_p, lay_p[:L], kv, token, n_cached, threads=8,
                                          fold=fold))
        out[L] = (res[0], _rel(res[1], res[0]))
    return out


def test_decode_step_order_drift_grows_with_depth():
    cfg = pe.Qwen2Config()
    d = step_drift(cfg, (1, 4, 24))
    e1, e4, e24 = d[1][1], d[4][1], d[24][1]
    print(f"oracle order drift: 1 layer {e1:.3e}, 4 layers {e4:.3e}, 24 layers {e24:.3e}")
    assert e1 <= 2e-3          # one layer: within the per-vector GEMV bound
    assert e1 < e4 < e24       # grows with depth
    assert 2e-3 < e24 < 1e-2   # 24 layers: past 2e-3 with nothing but the order changed


def test_fold_mode_refuses_sums_past_its_block_capacity():
    """Mode 1 keeps at most 2048 block sums (131072 terms).  A decode step
    whose attention runs over more positions than that would need more: the
    oracle raises instead of dropping the terms past the limit, and mode 0
    (the reference's fold) has no such limit."""
    cfg = pe.Qwen2Config(n_layers=1, hidden=64, n_heads=1, n_kv_heads=1, head_dim=64, intermediate=64,
                         vocab=32)
    embed, layers = pe.synth_weights(cfg, 3)
    emb_p, lay_p = pe.model.payloads(embed, layers)
    n = 2048 * 64 + 1  # softmax and value sums over n + 1 positions
    kv = oracle.KVState(1, cfg.kv_dim, n + 1)
    blk = oracle.kv_quant(np.zeros(cfg.kv_dim, np.uint16))
    ts = cfg.kv_dim + 4
    kv.k[0][:n * ts] = np.tile(blk, n)
    kv.v[0][:n * ts] = np.tile(blk, n)
    kv.len[0] = n
    with pytest.raises(ValueError, match="131072"):
        oracle.decode_step(cfg.oracle_dims(), cfg.rms_eps, emb_p, lay_p, kv.copy(), 1, n, fold=1)
    oracle.decode_step(cfg.oracle_dims(), cfg.rms_eps, emb_p, lay_p, kv, 1, n, fold=0)
