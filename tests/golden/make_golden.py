#!/usr/bin/env python3
"""Writes the small golden fixtures under tests/golden/ (inputs + expected
outputs, .npz without pickles).

Expected outputs come from the CPU oracle (oracle/, the C restatement of
lut_gemv_cpu, compute-core/src/lut/evaluator.rs:21-44) and are cross-checked
here against an independent numpy restatement (numpy unpack + sequential
float32 cumsum) before anything is written; the reference's own known
answers (evaluator.rs:231-246, :267-284, :286-298; palette.rs:410-425) are
checked by tests/test_oracle_pinning.py.

Usage: python tests/golden/make_golden.py
"""
import importlib
import os
import zlib
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

pe = importlib.import_module("prism-engine_amd")
oracle = importlib.import_module("oracle")


def numpy_gemv(x, payload, dm, dn, bits):
    w = pe.dequantize(payload, dm, dn, bits)
    keff = (dn // 8) * 8 if bits == 4 else dn
    xf = np.asarray(x).view(np.float16).astype(np.float32)
    prods = (w[:, :keff] * xf[None, :keff]).astype(np.float32)
    return np.cumsum(prods, axis=1, dtype=np.float32)[:, -1].astype(np.float16).view(np.uint16)


CASES = [
    # name, bits, N, K, batch
    ("gemv4_64x128", 4, 64, 128, 1),
    ("gemv4_ragged_13x40", 4, 13, 40, 1),
    ("gemv8_32x64_b3", 8, 32, 64, 3),
]


def main():
    for name, bits, N, K, B in CASES:
        t = pe.synth_tensor(N, K, bits, seed=zlib.crc32(name.encode()) % 10007)
        x = pe.synth_x(B, K, seed=N + K)
        y = oracle.gemv(x, t.payload, N, K, bits)
        for b in range(B):
            assert np.array_equal(y[b], numpy_gemv(x[b], t.payload, N, K, bits)), name
        np.savez(os.path.join(HERE, f"{name}.npz"), payload=t.payload, x=x, y=y,
                 shape=np.array([bits, N, K, B], dtype=np.int64))
    # gate_up + SwiGLU
    N, K = 48, 96
    g = pe.synth_tensor(N, K, 4, seed=31)
    u = pe.synth_tensor(N, K, 4, seed=32)
    x = pe.synth_x(1, K, seed=33)
    y = oracle.gateup_swiglu(x[0], g.payload, u.payload, N, K, 4)
    gg = numpy_gemv(x[0], g.payload, N, K, 4).view(np.float16).astype(np.float32)
    uu = numpy_gemv(x[0], u.payload, N, K, 4).view(np.float16).astype(np.float32)
    s = (gg / (np.float32(1) + np.exp(-gg))).astype(np.float16).astype(np.float32)
    ref = (s * uu).astype(np.float16).view(np.uint16)
    assert pe.rel_err(y, ref) <= 2e-3
    np.savez(os.path.join(HERE, "gateup4_48x96.npz"), gate=g.payload, up=u.payload, x=x, y=y,
             shape=np.array([4, N, K, 1], dtype=np.int64))
    # GEMM (M rows)
    M, N, K = 5, 40, 64
    t = pe.synth_tensor(N, K, 4, seed=41)
    X = pe.synth_x(M, K, seed=42)
    Y = oracle.gemm(X, t.payload, N, K, 4)
    for m in range(M):
        assert np.array_equal(Y[m], numpy_gemv(X[m], t.payload, N, K, 4))
    np.savez(os.path.join(HERE, "gemm4_5x40x64.npz"), payload=t.payload, x=X, y=Y,
             shape=np.array([4, N, K, M], dtype=np.int64))
    print("golden fixtures written")


if __name__ == "__main__":
    main()
