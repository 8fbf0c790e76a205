"""Committed golden fixtures (tests/golden/*.npz, written by
tests/golden/make_golden.py): the oracle must reproduce them bit for bit
(CPU), and the HIP path must meet the parity bar on them (GPU)."""
import glob
import os

import numpy as np
import pytest

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
GEMV = sorted(glob.glob(os.path.join(HERE, "gemv*.npz")))


def _load(path):
    return np.load(path, allow_pickle=False)


def test_fixtures_present():
    assert len(GEMV) >= 3
    assert os.path.exists(os.path.join(HERE, "gateup4_48x96.npz"))
    assert os.path.exists(os.path.join(HERE, "gemm4_5x40x64.npz"))


@pytest.mark.parametrize("path", GEMV, ids=os.path.basename)
def test_oracle_reproduces_gemv_fixture(oracle, path):
    d = _load(path)
    bits, N, K, B = (int(v) for v in d["shape"])
    assert np.array_equal(oracle.gemv(d["x"], d["payload"], N, K, bits), d["y"])


def test_oracle_reproduces_gateup_and_gemm(oracle):
    d = _load(os.path.join(HERE, "gateup4_48x96.npz"))
    bits, N, K, _ = (int(v) for v in d["shape"])
    assert np.array_equal(oracle.gateup_swiglu(d["x"][0], d["gate"], d["up"], N, K, bits), d["y"])
    d = _load(os.path.join(HERE, "gemm4_5x40x64.npz"))
    bits, N, K, M = (int(v) for v in d["shape"])
    assert np.array_equal(oracle.gemm(d["x"], d["payload"], N, K, bits), d["y"])


@pytest.mark.gpu
@pytest.mark.parametrize("path", GEMV, ids=os.path.basename)
def test_gpu_gemv_fixture(pe, gpu_ctx, path):
    d = _load(path)
    bits, N, K, B = (int(v) for v in d["shape"])
    w = gpu_ctx.upload(d["payload"], N, K, bits)
    y = gpu_ctx.gemv(w, d["x"])
    for b in range(B):
        assert pe.rel_err(y[b], d["y"][b]) <= 2e-3
    w.free()


@pytest.mark.gpu
def test_gpu_gateup_and_gemm_fixtures(pe, gpu_ctx):
    d = _load(os.path.join(HERE, "gateup4_48x96.npz"))
    bits, N, K, _ = (int(v) for v in d["shape"])
    g, u = gpu_ctx.upload(d["gate"], N, K, bits), gpu_ctx.upload(d["up"], N, K, bits)
    assert pe.rel_err(gpu_ctx.gateup_swiglu(g, u, d["x"]), d["y"]) <= 2e-3
    d = _load(os.path.join(HERE, "gemm4_5x40x64.npz"))
    bits, N, K, M = (int(v) for v in d["shape"])
    w = gpu_ctx.upload(d["payload"], N, K, bits)
    Y = gpu_ctx.gemm(w, d["x"])
    for m in range(M):
        assert pe.rel_err(Y[m], d["y"][m]) <= 2e-3
