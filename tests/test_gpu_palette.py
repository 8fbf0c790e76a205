"""Palette compiler on the GPU (prism_hip_palettize*) against the CPU oracle.

Bar: the payload (fp16 LUT block, then packed 4-bit indices) is
byte-identical to oracle.palettize_payload, the restatement of
palettize_matrix + compile_to_cimage's payload assembly
(src/quantization/palette.rs:230-272, src/lut/compiler.rs:47-60), whose
pinning is in test_palette_oracle.py.  At full model sizes, where the
oracle is slow, the compile -> decode round trip of rows drawn from at most
16 values must be exact.
"""
import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu


def decode(payload, rows, cols, pe):
    rb = (cols + 1) // 2
    lut = payload[:rows * 32].view(np.float16).reshape(rows, 16).astype(np.float32)
    idx = pe.palette.unpack_nibbles(payload[rows * 32:].reshape(rows, rb), cols)
    return np.take_along_axis(lut, idx.astype(np.int64), axis=1)


def weights(kind, rows, cols, seed):
    rng = np.random.default_rng(seed)
    if kind == "normal":  # trained-weight scale
        return (rng.standard_normal((rows, cols)) * 0.02).astype(np.float32)
    if kind == "unit":  # wider spread: more Lloyd iterations
        return rng.standard_normal((rows, cols)).astype(np.float32)
    if kind == "sin":  # the reference's 64x128 test data, extended
        i = np.arange(rows * cols, dtype=np.float32)
        return np.sin(i / np.float32(rows * cols) * np.float32(10.0) - np.float32(5.0)).astype(
            np.float32).reshape(rows, cols)
    if kind == "int":  # many exact ties in distances and sums
        return rng.integers(-40, 41, (rows, cols)).astype(np.float32)
    if kind == "few":  # at most 5 distinct values per row, one constant row
        vals = rng.standard_normal((rows, 5)).astype(np.float32)
        w = np.take_along_axis(vals, rng.integers(0, 5, (rows, cols)), axis=1)
        w[0] = 0.75
        return w
    if kind == "heavy":  # outliers far from the bulk
        w = (rng.standard_normal((rows, cols)) * 0.02).astype(np.float32)
        w[:, ::37] *= 50
        return w
    raise ValueError(kind)


CASES = [
    # kind, rows, cols, k, max_iter
    ("normal", 64, 896, 16, 50),     # Qwen2.5-0.5B hidden width, the compiler's k / max_iter
    ("normal", 16, 4864, 16, 50),    # down_proj width
    ("unit", 48, 512, 16, 50),
    ("sin", 64, 128, 16, 30),        # palette.rs:461-492
    ("int", 40, 333, 16, 50),        # odd width: (n+1)/2 index bytes
    ("few", 12, 200, 16, 50),
    ("heavy", 24, 1000, 16, 50),
    ("normal", 30, 7, 16, 50),       # k > n: k = n
    ("normal", 5, 1, 16, 50),
    ("unit", 20, 300, 4, 50),
    ("unit", 20, 300, 1, 50),
    ("unit", 20, 300, 16, 0),        # initialization only
    ("normal", 3, 20500, 16, 50),    # rows too long for LDS: workspace path
]


@pytest.mark.parametrize("kind,rows,cols,k,iters", CASES)
def test_palettize_matches_oracle(gpu_ctx, pe, kind, rows, cols, k, iters):
    w = weights(kind, rows, cols, 7000 + rows + cols)
    print(f"palettize {kind} {rows}x{cols} k={k} max_iter={iters}", flush=True)
    got = gpu_ctx.palettize(w, k, iters)
    want, _ = oracle.palettize_payload(w, k, iters, threads=8)
    assert got.size == want.size == gpu_ctx.palettize_bytes(rows, cols)
    bad = np.nonzero(got != want)[0]
    assert bad.size == 0, f"{bad.size} bytes differ, first at {bad[:8]}"


def test_palettize_dev_matches_host_and_oracle(gpu_ctx, pe):
    import torch
    w = weights("normal", 200, 896, 7101)
    d_w = torch.from_numpy(w).cuda()
    d_p = torch.empty(gpu_ctx.palettize_bytes(200, 896), dtype=torch.uint8, device="cuda")
    s = torch.cuda.Stream()
    gpu_ctx.palettize_dev(d_w, 200, 896, d_p, stream=s)
    s.synchronize()
    got = d_p.cpu().numpy()
    assert np.array_equal(got, gpu_ctx.palettize(w))
    want, _ = oracle.palettize_payload(w, 16, 50, threads=8)
    assert np.array_equal(got, want)


def test_palettize_gate_proj_size_matches_oracle(gpu_ctx, pe):
    """A full Qwen2.5-0.5B gate_proj (4864 x 896), byte for byte."""
    w = weights("normal", 4864, 896, 7102)
    print("palettize 4864x896", flush=True)
    got = gpu_ctx.palettize(w)
    want, _ = oracle.palettize_payload(w, 16, 50, threads=16)
    assert np.array_equal(got, want)


def test_palettize_embedding_round_trip(gpu_ctx, pe):
    """The tied embedding / LM head (151936 x 896): rows drawn from a
    synthetic 16-entry fp16 palette compile back to exactly those values,
    and the payload drives the GEMV like the original."""
    t = pe.palette.synth_tensor(151936, 896, 4, 7103)
    w = pe.palette.dequantize(t.payload, 151936, 896, 4)
    print("palettize 151936x896 round trip", flush=True)
    got = gpu_ctx.palettize(w)
    assert np.array_equal(decode(got, 151936, 896, pe), w)
    x = pe.palette.synth_x(1, 896, 7104)
    a = gpu_ctx.upload(got, 151936, 896, 4)
    b = gpu_ctx.upload(t.payload, 151936, 896, 4)
    assert np.array_equal(gpu_ctx.gemv(a, x), gpu_ctx.gemv(b, x))


SEEDED = [
    # kind, rows, cols, k, seeds
    ("normal", 64, 896, 16, [0.01, -0.02, 0.005]),
    ("unit", 32, 500, 16, np.linspace(-2, 2, 16).tolist()),   # k seeds: Lloyd only
    ("int", 20, 333, 8, [3.0, -7.0, 11.0, 0.0, 5.0, 5.0]),    # repeated seed
    ("normal", 3, 20500, 16, [0.0]),                          # workspace path
    ("normal", 10, 5, 16, [0.1, 0.2, 0.3, 0.4, 0.5, 0.6, 0.7]),  # k = n = 5 < nseeds
]


@pytest.mark.parametrize("kind,rows,cols,k,seeds", SEEDED)
def test_palettize_seeded_matches_oracle(gpu_ctx, pe, kind, rows, cols, k, seeds):
    """compute-core's palettize_matrix_phased with calibration seeds."""
    import torch
    w = weights(kind, rows, cols, 7200 + rows + cols)
    print(f"palettize seeded {kind} {rows}x{cols} k={k} nseeds={len(seeds)}", flush=True)
    want, _ = oracle.palettize_payload(w, k, 50, threads=8, seeds=seeds)
    assert np.array_equal(gpu_ctx.palettize(w, k, 50, seeds=seeds), want)
    d_w = torch.from_numpy(w).cuda()
    d_p = torch.empty(want.size, dtype=torch.uint8, device="cuda")
    gpu_ctx.palettize_dev(d_w, rows, cols, d_p, k, 50, seeds=seeds)
    torch.cuda.synchronize()
    assert np.array_equal(d_p.cpu().numpy(), want)


def test_palettize_errors(gpu_ctx, pe):
    w = weights("normal", 4, 32, 7105)
    for k in (0, 17):
        with pytest.raises(pe.PrismHipError):
            gpu_ctx.palettize(w, k)
    with pytest.raises(pe.PrismHipError):
        gpu_ctx.palettize(w, 16, 50, seeds=[])  # the reference panics on an empty seed list
    empty = gpu_ctx.palettize(np.zeros((0, 32), np.float32))
    assert empty.size == 0
    # in_dim 0: all-zero LUTs, no index bytes (fit_palette returns no entries)
    z = gpu_ctx.palettize(np.zeros((3, 0), np.float32))
    assert z.size == 96 and not z.any()
