"""HIP path vs the CPU oracle on identical seeded inputs, through the C ABI.

Bar: index unpack and LUT decode bit-exact; every output vector within
max|y - ref| / max|ref| <= 2e-3 (fp32 accumulation, fp16 output).  The GPU
sums in a different order than the sequential CPU fold, so a few outputs
may differ by one fp16 ulp; the tolerance is the contract.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

TOL = 2e-3


def _check(y, ref, what):
    y = np.asarray(y).reshape(-1, np.asarray(ref).shape[-1])
    ref = np.asarray(ref).reshape(y.shape)
    for b in range(y.shape[0]):
        err = _rel(y[b], ref[b])
        assert err <= TOL, f"{what}: vector {b} rel err {err:.3e}"
    return float(np.mean(y == ref))


def _rel(y, ref):
    a = y.view(np.float16).astype(np.float64)
    r = ref.view(np.float16).astype(np.float64)
    den = np.max(np.abs(r))
    return float(np.max(np.abs(a - r)) / den) if den > 0 else float(np.max(np.abs(a)))


# (bits, N, K): BASELINE shapes, decode-step shapes and ragged edges
GEMV_SHAPES = [
    (4, 4864, 896),      # config 1
    (4, 14336, 4096),    # hero
    (4, 18944, 3584),    # config 2 matrix
    (4, 896, 4864),      # Qwen down_proj
    (4, 128, 896),       # Qwen k/v proj
    (4, 151936, 896),    # Qwen tied LM head (tall: four one-wave tiles of 4 rows per workgroup)
    (4, 40001, 64),      # tall, ragged last workgroup (waves past the last row)
    (4, 4099, 1000), (4, 333, 520), (4, 3, 1024),  # 65..128 units: two one-wave tiles per workgroup, ragged
    (4, 1, 32), (4, 3, 64), (4, 17, 96), (4, 65, 160), (4, 100, 2080),
    (4, 5, 8), (4, 9, 24), (4, 7, 40), (4, 6, 100), (4, 4, 12), (4, 3, 4),  # ragged K: generic path
    (8, 14336, 4096),    # config 4
    (8, 1, 16), (8, 31, 48), (8, 64, 4096), (8, 9, 7), (8, 3, 100),
]


@pytest.mark.parametrize("bits,N,K", GEMV_SHAPES)
def test_gemv_b1(pe, oracle, gpu_ctx, bits, N, K):
    t = pe.synth_tensor(N, K, bits, seed=N * 7 + K)
    x = pe.synth_x(1, K, seed=N + K)
    w = gpu_ctx.upload_tensor(t)
    y = gpu_ctx.gemv(w, x)
    ref = oracle.gemv(x, t.payload, N, K, bits, threads=8)
    exact = _check(y, ref, f"{bits}-bit {N}x{K}")
    assert exact > 0.95
    w.free()


@pytest.mark.parametrize("bits,N,K", [(8, 14336, 4096), (4, 14336, 4096), (8, 300, 512), (4, 300, 896)])
@pytest.mark.parametrize("batch", [1, 2, 3, 4, 8, 11])
def test_gemv_batch(pe, oracle, gpu_ctx, bits, N, K, batch):
    if N * K > 10**7 and batch in (3, 11):
        pytest.skip("odd batches covered at the smaller shapes")
    t = pe.synth_tensor(N, K, bits, seed=batch + bits)
    x = pe.synth_x(batch, K, seed=batch)
    w = gpu_ctx.upload_tensor(t)
    y = gpu_ctx.gemv(w, x)
    ref = oracle.gemv(x, t.payload, N, K, bits, threads=8)
    _check(y, ref, f"{bits}-bit batch {batch}")
    w.free()


@pytest.mark.parametrize("bits,N,K,batch", [
    (8, 14336, 4096, 5), (8, 14336, 4096, 6),   # matrix-core kernel (5..8 vectors, N >= 4096)
    (4, 14336, 4096, 6),
    (8, 4100, 1024, 7), (4, 4100, 1024, 7),      # ragged last 32-row workgroup
    (8, 4096, 14336, 8), (4, 4096, 14336, 8),    # long rows on the matrix cores
    (8, 4096, 14336, 13),                        # up to 16 vectors a matrix-core pass
    (4, 14336, 4096, 16), (4, 4096, 1024, 19),   # 16 + 3
    (8, 4100, 1024, 20),                         # 16 + 4: the 4 by the tile kernel
    (4, 2048, 14336, 8),                         # too few rows for the matrix cores, rows too long
    (8, 2048, 14336, 6),                         #   for 8 vectors a tile pass: 4 + 4, 4 + 2
    (4, 64, 20000, 7),                           # 2 + 2 + 2 + 1
])
def test_gemv_batch_wide(pe, oracle, gpu_ctx, bits, N, K, batch):
    """Batches past 4 vectors: the 8-bit matrix-core kernel and the tile
    kernel's narrower passes for rows too long for 8 vectors at once."""
    t = pe.synth_tensor(N, K, bits, seed=batch + bits + K)
    x = pe.synth_x(batch, K, seed=batch + 17)
    w = gpu_ctx.upload_tensor(t)
    print(f"gemv {bits}-bit {N}x{K} batch {batch}", flush=True)
    y = gpu_ctx.gemv(w, x)
    ref = oracle.gemv(x, t.payload, N, K, bits, threads=8)
    _check(y, ref, f"{bits}-bit {N}x{K} batch {batch}")
    w.free()


@pytest.mark.parametrize("bits,N,K", [(4, 4864, 896), (4, 1000, 4096), (8, 700, 4096), (4, 33, 40), (8, 20, 24),
                                      (8, 4096, 1024), (4, 4096, 1024)])
def test_decode_bit_exact_through_gemv(pe, gpu_ctx, bits, N, K):
    """One-hot x (x = e_k) makes every output the decoded weight itself:
    y[r] = LUT_r[idx(r, k)] exactly, through the GEMV kernel's own decode."""
    t = pe.synth_tensor(N, K, bits, seed=K + 3)
    lut, idx = pe.unpack_payload(t.payload, N, K, bits)
    keff = (K // 8) * 8 if bits == 4 else K
    ks = sorted(set([0, 1, keff - 1, keff // 2, 7 % keff, (keff * 5) // 8]))
    x = np.zeros((len(ks), K), dtype=np.float16)
    for i, k in enumerate(ks):
        x[i, k] = 1.0
    w = gpu_ctx.upload_tensor(t)
    y = gpu_ctx.gemv(w, x.view(np.uint16))
    for i, k in enumerate(ks):
        want = lut[np.arange(N), idx[:, k]]
        want = np.where(want == 0x8000, 0, want)  # 0.0 + (-0.0) = +0.0
        assert np.array_equal(y[i], want), f"column {k}"
    w.free()


@pytest.mark.parametrize("bits,N,K", [(4, 4864, 896), (8, 300, 4096), (4, 7, 100), (8, 5, 33)])
def test_decode_rows_bit_exact(pe, oracle, gpu_ctx, bits, N, K):
    import torch
    t = pe.synth_tensor(N, K, bits, seed=N)
    w = gpu_ctx.upload_tensor(t)
    out = torch.empty((N, K), dtype=torch.int16, device="cuda")
    gpu_ctx.decode_rows_dev(w, 0, N, out)
    torch.cuda.synchronize()
    got = out.cpu().numpy().view(np.uint16)
    assert np.array_equal(got, oracle.decode_rows(t.payload, N, K, bits))
    for tok in (0, N // 2, N - 1, N, N + 5):
        e = gpu_ctx.lut_embed(w, tok)
        assert np.array_equal(e, oracle.decode_rows(t.payload, N, K, bits, tok, 1)[0] if tok < N
                              else np.zeros(K, np.uint16))
    if bits == 4:
        assert np.array_equal(gpu_ctx.lut_embed(w, 1), oracle.lut_embed(1, t.payload, N, K))
    w.free()


@pytest.mark.parametrize("bits,N,K", [(4, 18944, 3584), (4, 4864, 896), (4, 50, 128), (4, 9, 40), (8, 700, 1024),
                                      (4, 333, 1000)])
def test_gateup_swiglu(pe, oracle, gpu_ctx, bits, N, K):
    g = pe.synth_tensor(N, K, bits, seed=2 * N + 1)
    u = pe.synth_tensor(N, K, bits, seed=2 * N + 2)
    x = pe.synth_x(1, K, seed=K)
    wg, wu = gpu_ctx.upload_tensor(g), gpu_ctx.upload_tensor(u)
    y = gpu_ctx.gateup_swiglu(wg, wu, x)
    ref = oracle.gateup_swiglu(x[0], g.payload, u.payload, N, K, bits, threads=8)
    _check(y, ref, f"gate_up {N}x{K}")
    wg.free()
    wu.free()


@pytest.mark.parametrize("bits,M,N,K", [(4, 64, 256, 512), (4, 77, 200, 96), (8, 40, 130, 256),
                                        (4, 3, 5, 64), (4, 10, 20, 40), (4, 300, 1000, 1024),
                                        # 2, 3 and 5 K steps of 64: every tail of the 3-stage ring,
                                        # with 64-, 128- and 256-row blocks
                                        (4, 60, 300, 128), (4, 70, 260, 192), (4, 100, 260, 320),
                                        (4, 257, 513, 320), (4, 600, 300, 128), (4, 520, 300, 320),
                                        # up to 48 rows: GEMV passes of up to 16 (matrix cores at N >= 4096)
                                        (4, 48, 4096, 512), (8, 20, 4100, 256),
                                        # 64-, 128- and 256-row blocks (M <= 256, <= 512, more)
                                        (4, 49, 300, 512), (4, 200, 4100, 256), (4, 300, 700, 192),
                                        (4, 513, 260, 128),
                                        # 8-bit: GEMV passes up to 64 rows, the LDS-decode GEMM past them
                                        (8, 64, 4096, 256), (8, 80, 300, 256),
                                        # 8-bit over 256 rows: 256 x 128 blocks, K step 64; else 128 x 128, step 32
                                        (8, 300, 1000, 1024), (8, 513, 260, 192), (8, 257, 300, 64),
                                        (8, 256, 300, 128), (8, 300, 129, 96),
                                        # 4-bit split-K (33..256 rows, K >= 1024): 2, 3 and 4
                                        # splits, a short last split, ragged N
                                        (4, 33, 64, 4096), (4, 40, 300, 1024), (4, 100, 4100, 2048),
                                        (4, 129, 700, 1536), (4, 256, 520, 1088), (4, 160, 2000, 1024),
                                        # 8-bit split-K (49..256 rows, K >= 1024): 2, 3 and 4 splits
                                        (8, 49, 300, 1024), (8, 100, 4100, 2048), (8, 256, 700, 1536),
                                        (8, 129, 14336, 1088)])
def test_gemm_small(pe, oracle, gpu_ctx, bits, M, N, K):
    t = pe.synth_tensor(N, K, bits, seed=M + N)
    X = pe.synth_x(M, K, seed=M)
    w = gpu_ctx.upload_tensor(t)
    Y = gpu_ctx.gemm(w, X)
    ref = oracle.gemm(X, t.payload, N, K, bits, threads=8)
    _check(Y, ref, f"gemm {M}x{N}x{K}")
    w.free()


def test_gemm_short_prefill_split(pe, oracle, gpu_ctx):
    """A 128-row prefill over the config-5 weights (split K): every row
    against the oracle, through the device entry point on a torch stream,
    twice in a row (the second call reuses the pooled partials)."""
    import torch
    M, N, K = 128, 14336, 4096
    t = pe.synth_tensor(N, K, 4, seed=pe.SEEDS["cfg5"])
    X = pe.synth_x(M, K, seed=5)
    w = gpu_ctx.upload_tensor(t)
    dX = torch.from_numpy(X.view(np.int16)).cuda()
    ref = oracle.gemm(X, t.payload, N, K, 4, threads=8)
    s = torch.cuda.Stream()
    for _ in range(2):
        dY = torch.full((M, N), -1, dtype=torch.int16, device="cuda")
        torch.cuda.synchronize()
        gpu_ctx.gemm_dev(w, dX, M, dY, s)
        s.synchronize()
        _check(dY.cpu().numpy().view(np.uint16), ref, "gemm 128x14336x4096 split-K")
    w.free()


def test_split_gemm_two_streams(pe, oracle, gpu_ctx):
    """Two split-K GEMMs of different inputs enqueued on two streams with no
    synchronisation between them (each gets its own pooled partials), then
    a third on the first stream after both: every output against the oracle."""
    import torch
    M, N, K = 96, 2000, 2048
    t = pe.synth_tensor(N, K, 4, seed=31)
    w = gpu_ctx.upload_tensor(t)
    Xs = [pe.synth_x(M, K, seed=32 + i) for i in range(3)]
    dXs = [torch.from_numpy(X.view(np.int16)).cuda() for X in Xs]
    dYs = [torch.full((M, N), -1, dtype=torch.int16, device="cuda") for _ in range(3)]
    s0, s1 = torch.cuda.Stream(), torch.cuda.Stream()
    torch.cuda.synchronize()
    gpu_ctx.gemm_dev(w, dXs[0], M, dYs[0], s0)
    gpu_ctx.gemm_dev(w, dXs[1], M, dYs[1], s1)
    s0.wait_stream(s1)
    gpu_ctx.gemm_dev(w, dXs[2], M, dYs[2], s0)
    torch.cuda.synchronize()
    for i in range(3):
        _check(dYs[i].cpu().numpy().view(np.uint16), oracle.gemm(Xs[i], t.payload, N, K, 4, threads=8),
               f"split gemm on stream, input {i}")
    w.free()


def test_graph_replay_gemv_and_split_gemm(pe, oracle, gpu_ctx):
    """A GEMV and a split-K GEMM (its pooled partials become graph memory
    nodes) captured in one HIP graph and replayed three times, with eager
    library work and host synchronisation between replays: every replay
    reproduces the eager outputs bit for bit, which match the oracle."""
    import torch
    M, N, K = 64, 4100, 2048
    t = pe.synth_tensor(N, K, 4, seed=21)
    w = gpu_ctx.upload_tensor(t)
    X = pe.synth_x(M, K, seed=22)
    dX = torch.from_numpy(X.view(np.int16)).cuda()
    dYm = torch.empty((M, N), dtype=torch.int16, device="cuda")
    dYv = torch.empty((1, N), dtype=torch.int16, device="cuda")
    s = torch.cuda.Stream()
    gpu_ctx.gemm_dev(w, dX, M, dYm, s)
    gpu_ctx.gemv_dev(w, dX[:1], 1, dYv, s)
    s.synchronize()
    want_m = dYm.cpu().numpy().view(np.uint16).copy()
    want_v = dYv.cpu().numpy().view(np.uint16).copy()
    _check(want_m, oracle.gemm(X, t.payload, N, K, 4, threads=8), "eager split gemm")
    _check(want_v, oracle.gemv(X[:1], t.payload, N, K, 4), "eager gemv")
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        gpu_ctx.gemm_dev(w, dX, M, dYm, s)
        gpu_ctx.gemv_dev(w, dX[:1], 1, dYv, s)
    other = torch.empty((40, N), dtype=torch.int16, device="cuda")
    for rep in range(3):
        dYm.fill_(-1)
        dYv.fill_(-1)
        gpu_ctx.gemm_dev(w, dX[:40], 40, other)  # eager work on the context stream between replays
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(dYm.cpu().numpy().view(np.uint16), want_m), f"replay {rep}: gemm differs"
        assert np.array_equal(dYv.cpu().numpy().view(np.uint16), want_v), f"replay {rep}: gemv differs"
    del g
    w.free()


def test_gemm_config5_sampled(pe, oracle, gpu_ctx):
    """Config 5 at full size (X 2048x4096, W 14336x4096 4-bit): every one of
    the 2048 rows against a float32 CPU product of the dequantized W (second
    oracle, in 256-row chunks), and 3 rows of every 256-row M block (the
    GEMM's block height) plus 8 random rows against the oracle."""
    import torch
    M, N, K = 2048, 14336, 4096
    t = pe.synth_tensor(N, K, 4, seed=pe.SEEDS["cfg5"])
    X = pe.synth_x(M, K, seed=pe.SEEDS["cfg5"])
    w = gpu_ctx.upload_tensor(t)
    dX = torch.from_numpy(X.view(np.int16)).cuda()
    dY = torch.empty((M, N), dtype=torch.int16, device="cuda")
    gpu_ctx.gemm_dev(w, dX, M, dY)
    torch.cuda.synchronize()
    Y = dY.cpu().numpy().view(np.uint16)
    rng = np.random.default_rng(0)
    rows = sorted(set([b * 256 + o for b in range(M // 256) for o in (0, 131, 255)] +
                      list(rng.choice(M, 8, replace=False))))
    ref = oracle.gemm(np.ascontiguousarray(X[rows]), t.payload, N, K, 4, threads=16)
    _check(Y[rows], ref, "gemm cfg5 rows of every M block")
    Wt = torch.from_numpy(pe.dequantize(t.payload, N, K, 4)).T.contiguous()
    Xf = torch.from_numpy(X.view(np.float16).astype(np.float32))
    worst = 0.0
    for m0 in range(0, M, 256):
        R = (Xf[m0:m0 + 256] @ Wt).numpy()
        Yf = Y[m0:m0 + 256].view(np.float16).astype(np.float32)
        err = np.max(np.abs(Yf - R), axis=1) / np.max(np.abs(R), axis=1)
        worst = max(worst, float(err.max()))
        assert np.all(err <= TOL), f"rows {m0}..{m0 + 255}: worst {err.max():.3e} at row {m0 + int(err.argmax())}"
    print(f"cfg5: all {M} rows within {worst:.3e} of the fp32 product", flush=True)
    w.free()


def test_errors_never_crash(pe, gpu_ctx):
    lib = gpu_ctx.lib
    t = pe.synth_tensor(16, 64, 4, seed=1)
    p = t.payload
    assert lib.prism_hip_weight_upload(gpu_ctx.h, p.ctypes.data, p.size, 16, 64, 5, 0) is None
    assert "bits" in gpu_ctx.error()
    assert lib.prism_hip_weight_upload(gpu_ctx.h, p.ctypes.data, p.size - 1, 16, 64, 4, 0) is None
    assert "needs" in gpu_ctx.error()
    assert lib.prism_hip_weight_upload(gpu_ctx.h, p.ctypes.data, p.size, 16, 64, 4, 3) is None
    assert lib.prism_hip_weight_upload(gpu_ctx.h, p.ctypes.data, 0, 0, 64, 4, 0) is None
    w = gpu_ctx.upload_tensor(t)
    u = gpu_ctx.upload_tensor(pe.synth_tensor(16, 32, 4, seed=2))
    x = pe.synth_x(1, 64, seed=1)
    y = np.zeros(16, np.uint16)
    assert lib.prism_hip_gateup_swiglu(gpu_ctx.h, w.h, u.h, x.ctypes.data, y.ctypes.data) == -8
    assert lib.prism_hip_gemv(gpu_ctx.h, w.h, None, 1, y.ctypes.data) == -1
    assert lib.prism_hip_gemv(gpu_ctx.h, None, x.ctypes.data, 1, y.ctypes.data) == -1
    other = pe.Context(0)
    assert lib.prism_hip_gemv(other.h, w.h, x.ctypes.data, 1, y.ctypes.data) == -10
    other.close()
    assert lib.prism_hip_gemv(gpu_ctx.h, w.h, x.ctypes.data, 0, y.ctypes.data) == 0  # empty batch
    import torch
    d = torch.empty(16 * 64, dtype=torch.int16, device="cuda")
    assert lib.prism_hip_decode_rows_dev(gpu_ctx.h, w.h, 10, 7, d.data_ptr(), None) == -3
    w.free()
    u.free()


def test_backend_keyed_surface(pe, oracle):
    """HipBackend mirrors MetalBackend: keyed gemv / fused_gate_up, "miss
    <key>" on an unknown tensor, embed of an out-of-range token is zeros."""
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    q = pe.synth_tensor(896, 896, 4, seed=1, key="layers.0.q_proj")
    g = pe.synth_tensor(4864, 896, 4, seed=2, key="layers.0.gate_proj")
    u = pe.synth_tensor(4864, 896, 4, seed=3, key="layers.0.up_proj")
    b = pe.HipBackend.new({t.key: t for t in (q, g, u)})
    assert len(b) == 3
    x = pe.synth_x(1, 896, seed=4)[0]
    out = np.zeros(896, np.uint16)
    b.gemv("layers.0.q_proj", x, out)
    _check(out, oracle.lut_gemv4(x, q.payload, 896, 896), "backend gemv")
    with pytest.raises(pe.PrismHipError, match="miss nope"):
        b.gemv("nope", x, out)
    with pytest.raises(pe.PrismHipError):
        b.gemv("layers.0.q_proj", x[:100], out)
    y = np.zeros(4864, np.uint16)
    b.fused_gate_up("layers.0.gate_proj", "layers.0.up_proj", x, y)
    _check(y, oracle.gateup_swiglu(x, g.payload, u.payload, 4864, 896), "backend fused_gate_up")
    with pytest.raises(pe.PrismHipError, match="miss layers.0.nope"):
        b.fused_gate_up("layers.0.gate_proj", "layers.0.nope", x, y)
    e = np.ones(896, np.uint16)
    b.embed("layers.0.q_proj", 5000, e)
    assert np.all(e == 0)
    b.embed("layers.0.q_proj", 3, e)
    assert np.array_equal(e, oracle.lut_embed(3, q.payload, 896, 896))
    b.close()


def test_cimage_load_to_backend(pe, oracle, tmp_path):
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    path = str(tmp_path / "m.cimage")
    wr = pe.CImageWriter(path)
    ts = [pe.synth_tensor(256, 512, 4, seed=i, key=f"layers.{i}.o_proj") for i in range(3)]
    for t in ts:
        wr.append_palettized(t.key, t.payload, t.dim_m, t.dim_n)
    t8 = pe.synth_tensor(128, 256, 8, seed=9, key="w8")
    wr.append_palettized("w8", t8.payload, 128, 256, bits=8)
    wr.finalize()
    b = pe.load_cimage(path)
    assert len(b) == 4
    x = pe.synth_x(1, 512, seed=5)[0]
    for t in ts:
        out = np.zeros(256, np.uint16)
        b.gemv(t.key, x, out)
        _check(out, oracle.lut_gemv4(x, t.payload, 256, 512), t.key)
    b.close()
