"""The GI device layout (weights with rows of >= 2048 elements, K % 64 == 0
at 4 bits and K % 512 == 0 at 8, in groups of G = 32..64 rows,
G = ceil(N / num_cu) rounded up to a multiple of 8) and the two-output
gate/up GEMV, through the C ABI against the CPU oracle.

Every operation on a weight must give the same results whatever device
layout the library chose for it: the lane-per-row GEMVs (4-bit: 1..2
vectors; 8-bit: 1..8), the matrix-core GEMV over GI (more vectors), the
generic kernel (unaligned x), the GEMM, the row decode and the decode-step
model's copies.  4-bit shapes (on a 256-CU MI355X): 14336 x 4096 (56-row
groups, 256 of them), 9100 x 2048 (40-row groups, 228 with a ragged last
one), 8192 x 2112 (32-row groups; K % 128 != 0: no matrix-core pass),
16384 x 2048 (64-row groups); more than 64 rows per CU take 32-row groups
and the half-group kernels (two groups, or gate and up of one group, in the
two halves of a wave): 18944 x 3584 (config 2's matrices: 592 groups, 14
chunks per wave), 16416 x 2048 and 16416 x 2560 (513 groups: the last
workgroup's second half is past the matrix; 8 chunks per wave, and 10:
the run-time chunk loop).  8-bit shapes:
14336 x 4096 and 9100 x 2048 (chunk counts the 8-bit kernel takes as
compile-time constants), 8192 x 2560 (its loop form), 16384 x 2048.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

TOL = 2e-3
GI_SHAPES = [(14336, 4096), (9100, 2048), (8192, 2112), (16384, 2048), (18944, 3584), (16416, 2048),
             (16416, 2560)]
HG_SHAPES = [(18944, 3584), (16416, 2560)]  # 32-row groups, half-group kernels


def _rel(y, ref):
    a = np.asarray(y).view(np.float16).astype(np.float64)
    r = np.asarray(ref).view(np.float16).astype(np.float64)
    den = np.max(np.abs(r))
    return float(np.max(np.abs(a - r)) / den) if den > 0 else float(np.max(np.abs(a)))


def _check(y, ref, what):
    y = np.asarray(y).reshape(-1, np.asarray(ref).shape[-1])
    ref = np.asarray(ref).reshape(y.shape)
    for b in range(y.shape[0]):
        err = _rel(y[b], ref[b])
        assert err <= TOL, f"{what}: vector {b} rel err {err:.3e}"


def _gi(N, K, bits=4, num_cu=256):
    """The library's layout rule (prism_hip.hip gi_rows): the group rows, or 0."""
    if K < 2048 or bits not in (4, 8) or K % (64 if bits == 4 else 512):
        return 0
    G = (-(-N // num_cu) + 7) // 8 * 8
    if bits == 4 and G > 64 and -(-N // 64) <= 2 * num_cu:
        G = 32
    return G if 32 <= G <= 64 else 0


@pytest.mark.parametrize("N,K", GI_SHAPES)
@pytest.mark.parametrize("batch", [1, 2, 3, 5, 8, 16])
def test_gi_gemv(pe, oracle, gpu_ctx, N, K, batch):
    assert _gi(N, K)
    if N * K > 4 * 10**7 and batch in (3, 5):
        pytest.skip("odd batches covered at the smaller shapes")
    t = pe.synth_tensor(N, K, 4, seed=N + K + batch)
    x = pe.synth_x(batch, K, seed=batch * 3 + 1)
    w = gpu_ctx.upload_tensor(t)
    print(f"gi gemv {N}x{K} batch {batch}", flush=True)
    y = gpu_ctx.gemv(w, x)
    ref = oracle.gemv(x, t.payload, N, K, 4, threads=8)
    _check(y, ref, f"GI {N}x{K} batch {batch}")
    w.free()


@pytest.mark.parametrize("N,K", [(14336, 4096), (9100, 2048)])
def test_gi_decode_bit_exact_through_gemv(pe, gpu_ctx, N, K):
    """One-hot x: every output is the decoded weight itself, LUT_r[idx(r, k)],
    through the lane-per-row GEMV (one vector) and the matrix-core GEMV
    over GI (six vectors at once)."""
    t = pe.synth_tensor(N, K, 4, seed=K + 11)
    lut, idx = pe.unpack_payload(t.payload, N, K, 4)
    ks = [0, 1, 31, 32, K // 2 + 5, K - 1]
    x = np.zeros((len(ks), K), dtype=np.float16)
    for i, k in enumerate(ks):
        x[i, k] = 1.0
    w = gpu_ctx.upload_tensor(t)
    ys = gpu_ctx.gemv(w, x.view(np.uint16))
    for i, k in enumerate(ks):
        want = lut[np.arange(N), idx[:, k]]
        want = np.where(want == 0x8000, 0, want)  # 0.0 + (-0.0) = +0.0
        y1 = gpu_ctx.gemv(w, x[i:i + 1].view(np.uint16))[0]
        assert np.array_equal(y1, want), f"column {k}, one vector"
        assert np.array_equal(ys[i], want), f"column {k}, six vectors"
    w.free()


@pytest.mark.parametrize("nb", [1, 2])
def test_gi_lpr_x_on_16_byte_boundary(pe, oracle, gpu_ctx, nb):
    """x 16-byte aligned but not 64-byte aligned: the lane-per-row kernel
    reads x with scalar loads, which need dword alignment only."""
    import torch
    N, K = 14336, 4096
    t = pe.synth_tensor(N, K, 4, seed=77)
    x = pe.synth_x(nb, K, seed=78)
    w = gpu_ctx.upload_tensor(t)
    buf = torch.zeros(nb * K + 64, dtype=torch.int16, device="cuda")
    assert buf.data_ptr() % 64 == 0
    buf[8:8 + nb * K] = torch.from_numpy(x.reshape(-1).view(np.int16)).cuda()
    dx = buf[8:]  # 16 bytes past a 64-byte boundary
    dy = torch.empty(nb * N, dtype=torch.int16, device="cuda")
    print(f"LPR x at +16 B, nb={nb}", flush=True)
    gpu_ctx.gemv_dev(w, dx, nb, dy)
    torch.cuda.synchronize()
    y = dy.cpu().numpy().view(np.uint16).reshape(nb, N)
    want = oracle.gemv(x, t.payload, N, K, 4, threads=8)
    _check(y, want, f"GI LPR x at +16 B nb={nb}")
    # the same call on 64-byte-aligned x gives the same bits
    dx2 = torch.from_numpy(x.reshape(-1).view(np.int16)).cuda()
    dy2 = torch.empty(nb * N, dtype=torch.int16, device="cuda")
    gpu_ctx.gemv_dev(w, dx2, nb, dy2)
    torch.cuda.synchronize()
    assert np.array_equal(dy2.cpu().numpy().view(np.uint16).reshape(nb, N), y)
    w.free()


@pytest.mark.parametrize("N,K", [(14336, 4096), (9100, 2048), (16416, 2048)])
def test_gi_unaligned_x(pe, oracle, gpu_ctx, N, K):
    """x not 16-byte aligned: the generic kernel reads GI as well."""
    import torch
    t = pe.synth_tensor(N, K, 4, seed=N - K)
    x = pe.synth_x(2, K, seed=5)
    w = gpu_ctx.upload_tensor(t)
    buf = torch.zeros(2 * K + 8, dtype=torch.int16, device="cuda")
    buf[1:1 + 2 * K] = torch.from_numpy(x.reshape(-1).view(np.int16)).cuda()
    dx = buf[1:]
    dy = torch.empty(2 * N, dtype=torch.int16, device="cuda")
    gpu_ctx.gemv_dev(w, dx, 2, dy)
    torch.cuda.synchronize()
    y = dy.cpu().numpy().view(np.uint16).reshape(2, N)
    _check(y, oracle.gemv(x, t.payload, N, K, 4, threads=8), f"GI {N}x{K} unaligned x")
    w.free()


@pytest.mark.parametrize("N,K", [(14336, 4096), (9100, 2048), (16416, 2048)])
def test_gi_decode_rows(pe, oracle, gpu_ctx, N, K):
    """Row decode and lut_embed over GI are the oracle's bytes exactly,
    including rows of the ragged last group."""
    import torch
    t = pe.synth_tensor(N, K, 4, seed=3 * N + 1)
    w = gpu_ctx.upload_tensor(t)
    for r0, nr in [(0, 3), (63, 2), (N - 5, 5), (N // 2, 64)]:
        out = torch.empty(nr * K, dtype=torch.int16, device="cuda")
        gpu_ctx.decode_rows_dev(w, r0, nr, out)
        torch.cuda.synchronize()
        got = out.cpu().numpy().view(np.uint16).reshape(nr, K)
        want = oracle.decode_rows(t.payload, N, K, 4, r0, nr)
        assert np.array_equal(got, want), f"rows {r0}..{r0 + nr}"
    for tok in (0, 64, N - 1):
        assert np.array_equal(gpu_ctx.lut_embed(w, tok), oracle.lut_embed(tok, t.payload, N, K)), f"token {tok}"
    w.free()


@pytest.mark.parametrize("N,K", [(14336, 4096), (9100, 2048), (16416, 2048)])
def test_gi_upload_dev(pe, gpu_ctx, N, K):
    """A device-side payload is regrouped the same way as a host one."""
    import torch
    t = pe.synth_tensor(N, K, 4, seed=N * 2 + K)
    x = pe.synth_x(1, K, seed=9)
    w_host = gpu_ctx.upload_tensor(t)
    dpay = torch.from_numpy(t.payload.view(np.int8)).cuda()
    w_dev = gpu_ctx.upload_dev(dpay, N, K, 4)
    assert np.array_equal(gpu_ctx.gemv(w_host, x), gpu_ctx.gemv(w_dev, x))
    w_host.free()
    w_dev.free()


# (bits, N, K): split-block shapes of every tile form (one-wave tiles, two
# per workgroup, 8-bit), config 2's matrix, ragged K (generic kernel), and
# GI shapes (the lane-per-row kernel's pair form)
PAIR_SHAPES = [(4, 4864, 896), (4, 18944, 3584), (4, 300, 4096), (8, 300, 512), (8, 14336, 4096),
               (4, 7, 40), (8, 9, 7), (4, 14336, 4096), (4, 9100, 2048), (4, 16416, 2048),
               (4, 16416, 2560)]


@pytest.mark.parametrize("bits,N,K", PAIR_SHAPES)
def test_gate_up_pair(pe, oracle, gpu_ctx, bits, N, K):
    """prism_hip_gate_up: both raw outputs equal separate GEMVs bit for bit
    (same kernels, same summation order) and the oracle within tolerance."""
    tg = pe.synth_tensor(N, K, bits, seed=N + 1)
    tu = pe.synth_tensor(N, K, bits, seed=N + 2)
    x = pe.synth_x(1, K, seed=N + 3)
    wg, wu = gpu_ctx.upload_tensor(tg), gpu_ctx.upload_tensor(tu)
    print(f"gate_up pair {bits}-bit {N}x{K}", flush=True)
    yg, yu = gpu_ctx.gate_up(wg, wu, x)
    assert np.array_equal(yg, gpu_ctx.gemv(wg, x)[0]), "gate output differs from its GEMV"
    assert np.array_equal(yu, gpu_ctx.gemv(wu, x)[0]), "up output differs from its GEMV"
    _check(yg, oracle.gemv(x, tg.payload, N, K, bits, threads=8), "gate")
    _check(yu, oracle.gemv(x, tu.payload, N, K, bits, threads=8), "up")
    wg.free()
    wu.free()


def test_gate_up_pair_dev_and_errors(pe, gpu_ctx):
    """The device form on a torch stream matches the host form; shape and
    NULL checks return the documented codes."""
    import torch
    from importlib import import_module
    nat = import_module("prism-engine_amd._native")
    N, K = 14336, 4096
    tg, tu = pe.synth_tensor(N, K, 4, seed=1), pe.synth_tensor(N, K, 4, seed=2)
    x = pe.synth_x(1, K, seed=3)
    wg, wu = gpu_ctx.upload_tensor(tg), gpu_ctx.upload_tensor(tu)
    yg, yu = gpu_ctx.gate_up(wg, wu, x)
    s = torch.cuda.Stream()
    dx = torch.from_numpy(x.view(np.int16)).cuda()
    dg = torch.empty(N, dtype=torch.int16, device="cuda")
    du = torch.empty(N, dtype=torch.int16, device="cuda")
    gpu_ctx.gate_up_dev(wg, wu, dx, dg, du, stream=s)
    s.synchronize()
    assert np.array_equal(dg.cpu().numpy().view(np.uint16), yg)
    assert np.array_equal(du.cpu().numpy().view(np.uint16), yu)
    small = gpu_ctx.upload_tensor(pe.synth_tensor(64, K, 4, seed=4))
    with pytest.raises(nat.PrismHipError) as e:
        gpu_ctx.gate_up(wg, small, x)
    assert e.value.code == nat.ERR_MISMATCH
    lib = nat.load()
    assert lib.prism_hip_gate_up(gpu_ctx.h, wg.h, wu.h, None, None, None) == nat.ERR_NULL
    for w in (wg, wu, small):
        w.free()


@pytest.mark.parametrize("N,K", [(14336, 4096), (9100, 2048)] + HG_SHAPES)
def test_gi_gateup_swiglu(pe, oracle, gpu_ctx, N, K):
    tg = pe.synth_tensor(N, K, 4, seed=N + 5)
    tu = pe.synth_tensor(N, K, 4, seed=N + 6)
    x = pe.synth_x(1, K, seed=N + 7)
    wg, wu = gpu_ctx.upload_tensor(tg), gpu_ctx.upload_tensor(tu)
    y = gpu_ctx.gateup_swiglu(wg, wu, x)
    ref = oracle.gateup_swiglu(x[0], tg.payload, tu.payload, N, K, 4, threads=8)
    _check(y, ref, f"GI gate_up + SwiGLU {N}x{K}")
    wg.free()
    wu.free()


@pytest.mark.parametrize("N,M", [(9100, 24), (9100, 64), (9100, 200), (9100, 300), (16416, 24), (16416, 64),
                                 (16416, 300)])
def test_gi_gemm(pe, oracle, gpu_ctx, N, M):
    """Prefill GEMM over GI weights with a ragged last group (9100: 40-row
    groups, so a wave's 64 rows span two of them; 16416: 32-row groups, the
    last one half full): GEMV passes (24 rows), split K (64, 200) and
    whole-K blocks (300); every row checked against the float32 product of
    the decoded weights, a spread of rows against the oracle."""
    K = 2048
    assert _gi(N, K)
    t = pe.synth_tensor(N, K, 4, seed=M + 40)
    X = pe.synth_x(M, K, seed=M + 41)
    w = gpu_ctx.upload_tensor(t)
    print(f"gi gemm {N}x{K} M={M}", flush=True)
    Y = gpu_ctx.gemm(w, X)
    dense = oracle.decode_rows(t.payload, N, K, 4, 0, N).view(np.float16).astype(np.float32)
    Yf = X.view(np.float16).astype(np.float32) @ dense.T
    got = Y.view(np.float16).astype(np.float32)
    for m in range(M):
        err = np.max(np.abs(got[m] - Yf[m])) / np.max(np.abs(Yf[m]))
        assert err <= TOL, f"row {m}: {err:.3e}"
    rows = sorted(set([0, M // 3, M // 2, M - 1]))
    ref = oracle.gemm(np.ascontiguousarray(X[rows]), t.payload, N, K, 4, threads=8)
    for i, m in enumerate(rows):
        assert _rel(Y[m], ref[i]) <= TOL
    w.free()


@pytest.mark.parametrize("inter", [8192, 16416])
def test_gi_model_step(pe, oracle, gpu_ctx, inter):
    """A decode-step model whose embedding (9000 x 2048) and gate/up
    (8192 or 16416 x 2048: 32-row groups, the second in half-group form)
    weights were uploaded in the GI layout: the model's split-block copies
    are regrouped back, and the step matches the oracle."""
    cfg = pe.Qwen2Config(n_layers=1, hidden=2048, n_heads=32, n_kv_heads=4, head_dim=64, intermediate=inter,
                         vocab=9000)
    assert _gi(cfg.vocab, cfg.hidden) and _gi(cfg.intermediate, cfg.hidden)
    embed, layers = pe.synth_weights(cfg, 21)
    m = pe.Model.from_tensors(gpu_ctx, cfg, embed, layers, max_seq=16)
    kv = oracle.KVState(cfg.n_layers, cfg.kv_dim, 16)
    for l, (k, v) in enumerate(pe.synth_kv(cfg, 4, 21)):
        m.kv_append(l, k, v)
        for i in range(4):
            kv.append(l, k[i], v[i])
    got = m.step(77, 4)
    emb_p, lay_p = pe.model.payloads(embed, layers)
    want = oracle.decode_step(cfg.oracle_dims(), cfg.rms_eps, emb_p, lay_p, kv, 77, 4, threads=8)
    err = _rel(got, want)
    assert err <= TOL, f"logits rel err {err:.3e}"
    m.close()


GI8_SHAPES = [(14336, 4096), (9100, 2048), (8192, 2560), (16384, 2048)]


@pytest.mark.parametrize("N,K", GI8_SHAPES)
@pytest.mark.parametrize("batch", [1, 2, 3, 4, 5, 8, 9, 20])
def test_gi8_gemv(pe, oracle, gpu_ctx, N, K, batch):
    """8-bit GI: k_gemv_lpr8 passes of 1 / 2 vectors, k_gemv_lpr8m for 3..8
    (lookups into the matrix cores) and the matrix-core GEMV over GI from 9
    vectors on."""
    assert _gi(N, K, 8)
    if N * K > 4 * 10**7 and batch in (3, 5, 9):
        pytest.skip("odd batches covered at the smaller shapes")
    t = pe.synth_tensor(N, K, 8, seed=N + K + batch + 8)
    x = pe.synth_x(batch, K, seed=batch * 5 + 2)
    w = gpu_ctx.upload_tensor(t)
    print(f"gi8 gemv {N}x{K} batch {batch}", flush=True)
    y = gpu_ctx.gemv(w, x)
    ref = oracle.gemv(x, t.payload, N, K, 8, threads=8)
    _check(y, ref, f"GI8 {N}x{K} batch {batch}")
    w.free()


@pytest.mark.parametrize("N,K", [(14336, 4096), (9100, 2048), (8192, 2112)] + HG_SHAPES)
def test_gi4_decode_bit_exact_through_lpr(pe, gpu_ctx, N, K):
    """One-hot x through the 4-bit lane-per-row GEMV (one vector): every
    output is LUT_r[idx(r, k)] exactly.  k runs over every element of the
    first wave's K slice (every chunk and product position; with 16 / 8
    chunks per wave the kernel's chunk sequence is compile-time) and the
    last 64 elements of the row (the last wave's last products, summed right
    after the chunk sequence); 2112 (66 chunks, not a multiple of 8 waves)
    and 2560 (10 chunks per wave) take the run-time loop.  The half-group
    shapes check both halves of every wave (rows of two groups)."""
    assert _gi(N, K)
    t = pe.synth_tensor(N, K, 4, seed=K + 29)
    lut, idx = pe.unpack_payload(t.payload, N, K, 4)
    nc = K // 32
    first = 32 * ((nc + 7) // 8)
    ks = list(range(first)) + list(range(K - 64, K))
    w = gpu_ctx.upload_tensor(t)
    print(f"gi4 one-hot {N}x{K}: {len(ks)} columns", flush=True)
    x = np.zeros((1, K), dtype=np.float16)
    rows = np.arange(N)
    for k in ks:
        x[0, :] = 0
        x[0, k] = 1.0
        y = gpu_ctx.gemv(w, x.view(np.uint16))[0]
        want = lut[rows, idx[:, k]]
        want = np.where(want == 0x8000, 0, want)  # 0.0 + (-0.0) = +0.0
        bad = np.nonzero(y != want)[0]
        assert bad.size == 0, f"column {k}: {bad.size} rows differ (first {bad[:4]})"
    w.free()


@pytest.mark.parametrize("N,K", [(14336, 4096), (9100, 2048)])
def test_gi4_decode_bit_exact_through_lpr4m(pe, gpu_ctx, N, K):
    """One-hot x, a different column per vector, through the 4-bit
    lane-per-row lookups feeding the matrix cores (k_gemv_lpr4q at 3
    vectors, k_gemv_lpr4m at 8): every output is LUT_r[idx(r, k)] exactly.  The columns cover
    both lanes of a row (chunks 2s and 2s + 1), every MFMA of a step (index
    dwords 0..3 of a chunk), the K quarters' edges and the row's end."""
    t = pe.synth_tensor(N, K, 4, seed=K + 41)
    lut, idx = pe.unpack_payload(t.payload, N, K, 4)
    q = K // 4
    ks = [0, 1, 7, 8, 31, 32, 33, 63, 64 + 17, q - 1, q, K // 2 + 5, K - 33, K - 32, K - 9, K - 1]
    w = gpu_ctx.upload_tensor(t)
    print(f"gi4 one-hot lpr4m {N}x{K}", flush=True)
    rows = np.arange(N)
    for nb in (3, 8):
        for c0 in range(0, len(ks), nb):
            cols = ks[c0:c0 + nb]
            if len(cols) < 3:
                continue
            x = np.zeros((len(cols), K), dtype=np.float16)
            for v, k in enumerate(cols):
                x[v, k] = 1.0
            y = gpu_ctx.gemv(w, x.view(np.uint16))
            assert gpu_ctx.last_kernels() == ("k_gemv_lpr4m" if len(cols) > 4 else f"k_gemv_lpr4q<{K // 256}>")
            for v, k in enumerate(cols):
                want = lut[rows, idx[:, k]]
                want = np.where(want == 0x8000, 0, want)  # 0.0 + (-0.0) = +0.0
                bad = np.nonzero(y[v] != want)[0]
                assert bad.size == 0, f"column {k}, {len(cols)} vectors: {bad.size} rows differ"
    w.free()


@pytest.mark.parametrize("N,K", [(14336, 4096), (9100, 2048), (12000, 3328)])
def test_gi4_decode_bit_exact_through_lpr4q(pe, gpu_ctx, N, K):
    """One-hot x through k_gemv_lpr4q at 4 vectors (every block column
    live), a different column per vector: every element of the first wave's
    first chunk (all eight 4 x 4 x 4 steps, both halves of each step's A
    operand), then the first element of every chunk of a wave's range, the
    waves' edges and the row's end.  The one nonzero product is added to
    zeros, so each output is LUT_r[idx(r, k)] exactly."""
    t = pe.synth_tensor(N, K, 4, seed=K + 43)
    lut, idx = pe.unpack_payload(t.payload, N, K, 4)
    wk = K // 8  # elements of a wave's range
    ks = list(range(32)) + [32 * c for c in range(1, wk // 32)] + [wk - 1, wk, 3 * wk + 5, K - 33, K - 32, K - 2, K - 1]
    ks += [ks[-1]] * (-len(ks) % 4)
    w = gpu_ctx.upload_tensor(t)
    print(f"gi4 one-hot lpr4q {N}x{K}", flush=True)
    rows = np.arange(N)
    want_kernel = f"k_gemv_lpr4q<{K // 256 if K // 256 in (8, 16) else 0}>"
    for c0 in range(0, len(ks), 4):
        cols = ks[c0:c0 + 4]
        x = np.zeros((4, K), dtype=np.float16)
        for v, k in enumerate(cols):
            x[v, k] = 1.0
        y = gpu_ctx.gemv(w, x.view(np.uint16))
        assert gpu_ctx.last_kernels() == want_kernel
        for v, k in enumerate(cols):
            want = lut[rows, idx[:, k]]
            want = np.where(want == 0x8000, 0, want)  # 0.0 + (-0.0) = +0.0
            bad = np.nonzero(y[v] != want)[0]
            assert bad.size == 0, f"column {k}: {bad.size} rows differ (first {bad[:4]})"
    w.free()


@pytest.mark.parametrize("batch,kernel", [(3, "k_gemv_lpr4q<0>"), (4, "k_gemv_lpr4q<0>"), (5, "k_gemv_mfma<4, true>")])
def test_gi4_k8192_lpr4m_edge(pe, oracle, gpu_ctx, batch, kernel):
    """4-bit GI rows of 8192: 3 and 4 vectors of x (4 x 4100 dwords) fit the
    LDS of k_gemv_lpr4q (32 chunks per wave: its run-time loop), 5 do not
    and take the matrix-core GEMV; against the oracle."""
    N, K = 14336, 8192
    assert _gi(N, K) == 56
    t = pe.synth_tensor(N, K, 4, seed=K + batch + 4)
    x = pe.synth_x(batch, K, seed=batch + 44)
    w = gpu_ctx.upload_tensor(t)
    print(f"gi4 gemv {N}x{K} batch {batch}", flush=True)
    y = gpu_ctx.gemv(w, x)
    assert gpu_ctx.last_kernels() == kernel
    _check(y, oracle.gemv(x, t.payload, N, K, 4, threads=8), f"GI4 {N}x{K} batch {batch}")
    w.free()


@pytest.mark.parametrize("N,K,batch,kernel", [(9000, 2304, 5, "k_gemv_lpr4m"), (12000, 3328, 7, "k_gemv_lpr4m"),
                                              (16384, 2048, 4, "k_gemv_lpr4q<8>"), (9000, 2304, 3, "k_gemv_lpr4q<0>"),
                                              (12000, 3328, 4, "k_gemv_lpr4q<0>"), (16384, 2048, 6, "k_gemv_lpr4m")])
def test_gi4_lpr4m_row_lengths(pe, oracle, gpu_ctx, N, K, batch, kernel):
    """k_gemv_lpr4m where a wave's double steps are not a multiple of the
    four in flight (K = 2304: 9 per wave; 3328: 13), and over 64-row groups;
    k_gemv_lpr4q where a wave's chunks are not a multiple of its run-time
    loop's blocks of four (9, 13); against the oracle."""
    assert _gi(N, K) > 32
    t = pe.synth_tensor(N, K, 4, seed=N + K + batch)
    x = pe.synth_x(batch, K, seed=batch + 61)
    w = gpu_ctx.upload_tensor(t)
    print(f"gi4 {kernel} {N}x{K} batch {batch}", flush=True)
    y = gpu_ctx.gemv(w, x)
    assert gpu_ctx.last_kernels() == kernel
    _check(y, oracle.gemv(x, t.payload, N, K, 4, threads=8), f"GI4 {N}x{K} batch {batch}")
    w.free()


@pytest.mark.parametrize("N,K", [(14336, 4096), (8192, 2560)])
def test_gi8_decode_bit_exact_through_gemv(pe, gpu_ctx, N, K):
    """One-hot x: every output is LUT_r[idx(r, k)] exactly, through the
    8-bit lane-per-row GEMV at 1 and 2 vectors, its matrix-core form at 4 and
    8 and the matrix-core GEMV over GI (eleven vectors)."""
    t = pe.synth_tensor(N, K, 8, seed=K + 13)
    lut, idx = pe.unpack_payload(t.payload, N, K, 8)
    ks = [0, 1, 15, 16, 17, K // 2 + 5, K // 3, K - 17, K - 16, K - 2, K - 1]
    x = np.zeros((len(ks), K), dtype=np.float16)
    for i, k in enumerate(ks):
        x[i, k] = 1.0
    w = gpu_ctx.upload_tensor(t)
    print(f"gi8 one-hot {N}x{K}", flush=True)
    ys = gpu_ctx.gemv(w, x.view(np.uint16))
    y2 = gpu_ctx.gemv(w, x[:2].view(np.uint16))
    y4 = gpu_ctx.gemv(w, x[:4].view(np.uint16))
    y8 = gpu_ctx.gemv(w, x[:8].view(np.uint16))
    for i, k in enumerate(ks):
        want = lut[np.arange(N), idx[:, k]]
        want = np.where(want == 0x8000, 0, want)  # 0.0 + (-0.0) = +0.0
        y1 = gpu_ctx.gemv(w, x[i:i + 1].view(np.uint16))[0]
        assert np.array_equal(y1, want), f"column {k}, one vector"
        assert np.array_equal(ys[i], want), f"column {k}, eleven vectors"
        if i < 2:
            assert np.array_equal(y2[i], want), f"column {k}, two vectors"
        if i < 4:
            assert np.array_equal(y4[i], want), f"column {k}, four vectors (matrix cores fed by lookups)"
        if i < 8:
            assert np.array_equal(y8[i], want), f"column {k}, eight vectors (matrix cores fed by lookups)"
    w.free()


@pytest.mark.parametrize("N,K,batch", [(9000, 4608, 7), (9000, 6144, 5), (9000, 6144, 6), (12000, 2048, 6),
                                     (12000, 2048, 21)])
def test_gi8_lpr8m_row_lengths(pe, oracle, gpu_ctx, N, K, batch):
    """k_gemv_lpr8m at row lengths whose quarter is not a power of two
    (K = 4608: 36 double steps per wave; 6144: 48) and at the edge of its LDS
    (6 vectors of 6144 do not fit: the other kernels take them); 21 vectors
    of 2048: 16 on the matrix-core GEMV over GI, then 5 on k_gemv_lpr8m."""
    assert _gi(N, K, 8)
    t = pe.synth_tensor(N, K, 8, seed=N + K + batch)
    x = pe.synth_x(batch, K, seed=batch + 31)
    w = gpu_ctx.upload_tensor(t)
    print(f"gi8 lpr8m {N}x{K} batch {batch}", flush=True)
    y = gpu_ctx.gemv(w, x)
    _check(y, oracle.gemv(x, t.payload, N, K, 8, threads=8), f"GI8 {N}x{K} batch {batch}")
    w.free()


@pytest.mark.parametrize("N,K", [(14336, 4096), (9100, 2048)])
def test_gi8_unaligned_x_and_decode_rows(pe, oracle, gpu_ctx, N, K):
    """8-bit GI: x not 16-byte aligned takes the generic kernel; row decode
    and lut_embed are the oracle's bytes exactly (ragged last group too)."""
    import torch
    t = pe.synth_tensor(N, K, 8, seed=N - K + 8)
    x = pe.synth_x(2, K, seed=6)
    w = gpu_ctx.upload_tensor(t)
    buf = torch.zeros(2 * K + 8, dtype=torch.int16, device="cuda")
    buf[1:1 + 2 * K] = torch.from_numpy(x.reshape(-1).view(np.int16)).cuda()
    dy = torch.empty(2 * N, dtype=torch.int16, device="cuda")
    print(f"gi8 unaligned {N}x{K}", flush=True)
    gpu_ctx.gemv_dev(w, buf[1:], 2, dy)
    torch.cuda.synchronize()
    y = dy.cpu().numpy().view(np.uint16).reshape(2, N)
    _check(y, oracle.gemv(x, t.payload, N, K, 8, threads=8), f"GI8 {N}x{K} unaligned x")
    for r0, nr in [(0, 3), (63, 2), (N - 5, 5), (N // 2, 64)]:
        out = torch.empty(nr * K, dtype=torch.int16, device="cuda")
        gpu_ctx.decode_rows_dev(w, r0, nr, out)
        torch.cuda.synchronize()
        got = out.cpu().numpy().view(np.uint16).reshape(nr, K)
        want = oracle.decode_rows(t.payload, N, K, 8, r0, nr)
        assert np.array_equal(got, want), f"rows {r0}..{r0 + nr}"
    for tok in (0, 64, N - 1):
        assert np.array_equal(gpu_ctx.lut_embed(w, tok), oracle.decode_rows(t.payload, N, K, 8, tok, 1)[0])
    w.free()


@pytest.mark.parametrize("N,K", [(14336, 4096), (8192, 2560)])
def test_gi8_gateup_swiglu_and_upload_dev(pe, oracle, gpu_ctx, N, K):
    """8-bit GI gate/up with the SwiGLU epilogue against the oracle; a
    device-side payload regrouped like a host one."""
    import torch
    tg = pe.synth_tensor(N, K, 8, seed=N + 15)
    tu = pe.synth_tensor(N, K, 8, seed=N + 16)
    x = pe.synth_x(1, K, seed=N + 17)
    wg, wu = gpu_ctx.upload_tensor(tg), gpu_ctx.upload_tensor(tu)
    print(f"gi8 gate_up {N}x{K}", flush=True)
    y = gpu_ctx.gateup_swiglu(wg, wu, x)
    ref = oracle.gateup_swiglu(x[0], tg.payload, tu.payload, N, K, 8, threads=8)
    _check(y, ref, f"GI8 gate_up + SwiGLU {N}x{K}")
    dpay = torch.from_numpy(tg.payload.view(np.int8)).cuda()
    w_dev = gpu_ctx.upload_dev(dpay, N, K, 8)
    assert np.array_equal(gpu_ctx.gemv(wg, x), gpu_ctx.gemv(w_dev, x))
    for w in (wg, wu, w_dev):
        w.free()


@pytest.mark.parametrize("M", [24, 64, 200, 300])
def test_gi8_gemm(pe, oracle, gpu_ctx, M):
    """8-bit prefill GEMM over GI weights with a ragged last group (40-row
    groups, so a 128-row block spans four of them): GEMV passes (24 rows),
    split K (64, 200; 2048 / 64 = 32 K steps) and whole-K blocks (300);
    every row against the float32 product of the decoded weights, a spread
    of rows against the oracle."""
    N, K = 9100, 2048
    t = pe.synth_tensor(N, K, 8, seed=M + 80)
    X = pe.synth_x(M, K, seed=M + 81)
    w = gpu_ctx.upload_tensor(t)
    print(f"gi8 gemm M={M}", flush=True)
    Y = gpu_ctx.gemm(w, X)
    dense = oracle.decode_rows(t.payload, N, K, 8, 0, N).view(np.float16).astype(np.float32)
    Yf = X.view(np.float16).astype(np.float32) @ dense.T
    got = Y.view(np.float16).astype(np.float32)
    for m in range(M):
        err = np.max(np.abs(got[m] - Yf[m])) / np.max(np.abs(Yf[m]))
        assert err <= TOL, f"row {m}: {err:.3e}"
    rows = sorted(set([0, M // 3, M // 2, M - 1]))
    ref = oracle.gemm(np.ascontiguousarray(X[rows]), t.payload, N, K, 8, threads=8)
    for i, m in enumerate(rows):
        assert _rel(Y[m], ref[i]) <= TOL
    w.free()


@pytest.mark.parametrize("batch,kernel", [(1, "k_gemv_lpr8<8, 1, 1, 0, 64>"), (2, "k_gemv_lpr8<8, 1, 2, 0, 64>"),
                                          (3, "k_gemv_lpr8m"), (4, "k_gemv_lpr8m"),
                                          (5, "k_gemv_lpr8<8, 1, 8, 0, 64>"), (8, "k_gemv_lpr8<8, 1, 8, 0, 64>")])
def test_gi8_gemv_k8192(pe, oracle, gpu_ctx, batch, kernel):
    """8-bit GI with K = 8192: each wave's 64 chunks as a compile-time
    count.  1 and 2 vectors a pass, k_gemv_lpr8m at 3 and 4 (4 x 4100
    dwords of x fit its 16512-dword LDS), and the 8-vector form for 5..8
    (x of five 8192-element vectors, 5 x 4100 dwords, does not fit),
    against the oracle; the library's launch report names the kernel that
    ran."""
    N, K = 14336, 8192
    assert _gi(N, K, 8)
    t = pe.synth_tensor(N, K, 8, seed=K + batch)
    x = pe.synth_x(batch, K, seed=batch + 81)
    w = gpu_ctx.upload_tensor(t)
    print(f"gi8 gemv {N}x{K} batch {batch}", flush=True)
    y = gpu_ctx.gemv(w, x)
    assert gpu_ctx.last_kernels() == kernel
    _check(y, oracle.gemv(x, t.payload, N, K, 8, threads=8), f"GI8 {N}x{K} batch {batch}")
    w.free()


@pytest.mark.parametrize("batch,kernel", [(3, "k_gemv_lpr8m"), (4, "k_gemv_lpr8<8, 1, 4, 0, 0>")])
def test_gi8_wide_rows_three_four_vectors(pe, oracle, gpu_ctx, batch, kernel):
    """3 and 4 vectors of 8704-element rows: 3 x 4356 dwords of x fit
    k_gemv_lpr8m's LDS, 4 x 4356 do not, so 4 vectors take k_gemv_lpr8's
    4-vector pass in its run-time chunk loop (68 chunks per wave), the only
    shapes that reach that pass; against the oracle."""
    N, K = 8192, 8704
    assert _gi(N, K, 8)
    t = pe.synth_tensor(N, K, 8, seed=K + batch)
    x = pe.synth_x(batch, K, seed=batch + 87)
    w = gpu_ctx.upload_tensor(t)
    print(f"gi8 gemv {N}x{K} batch {batch}", flush=True)
    y = gpu_ctx.gemv(w, x)
    assert gpu_ctx.last_kernels() == kernel
    _check(y, oracle.gemv(x, t.payload, N, K, 8, threads=8), f"GI8 {N}x{K} batch {batch}")
    w.free()


def test_gi8_gate_up_k8192(pe, oracle, gpu_ctx):
    """8-bit GI gate/up at K = 8192 (k_gemv_lpr8 with two matrices and 64
    chunks per wave): the SwiGLU form against the oracle, the two-output
    form bit for bit against the separate GEMVs."""
    N, K = 14336, 8192
    tg = pe.synth_tensor(N, K, 8, seed=K + 21)
    tu = pe.synth_tensor(N, K, 8, seed=K + 22)
    x = pe.synth_x(1, K, seed=K + 23)
    wg, wu = gpu_ctx.upload_tensor(tg), gpu_ctx.upload_tensor(tu)
    print(f"gi8 gate_up {N}x{K}", flush=True)
    y = gpu_ctx.gateup_swiglu(wg, wu, x)
    assert gpu_ctx.last_kernels() == "k_gemv_lpr8<8, 2, 1, 1, 64>"
    _check(y, oracle.gateup_swiglu(x[0], tg.payload, tu.payload, N, K, 8, threads=8), "GI8 K=8192 SwiGLU")
    yg, yu = gpu_ctx.gate_up(wg, wu, x)
    assert gpu_ctx.last_kernels() == "k_gemv_lpr8<8, 2, 1, 2, 64>"
    assert np.array_equal(yg, gpu_ctx.gemv(wg, x)[0])
    assert np.array_equal(yu, gpu_ctx.gemv(wu, x)[0])
    _check(yg, oracle.gemv(x, tg.payload, N, K, 8, threads=8), "GI8 K=8192 gate")
    wg.free()
    wu.free()


def test_last_kernels_reports_the_dispatch(pe, gpu_ctx):
    """prism_hip_last_kernels names the hero's lane-per-row kernel, repeats
    as " x n" for passes, and is cleared by the next call."""
    N, K = 14336, 4096
    t = pe.synth_tensor(N, K, 4, seed=5)
    w = gpu_ctx.upload_tensor(t)
    gpu_ctx.gemv(w, pe.synth_x(1, K, seed=1))
    assert gpu_ctx.last_kernels() == "k_gemv_lpr<8, 1, 1, 0, 16>"
    gpu_ctx.gemv(w, pe.synth_x(2, K, seed=1))
    assert gpu_ctx.last_kernels() == "k_gemv_lpr<8, 1, 2, 0, 16>"
    gpu_ctx.gemv(w, pe.synth_x(40, K, seed=1))  # 16 + 16 on the matrix-core GEMV, 8 on k_gemv_lpr4m
    assert gpu_ctx.last_kernels() == "k_gemv_mfma<4, true> x2 + k_gemv_lpr4m"
    small = gpu_ctx.upload_tensor(pe.synth_tensor(4864, 896, 4, seed=6))
    gpu_ctx.gemv(small, pe.synth_x(1, 896, seed=1))
    assert gpu_ctx.last_kernels().startswith("k_gemv_tile<")
    w.free()
    small.free()
