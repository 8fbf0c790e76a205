"""Asynchronous uploads through the pinned staging ring (prism_hip_weight_
upload_async, prism_hip_ctx_synchronize, the keyed backend's add_tensor).

The device copy of each payload must equal the payload (the LUT decode of
every row is bit-exact against the host decode), whether the weight was
uploaded synchronously or asynchronously, with the payload overwritten
right after the call returned, and across more data than the ring holds
(4 slots of 16 MB), so every slot is reused while earlier copies may still
be in flight.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

# (N, K, bits): GI (hero, 56-row groups), split-block 4-bit, 8-bit, a payload of many ring
# slots, and tiny/ragged ones
SHAPES = [(14336, 4096, 4), (4864, 896, 4), (1000, 2048, 8), (18944, 3584, 4), (3, 100, 4), (7, 24, 8)]


def _x(pe, K, seed):
    return pe.synth_x(1, K, seed=seed)


def test_upload_async_equals_sync(pe, gpu_ctx):
    ts = [pe.synth_tensor(N, K, b, seed=N + K + b) for N, K, b in SHAPES]
    ws = [gpu_ctx.upload_async(t.payload, t.dim_m, t.dim_n, t.bits) for t in ts]
    gpu_ctx.synchronize()
    for t, w in zip(ts, ws):
        ref = gpu_ctx.upload(t.payload, t.dim_m, t.dim_n, t.bits)
        x = _x(pe, t.dim_n, t.dim_m)
        print(f"[upload] {t.dim_m}x{t.dim_n} {t.bits}-bit", flush=True)
        assert np.array_equal(gpu_ctx.gemv(w, x), gpu_ctx.gemv(ref, x))
        ref.free()
        w.free()


def test_upload_async_consumes_payload_before_return(pe, gpu_ctx):
    """Overwriting the host payload right after the call does not change the
    device copy (it was staged before the call returned)."""
    N, K = 14336, 4096
    t = pe.synth_tensor(N, K, 4, seed=77)
    keep = t.payload.copy()
    w = gpu_ctx.upload_async(t.payload, N, K, 4)
    t.payload[:] = 0
    gpu_ctx.synchronize()
    ref = gpu_ctx.upload(keep, N, K, 4)
    for row in (0, 1, 8191, N - 1):
        assert np.array_equal(gpu_ctx.lut_embed(w, row), gpu_ctx.lut_embed(ref, row)), f"row {row}"
    x = _x(pe, K, 5)
    assert np.array_equal(gpu_ctx.gemv(w, x), gpu_ctx.gemv(ref, x))
    w.free()
    ref.free()


def test_upload_async_ring_wraps(pe, oracle, gpu_ctx):
    """Eight 29.8 MB tensors (15 ring slots' worth) uploaded back to back,
    each from a buffer reused for the next: every device copy decodes to
    its own payload."""
    N, K = 14336, 4096
    buf = np.empty(N * 32 + N * K // 2, dtype=np.uint8)
    ws, seeds = [], list(range(900, 908))
    for s in seeds:
        buf[:] = pe.synth_tensor(N, K, 4, seed=s).payload
        ws.append(gpu_ctx.upload_async(buf, N, K, 4))
    gpu_ctx.synchronize()
    for s, w in zip(seeds, ws):
        t = pe.synth_tensor(N, K, 4, seed=s)
        for row in (0, 4097, N - 1):
            got = gpu_ctx.lut_embed(w, row)
            ref = oracle.lut_embed(row, t.payload, N, K)
            assert np.array_equal(got, ref), f"seed {s} row {row}"
        w.free()


def test_backend_uploads_then_synchronize(pe, gpu_ctx):
    """The keyed backend uploads asynchronously; its own calls see the data
    (same stream) and synchronize() returns cleanly."""
    b = pe.HipBackend(0)
    ts = [pe.synth_tensor(N, K, bits, seed=N * 3 + K, key=f"t{i}") for i, (N, K, bits) in enumerate(SHAPES[:3])]
    for t in ts:
        b.add_tensor(t.key, t.payload, t.dim_m, t.dim_n, t.bits)
    for t in ts:
        x = _x(pe, t.dim_n, 11)
        want = gpu_ctx.gemv(gpu_ctx.upload_tensor(t), x)
        assert np.array_equal(b.gemv(t.key, x, dim_m=t.dim_m).reshape(want.shape), want)
    b.synchronize()
    b.close()


def test_weight_chunks_and_lifetimes(pe, gpu_ctx):
    """Weights carved out of shared device chunks (8, 16, 32, 64 MB; over
    16 MB a chunk of their own): freeing some, uploading more and
    destroying the context leave every live weight's bytes intact, and
    weights that outlive their context can still be freed."""
    ctx = pe.Context(0)
    shapes = [(896, 896), (4864, 896), (896, 4864), (128, 896), (1000, 2048), (151, 4000), (3, 100)] * 6
    shapes.insert(5, (14336, 4096))  # 29.8 MB: its own chunk
    ts = [pe.synth_tensor(N, K, 4, seed=i * 7 + N) for i, (N, K) in enumerate(shapes)]
    ws = [ctx.upload_tensor(t) for t in ts]
    xs = [pe.synth_x(1, t.dim_n, seed=i) for i, t in enumerate(ts)]
    ys = [ctx.gemv(w, x) for w, x in zip(ws, xs)]
    print(f"[chunks] {len(ws)} weights, {sum(t.payload.nbytes for t in ts) / 1e6:.1f} MB", flush=True)
    for i in range(0, len(ws), 2):  # free every other weight
        ws[i].free()
    more = [ctx.upload_tensor(pe.synth_tensor(N, K, 4, seed=1000 + i)) for i, (N, K) in enumerate(shapes[:12])]
    for i in range(1, len(ws), 2):
        assert np.array_equal(ctx.gemv(ws[i], xs[i]), ys[i]), f"weight {i} changed"
    half = len(ws) // 2 | 1  # an odd index: the weights still live are the odd ones
    for i in range(1, half, 2):  # free the first chunks' remaining weights
        ws[i].free()
    for i in range(half, len(ws), 2):
        assert np.array_equal(ctx.gemv(ws[i], xs[i]), ys[i]), f"weight {i} changed after chunk frees"
    ctx.close()  # weights outlive it
    for w in more + ws:
        w.free()


@pytest.mark.parametrize("N,K,bits", [(9100, 2048, 4), (6000, 3072, 4), (10000, 896, 8)])
def test_first_weight_larger_than_first_chunk(pe, oracle, gpu_ctx, N, K, bits):
    """A fresh context's first weight between the first chunk size (8 MB)
    and the own-chunk limit (16 MB) gets a chunk that holds it (it once got
    an 8 MB chunk and was written past its end); the next small weight
    carves after it.  Both match the oracle."""
    ctx = pe.Context(0)
    try:
        t = pe.synth_tensor(N, K, bits, seed=N + K)
        t2 = pe.synth_tensor(896, 896, 4, seed=3)
        print(f"[first chunk] {N}x{K} {bits}-bit, {t.payload.nbytes / 1e6:.2f} MB", flush=True)
        w = ctx.upload_tensor(t)
        w2 = ctx.upload_tensor(t2)
        for tt, ww in ((t, w), (t2, w2)):
            x = pe.synth_x(1, tt.dim_n, seed=tt.dim_m)
            y = ctx.gemv(ww, x)
            ref = oracle.gemv(x, tt.payload, tt.dim_m, tt.dim_n, tt.bits, threads=8)
            err = pe.rel_err(y[0], ref[0])  # on the fp16 values, not their bit patterns
            assert err <= 2e-3, f"{tt.dim_m}x{tt.dim_n}: rel_err {err:.3e}"
        w2.free()
        w.free()
    finally:
        ctx.close()


def test_replacing_a_key_does_not_grow_device_memory(pe, gpu_ctx):
    """Weight memory comes back when a chunk's last weight is freed: a key
    replaced 150 times in a HipBackend (each upload carved from the current
    chunk, the replaced weight freed), next to a weight kept for the whole
    loop, grows device memory by at most the chunks it can pin (the kept
    weight's chunk and the current one, 64 MB each at most), not by the
    150 uploads (345 MB)."""
    import torch
    b = pe.HipBackend(0)
    keep = pe.synth_tensor(4864, 896, 4, seed=1)
    tmp = pe.synth_tensor(4864, 896, 4, seed=2)
    b.add_tensor("keep", keep.payload, 4864, 896, 4)
    b.synchronize()
    torch.cuda.synchronize()
    free0 = torch.cuda.mem_get_info()[0]
    for i in range(150):
        b.add_tensor("tmp", tmp.payload, 4864, 896, 4)
    b.synchronize()
    grown = free0 - torch.cuda.mem_get_info()[0]
    print(f"[replace] device memory grew by {grown / 1e6:.1f} MB over 150 replacements", flush=True)
    assert grown <= 3 * (64 << 20), f"grew {grown / 1e6:.1f} MB"
    x = pe.synth_x(1, 896, seed=3)
    y = np.zeros(4864, dtype=np.uint16)
    b.gemv("tmp", x[0], y)
    w = gpu_ctx.upload_tensor(tmp)
    assert np.array_equal(y, gpu_ctx.gemv(w, x)[0])
    w.free()
    b.close()
