"""prism_hip_gemm_dev_noalloc (the GEMM entry point that allocates nothing)
against prism_hip_gemm_dev, through the C ABI.

Both run the same kernels with the same split-K plan; only where the fp32
partials live differs (the library's static per-GPU scratch instead of the
context's pool), so the outputs must be bit-identical.  Each case makes two
calls in a row, the second with fewer rows of X, so a stale first call's
partials in the shared scratch would show in the second.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

# (bits, N, K, M first call, M second call): split-K 4-bit (4 and 2 splits),
# GI and split-block device layouts, split-K 8-bit, an unsplit prefill and
# the GEMV path (no partials at all).
CASES = [
    (4, 14336, 4096, 256, 64),
    (4, 2000, 2048, 200, 96),
    (4, 4864, 896, 128, 40),
    (8, 14336, 4096, 200, 65),
    (4, 4096, 1024, 600, 520),
    (4, 1024, 512, 24, 9),
]


@pytest.mark.parametrize("bits,N,K,M1,M2", CASES)
def test_gemm_noalloc_matches_gemm_dev(pe, gpu_ctx, bits, N, K, M1, M2):
    import torch
    print(f"[no_alloc] bits={bits} N={N} K={K} M={M1},{M2}", flush=True)
    t = pe.synth_tensor(N, K, bits, seed=N + K + bits)
    w = gpu_ctx.upload_tensor(t)
    s = torch.cuda.Stream()
    for i, M in enumerate((M1, M2)):
        X = pe.synth_x(M, K, seed=100 * i + M)
        dX = torch.from_numpy(X.view(np.int16)).cuda()
        want = torch.full((M, N), -1, dtype=torch.int16, device="cuda")
        got = torch.full((M, N), -2, dtype=torch.int16, device="cuda")
        torch.cuda.synchronize()
        gpu_ctx.gemm_dev(w, dX, M, want, s)
        gpu_ctx.gemm_dev_noalloc(w, dX, M, got, s)
        s.synchronize()
        a = want.cpu().numpy()
        b = got.cpu().numpy()
        assert np.array_equal(a, b), (f"call {i}: M={M}: {int(np.sum(a != b))} of {a.size} outputs differ "
                                      "from prism_hip_gemm_dev")
    w.free()


def test_gemm_noalloc_errors(pe, gpu_ctx):
    """NULL buffers are rejected like prism_hip_gemm_dev's; M = 0 is a no-op."""
    import torch
    t = pe.synth_tensor(256, 512, 4, seed=3)
    w = gpu_ctx.upload_tensor(t)
    dX = torch.zeros((64, 512), dtype=torch.int16, device="cuda")
    with pytest.raises(pe.PrismHipError):
        rc = gpu_ctx.lib.prism_hip_gemm_dev_noalloc(gpu_ctx.h, w.h, None, 64, None, None)
        gpu_ctx.check(rc)
    gpu_ctx.gemm_dev_noalloc(w, dX, 0, dX)
    torch.cuda.synchronize()
    w.free()


def test_gemm_noalloc_replayed_from_a_hip_graph(pe, gpu_ctx):
    """The no-alloc GEMM captured in a HIP graph: the split-K path (4-bit
    14336 x 4096, M = 64: k_gemm_w4 in 4 K splits writing the static
    scratch, then k_gemm_split_sum) makes no call that capture rejects, and
    every replay, each with new X copied in eagerly between replays,
    equals prism_hip_gemm_dev on the same X bit for bit."""
    import torch
    N, K, M = 14336, 4096, 64
    t = pe.synth_tensor(N, K, 4, seed=404)
    w = gpu_ctx.upload_tensor(t)
    s = torch.cuda.Stream()
    dX = torch.from_numpy(pe.synth_x(M, K, seed=1).view(np.int16)).cuda()
    dY = torch.zeros((M, N), dtype=torch.int16, device="cuda")
    want = torch.zeros_like(dY)
    torch.cuda.synchronize()
    print("[no_alloc graph] eager call", flush=True)
    gpu_ctx.gemm_dev_noalloc(w, dX, M, dY, s)  # first call looks up the scratch address
    s.synchronize()
    assert "k_gemm_split_sum" in gpu_ctx.last_kernels()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        gpu_ctx.gemm_dev_noalloc(w, dX, M, dY, s)
    torch.cuda.synchronize()
    for i in range(3):
        print(f"[no_alloc graph] replay {i}", flush=True)
        dX.copy_(torch.from_numpy(pe.synth_x(M, K, seed=10 + i).view(np.int16)))
        dY.fill_(-1)
        torch.cuda.synchronize()
        with torch.cuda.stream(s):
            g.replay()
        s.synchronize()
        gpu_ctx.gemm_dev(w, dX, M, want, s)
        s.synchronize()
        a, b = want.cpu().numpy(), dY.cpu().numpy()
        assert np.array_equal(a, b), f"replay {i}: {int(np.sum(a != b))} of {a.size} outputs differ"
    del g
    w.free()
