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
