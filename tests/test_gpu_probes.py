"""The measuring sticks (measure_kernels.hpp; no counterpart in the
reference): the read floor, the empty kernel and the register-only MFMA
probe run through the C ABI, write nothing to their sinks, name their
kernels, and reject what they cannot take."""
import pytest

pytestmark = pytest.mark.gpu


def test_probes_run_and_write_nothing(gpu_ctx):
    import torch
    sink = torch.zeros(256, dtype=torch.float32, device="cuda")
    buf = torch.randint(0, 256, (1 << 20,), dtype=torch.uint8, device="cuda")
    print("probes: read floor, empty kernel, MFMA probe", flush=True)
    gpu_ctx.stream_read_dev(buf, buf.numel(), sink)
    assert gpu_ctx.last_kernels() == "k_stream_read"
    gpu_ctx.launch_empty_dev()
    assert gpu_ctx.last_kernels() == "k_launch_empty"
    gpu_ctx.mfma_probe_dev(8, 16, sink)
    assert gpu_ctx.last_kernels() == "k_mfma_probe"
    torch.cuda.synchronize()
    assert int(torch.count_nonzero(sink)) == 0


def test_mfma_probe_rejects_bad_sizes(pe, gpu_ctx):
    import torch
    sink = torch.zeros(256, dtype=torch.float32, device="cuda")
    with pytest.raises(pe.PrismHipError):
        gpu_ctx.mfma_probe_dev(0, 16, sink)
    with pytest.raises(pe.PrismHipError):
        gpu_ctx.mfma_probe_dev(65537, 16, sink)
    lib = gpu_ctx.lib
    assert lib.prism_hip_mfma_probe_dev(gpu_ctx.h, 8, 16, None, None) != 0
    assert lib.prism_hip_launch_empty_dev(None, None) != 0


def test_issue_probe_runs_names_and_rejects(pe, gpu_ctx):
    """k_issue_probe at every instruction kind and occupancy: runs, names its
    instantiation, writes nothing; bad kinds, occupancies and sizes are
    rejected before any launch."""
    import torch
    sink = torch.zeros(256, dtype=torch.float32, device="cuda")
    print("probes: issue rates", flush=True)
    for op in range(4):
        for wps in (1, 2, 4):
            gpu_ctx.issue_probe_dev(op, 8, wps, 16, sink)
            assert gpu_ctx.last_kernels() == f"k_issue_probe<{op}>"
    torch.cuda.synchronize()
    assert int(torch.count_nonzero(sink)) == 0
    for bad in ((4, 8, 1), (0, 8, 3), (0, 0, 1), (0, 65537, 1)):
        with pytest.raises(pe.PrismHipError):
            gpu_ctx.issue_probe_dev(bad[0], bad[1], bad[2], 16, sink)
    assert gpu_ctx.lib.prism_hip_issue_probe_dev(gpu_ctx.h, 0, 8, 1, 16, None, None) != 0
