"""The C-ABI library loads and exports every symbol include/prism_hip.h
declares; calls that need no GPU behave per the contract (NULL handling,
no-device errors).  No compute calls here."""
import ctypes
import subprocess

import pytest


def test_header_declares_the_boundary(pe):
    names = pe.header_functions()
    for must in ("prism_hip_ctx_create", "prism_hip_weight_upload", "prism_hip_gemv", "prism_hip_gemv_dev",
                 "prism_hip_gateup_swiglu", "prism_hip_gemm", "prism_hip_lut_embed", "prism_hip_last_error",
                 "prism_hip_backend_gemv", "prism_hip_backend_fused_gate_up"):
        assert must in names


def test_library_exports_every_header_symbol(pe):
    lib = pe.load_library()
    from importlib import import_module
    native = import_module("prism-engine_amd._native")
    names = pe.header_functions()
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    # the ctypes signature table covers the whole header
    assert sorted(native.SIGNATURES) == names
    out = subprocess.run(["nm", "-D", "--defined-only", native.LIB_PATH], capture_output=True, text=True,
                         check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if line.strip()}
    assert set(names) <= exported


def test_null_handling_without_gpu(pe):
    lib = pe.load_library()
    assert lib.prism_hip_version().startswith(b"prism_hip")
    lib.prism_hip_ctx_destroy(None)
    lib.prism_hip_weight_free(None)
    lib.prism_hip_backend_free(None)
    assert lib.prism_hip_gemv(None, None, None, 1, None) == -1
    assert lib.prism_hip_gemv_dev(None, None, None, 1, None, None) == -1
    assert lib.prism_hip_gateup_swiglu(None, None, None, None, None) == -1
    assert lib.prism_hip_gemm(None, None, None, 1, None) == -1
    assert lib.prism_hip_lut_embed(None, None, 0, None) == -1
    assert lib.prism_hip_weight_info(None, None, None, None, None) == -1
    assert lib.prism_hip_backend_gemv(None, b"k", None, 0, None, 0) == -1
    assert lib.prism_hip_backend_len(None) == 0
    assert lib.prism_hip_weight_upload(None, None, 0, 1, 8, 4, 0) is None
    assert lib.prism_hip_last_kernels(None) == b""


def test_ctx_create_reports_error_when_no_gpu(pe):
    import torch
    if torch.cuda.is_available():
        pytest.skip("GPU present")
    lib = pe.load_library()
    assert lib.prism_hip_ctx_create(0) is None
    assert len(lib.prism_hip_last_error(None)) > 0
    assert lib.prism_hip_backend_new(0) is None
    assert len(lib.prism_hip_backend_last_error(None)) > 0


def test_library_has_gfx950_code_object(pe):
    """The in-tree build carries a gfx950 device code object (offload bundle id)."""
    from importlib import import_module
    native = import_module("prism-engine_amd._native")
    with open(native.LIB_PATH, "rb") as f:
        blob = f.read()
    assert b"amdgcn-amd-amdhsa--gfx950" in blob
