"""ctypes binding of libprism_hip.so (the C ABI in include/prism_hip.h).

The library is built in-tree by ``__graft_entry__.build()`` (``make -C
prism-engine_amd/csrc``).  Loading fails loudly when it is missing: there is
no CPU fallback anywhere in this package.
"""
from __future__ import annotations

import ctypes
import os
import re

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libprism_hip.so")
HEADER_PATH = os.path.join(os.path.dirname(HERE), "include", "prism_hip.h")

OK = 0
ERR_NULL = -1
ERR_NOT_LINKED = -2
ERR_SHAPE = -3
ERR_BITS = -4
ERR_SIZE = -5
ERR_LAYOUT = -6
ERR_DEVICE = -7
ERR_MISMATCH = -8
ERR_KEY = -9
ERR_CONTEXT = -10
LAYOUT_SPLIT_BLOCK = 0

_c = ctypes
_vp = _c.c_void_p
_u8p = _c.POINTER(_c.c_uint8)
_u16p = _c.POINTER(_c.c_uint16)
_u32p = _c.POINTER(_c.c_uint32)
_szp = _c.POINTER(_c.c_size_t)



class ModelConfig(ctypes.Structure):
    """prism_hip_model_config (include/prism_hip.h)."""
    _fields_ = [("n_layers", ctypes.c_uint32), ("hidden", ctypes.c_uint32), ("n_heads", ctypes.c_uint32),
                ("n_kv_heads", ctypes.c_uint32), ("head_dim", ctypes.c_uint32), ("intermediate", ctypes.c_uint32),
                ("vocab", ctypes.c_uint32), ("max_seq", ctypes.c_uint32), ("rms_eps", ctypes.c_float),
                ("rope_theta", ctypes.c_float)]


_cfgp = ctypes.POINTER(ModelConfig)

# name -> (restype, argtypes); must cover every function in prism_hip.h
SIGNATURES = {
    "prism_hip_ctx_create": (_vp, [_c.c_int]),
    "prism_hip_ctx_destroy": (None, [_vp]),
    "prism_hip_last_error": (_c.c_char_p, [_vp]),
    "prism_hip_version": (_c.c_char_p, []),
    "prism_hip_weight_upload": (_vp, [_vp, _vp, _c.c_size_t, _c.c_uint32, _c.c_uint32, _c.c_uint32, _c.c_uint32]),
    "prism_hip_weight_upload_dev": (_vp, [_vp, _vp, _c.c_size_t, _c.c_uint32, _c.c_uint32, _c.c_uint32,
                                          _c.c_uint32]),
    "prism_hip_weight_upload_async": (_vp, [_vp, _vp, _c.c_size_t, _c.c_uint32, _c.c_uint32, _c.c_uint32,
                                            _c.c_uint32]),
    "prism_hip_ctx_synchronize": (_c.c_int, [_vp]),
    "prism_hip_weight_free": (None, [_vp]),
    "prism_hip_weight_info": (_c.c_int, [_vp, _u32p, _u32p, _u32p, _szp]),
    "prism_hip_gemv": (_c.c_int, [_vp, _vp, _vp, _c.c_uint32, _vp]),
    "prism_hip_gemv_dev": (_c.c_int, [_vp, _vp, _vp, _c.c_uint32, _vp, _vp]),
    "prism_hip_gateup_swiglu": (_c.c_int, [_vp, _vp, _vp, _vp, _vp]),
    "prism_hip_gateup_swiglu_dev": (_c.c_int, [_vp, _vp, _vp, _vp, _vp, _vp]),
    "prism_hip_gate_up": (_c.c_int, [_vp, _vp, _vp, _vp, _vp, _vp]),
    "prism_hip_gate_up_dev": (_c.c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "prism_hip_gemm": (_c.c_int, [_vp, _vp, _vp, _c.c_uint32, _vp]),
    "prism_hip_gemm_dev": (_c.c_int, [_vp, _vp, _vp, _c.c_uint32, _vp, _vp]),
    "prism_hip_gemm_dev_noalloc": (_c.c_int, [_vp, _vp, _vp, _c.c_uint32, _vp, _vp]),
    "prism_hip_lut_embed": (_c.c_int, [_vp, _vp, _c.c_uint32, _vp]),
    "prism_hip_decode_rows_dev": (_c.c_int, [_vp, _vp, _c.c_uint32, _c.c_uint32, _vp, _vp]),
    "prism_hip_palettize_bytes": (_c.c_size_t, [_c.c_uint32, _c.c_uint32]),
    "prism_hip_palettize": (_c.c_int, [_vp, _vp, _c.c_uint32, _c.c_uint32, _c.c_uint32, _c.c_uint32, _vp,
                                       _c.c_uint32, _vp]),
    "prism_hip_palettize_dev": (_c.c_int, [_vp, _vp, _c.c_uint32, _c.c_uint32, _c.c_uint32, _c.c_uint32, _vp,
                                           _c.c_uint32, _vp, _vp]),
    "prism_hip_backend_new": (_vp, [_c.c_int]),
    "prism_hip_backend_free": (None, [_vp]),
    "prism_hip_backend_last_error": (_c.c_char_p, [_vp]),
    "prism_hip_backend_add_tensor": (_c.c_int, [_vp, _c.c_char_p, _vp, _c.c_size_t, _c.c_uint32, _c.c_uint32,
                                                _c.c_uint32]),
    "prism_hip_backend_gemv": (_c.c_int, [_vp, _c.c_char_p, _vp, _c.c_size_t, _vp, _c.c_size_t]),
    "prism_hip_backend_fused_gate_up": (_c.c_int, [_vp, _c.c_char_p, _c.c_char_p, _vp, _c.c_size_t, _vp,
                                                   _c.c_size_t]),
    "prism_hip_backend_gemm": (_c.c_int, [_vp, _c.c_char_p, _vp, _c.c_uint32, _vp]),
    "prism_hip_backend_embed": (_c.c_int, [_vp, _c.c_char_p, _c.c_uint32, _vp, _c.c_size_t]),
    "prism_hip_backend_len": (_c.c_size_t, [_vp]),
    "prism_hip_backend_synchronize": (_c.c_int, [_vp]),
    "prism_hip_model_create": (_vp, [_vp, _cfgp]),
    "prism_hip_model_free": (None, [_vp]),
    "prism_hip_model_set_embedding": (_c.c_int, [_vp, _vp]),
    "prism_hip_model_set_layer": (_c.c_int, [_vp, _c.c_uint32, _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "prism_hip_model_kv_append": (_c.c_int, [_vp, _c.c_uint32, _vp, _vp, _c.c_uint32]),
    "prism_hip_model_kv_len": (_c.c_int, [_vp, _c.c_uint32, _u32p]),
    "prism_hip_model_kv_read": (_c.c_int, [_vp, _c.c_uint32, _vp, _vp]),
    "prism_hip_model_kv_reset": (_c.c_int, [_vp]),
    "prism_hip_model_kv_truncate": (_c.c_int, [_vp, _c.c_uint32]),
    "prism_hip_model_step": (_c.c_int, [_vp, _c.c_uint32, _c.c_int64, _vp]),
    "prism_hip_model_step_dev": (_c.c_int, [_vp, _c.c_uint32, _c.c_int64, _vp]),
    "prism_hip_model_logits_dev": (_vp, [_vp]),
    "prism_hip_stream_read_dev": (_c.c_int, [_vp, _vp, _c.c_size_t, _vp, _vp]),
    "prism_hip_launch_empty_dev": (_c.c_int, [_vp, _vp]),
    "prism_hip_mfma_probe_dev": (_c.c_int, [_vp, _c.c_uint32, _c.c_uint32, _vp, _vp]),
    "prism_hip_issue_probe_dev": (_c.c_int, [_vp, _c.c_uint32, _c.c_uint32, _c.c_uint32, _c.c_uint32, _vp, _vp]),
    "prism_hip_last_kernels": (_c.c_char_p, [_vp]),
}

_lib = None


class PrismHipError(RuntimeError):
    """A negative result code from the C ABI, with the library's error text."""

    def __init__(self, code: int, message: str):
        super().__init__(f"[{code}] {message}")
        self.code = code
        self.message = message


def header_functions(path: str = HEADER_PATH) -> list[str]:
    """Names of the functions declared in include/prism_hip.h."""
    text = open(path).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(prism_hip_\w+)\s*\(", text)))


def load():
    """Load libprism_hip.so; raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(
            f"HIP extension {LIB_PATH} is missing: build it with `python -c 'import __graft_entry__ as g; "
            f"g.build()'` (there is no CPU fallback)")
    lib = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        f = getattr(lib, name)
        f.restype = res
        f.argtypes = args
    _lib = lib
    return lib


def ptr(a) -> int:
    """Address of a numpy array or torch tensor's data."""
    if hasattr(a, "data_ptr"):
        return a.data_ptr()
    return a.ctypes.data
