"""CPU oracle for the palettized-LUT contraction -- TEST INFRASTRUCTURE ONLY.

ctypes bindings to ``libprism_cpuref.so`` (built from ``prism_cpuref.c`` by
``oracle/Makefile``).  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this module, and only as the
checker.  The product (``prism-engine_amd``) never imports it and has no CPU
fallback.

Each function cites the reference function it restates; the C file holds the
full list.  Parity status per function (what pins it):

* ``f16_to_f32`` / ``f32_to_f16``: numpy float16 casts (exhaustive for
  f16->f32, edge cases plus 10^6 random floats for f32->f16) -- pinned.
* ``lut_gemv4``: reference KAT evaluator.rs:231-246, closed forms (constant
  LUT, one-hot x), float64 error bound, brute force -- pinned.
* ``lut_gemv8``, ``gemv_batch``, ``gemm``: build extensions with no reference
  implementation; pinned by closed forms, brute force and float64 bound.
* ``silu``/``swiglu``: KAT evaluator.rs:286-298 and numpy float32 closed form.
* ``lut_embed`` / ``decode_rows``: KAT evaluator.rs:267-284, nibble-order KAT
  palette.rs:410-425 and numpy unpack -- pinned.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libprism_cpuref.so")
_lib = None

_u16p = ctypes.POINTER(ctypes.c_uint16)
_u8p = ctypes.POINTER(ctypes.c_uint8)


def build() -> str:
    """Compile libprism_cpuref.so with oracle/Makefile (always rebuilds)."""
    subprocess.run(["make", "-B", "-C", _HERE, "libprism_cpuref.so"], check=True,
                   stdout=subprocess.DEVNULL)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        L.cpuref_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.cpuref_f16_to_f32.restype = ctypes.c_float
        L.cpuref_f32_to_f16.argtypes = [ctypes.c_float]
        L.cpuref_f32_to_f16.restype = ctypes.c_uint16
        for name in ("cpuref_lut_gemv4", "cpuref_lut_gemv8"):
            f = getattr(L, name)
            f.argtypes = [_u16p, _u8p, ctypes.c_uint32, ctypes.c_uint32, _u16p]
            f.restype = None
        for name in ("cpuref_lut_gemv4_mt", "cpuref_lut_gemv8_mt"):
            f = getattr(L, name)
            f.argtypes = [_u16p, _u8p, ctypes.c_uint32, ctypes.c_uint32, _u16p, ctypes.c_int]
            f.restype = None
        L.cpuref_gemv_batch.argtypes = [_u16p, ctypes.c_uint32, _u8p, ctypes.c_uint32, ctypes.c_uint32,
                                        ctypes.c_uint32, _u16p]
        L.cpuref_gemv_batch.restype = ctypes.c_int
        L.cpuref_gemm.argtypes = [_u16p, ctypes.c_uint32, _u8p, ctypes.c_uint32, ctypes.c_uint32,
                                  ctypes.c_uint32, _u16p, ctypes.c_int]
        L.cpuref_gemm.restype = ctypes.c_int
        L.cpuref_silu_inplace.argtypes = [_u16p, ctypes.c_size_t]
        L.cpuref_silu_inplace.restype = None
        L.cpuref_swiglu.argtypes = [_u16p, _u16p, ctypes.c_size_t]
        L.cpuref_swiglu.restype = None
        L.cpuref_gateup_swiglu.argtypes = [_u16p, _u8p, _u8p, ctypes.c_uint32, ctypes.c_uint32,
                                           ctypes.c_uint32, _u16p, _u16p, ctypes.c_int]
        L.cpuref_gateup_swiglu.restype = ctypes.c_int
        L.cpuref_lut_embed.argtypes = [ctypes.c_uint32, _u8p, ctypes.c_uint32, ctypes.c_uint32, _u16p]
        L.cpuref_lut_embed.restype = None
        L.cpuref_decode_rows.argtypes = [_u8p, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32,
                                         ctypes.c_uint32, ctypes.c_uint32, _u16p]
        L.cpuref_decode_rows.restype = ctypes.c_int
        _lib = L
    return _lib


def _p16(a: np.ndarray):
    assert a.dtype == np.uint16 and a.flags.c_contiguous
    return a.ctypes.data_as(_u16p)


def _p8(a: np.ndarray):
    assert a.dtype == np.uint8 and a.flags.c_contiguous
    return a.ctypes.data_as(_u8p)


def _bits16(x) -> np.ndarray:
    x = np.ascontiguousarray(x)
    if x.dtype == np.float16:
        x = x.view(np.uint16)
    assert x.dtype == np.uint16
    return x


def f16_to_f32(h: int) -> float:
    return float(lib().cpuref_f16_to_f32(h))


def f32_to_f16(f: float) -> int:
    return int(lib().cpuref_f32_to_f16(ctypes.c_float(f)))


def lut_gemv4(x, payload: np.ndarray, dm: int, dn: int, threads: int = 1) -> np.ndarray:
    """lut_gemv_cpu (compute-core/src/lut/evaluator.rs:21-44); returns fp16 bits [dm]."""
    x = _bits16(x)
    assert x.size >= (dn // 8) * 8
    out = np.zeros(dm, dtype=np.uint16)
    if threads > 1:
        lib().cpuref_lut_gemv4_mt(_p16(x), _p8(payload), dm, dn, _p16(out), threads)
    else:
        lib().cpuref_lut_gemv4(_p16(x), _p8(payload), dm, dn, _p16(out))
    return out


def lut_gemv8(x, payload: np.ndarray, dm: int, dn: int, threads: int = 1) -> np.ndarray:
    """8-bit generalisation of lut_gemv_cpu (build extension)."""
    x = _bits16(x)
    assert x.size >= dn
    out = np.zeros(dm, dtype=np.uint16)
    if threads > 1:
        lib().cpuref_lut_gemv8_mt(_p16(x), _p8(payload), dm, dn, _p16(out), threads)
    else:
        lib().cpuref_lut_gemv8(_p16(x), _p8(payload), dm, dn, _p16(out))
    return out


def gemv(x, payload, dm, dn, bits, threads: int = 1) -> np.ndarray:
    """B independent GEMVs; x is [B, dn] (or [dn]); returns [B, dm] fp16 bits."""
    x = _bits16(x)
    xb = x.reshape(-1, dn)
    out = np.zeros((xb.shape[0], dm), dtype=np.uint16)
    f = lut_gemv4 if bits == 4 else lut_gemv8
    for b in range(xb.shape[0]):
        out[b] = f(np.ascontiguousarray(xb[b]), payload, dm, dn, threads)
    return out


def gemm(X, payload, dm, dn, bits, threads: int = 1) -> np.ndarray:
    """Y[M, dm] = X[M, dn] . W^T as M independent lut_gemv_cpu rows."""
    X = _bits16(X).reshape(-1, dn)
    X = np.ascontiguousarray(X)
    Y = np.zeros((X.shape[0], dm), dtype=np.uint16)
    rc = lib().cpuref_gemm(_p16(X), X.shape[0], _p8(payload), dm, dn, bits, _p16(Y), threads)
    assert rc == 0
    return Y


def silu(v) -> np.ndarray:
    """silu_inplace (evaluator.rs:78-83) on a copy."""
    v = _bits16(v).copy()
    lib().cpuref_silu_inplace(_p16(v), v.size)
    return v


def swiglu(gate, up) -> np.ndarray:
    """evaluate_activations(Silu, gate, Some(up)) (evaluator.rs:209-225)."""
    g = _bits16(gate).copy()
    u = _bits16(up)
    lib().cpuref_swiglu(_p16(g), _p16(u), g.size)
    return g


def gateup_swiglu(x, pg, pu, dm, dn, bits=4, threads: int = 1) -> np.ndarray:
    """Two lut_gemv_cpu calls then swiglu (engine_impl.rs:1120-1127, 1349-1374)."""
    x = _bits16(x)
    y = np.zeros(dm, dtype=np.uint16)
    tmp = np.zeros(dm, dtype=np.uint16)
    rc = lib().cpuref_gateup_swiglu(_p16(x), _p8(pg), _p8(pu), dm, dn, bits, _p16(y), _p16(tmp), threads)
    assert rc == 0
    return y


def lut_embed(token: int, payload, vocab: int, hidden: int) -> np.ndarray:
    """lut_embed (evaluator.rs:176-197)."""
    out = np.zeros(hidden, dtype=np.uint16)
    lib().cpuref_lut_embed(token, _p8(payload), vocab, hidden, _p16(out))
    return out


def decode_rows(payload, dm, dn, bits, r0=0, nrows=None) -> np.ndarray:
    """Dense fp16 bits of rows [r0, r0+nrows)."""
    if nrows is None:
        nrows = dm - r0
    out = np.zeros((nrows, dn), dtype=np.uint16)
    rc = lib().cpuref_decode_rows(_p8(payload), dm, dn, bits, r0, nrows, _p16(out))
    assert rc == 0
    return out
