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

Decode step (``prism_cpuref_step.c``, the reference's PrismEngine::step for a
Qwen2 graph):

* ``rms_norm``: KAT evaluator.rs:249-257 (ones stay 1), constant-vector
  closed form, numpy float64 bound, scale invariance -- pinned.
* ``vec_add``: KAT evaluator.rs:258-265 and numpy float16 addition
  (exhaustive over a grid) -- pinned.
* ``rope``: pos 0 is the identity, pair j=0 rotates by exactly `pos`
  radians (numpy float64 rotation), norm preservation, theta ignored --
  pinned.
* ``kv_quant`` / ``kv_dequant``: hand-computed blocks (round half away from
  zero, clamp, zero-vector scale 1.0), round-trip bound max|x|/254 -- pinned.
* ``attention``: one position returns v, equal keys return the mean of v,
  numpy float64 softmax attention bound, GQA head mapping -- pinned.
* ``decode_step``: recomposed in the tests from the pinned pieces above
  following engine_impl.rs:1076-1405 (node order, Q-only RoPE, residual
  placement, KV append) -- pinned by composition.

Palette compiler (``prism_cpuref_palette.c``, fit_palette / encode_channel /
palettize_matrix and compile_to_cimage's payload):

* ``encode_channel``: KAT palette.rs:410-425 (0x10, 0x32, MSE 0), brute-force
  argmin over the codebook on random data -- pinned.
* ``fit_palette``: KATs palette.rs:373-408 (three clusters), :495-523 (empty,
  constant channel); exact integer arithmetic on small-integer channels (the
  k-means++ picks, the zero-total fallback and one Lloyd step follow from
  Python integers); closed forms (k = n distinct values gives the channel
  sorted by magnitude; at most k distinct values are reproduced exactly)
  -- pinned.
* ``palettize_payload``: KATs palette.rs:427-492 (3x4 round trip, 64x128 MSE
  bound), layout of compiler.rs:47-60 -- pinned.
* seeded variant (compute-core's palettize_matrix_phased seeds): closed
  forms (k distinct seeds reproduce themselves; seeds that hit every value
  give an exact payload) and exact-integer picks continuing from the last
  seed -- pinned.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
import threading

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libprism_cpuref.so")
_lib = None
# serialises calls that switch the C library's fold mode (cpuref_set_fold_mode)
FOLD_LOCK = threading.Lock()

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
        L.cpuref_rms_norm_inplace.argtypes = [_u16p, ctypes.c_size_t, ctypes.c_float]
        L.cpuref_rms_norm_inplace.restype = None
        L.cpuref_vec_add_inplace.argtypes = [_u16p, _u16p, ctypes.c_size_t]
        L.cpuref_vec_add_inplace.restype = None
        L.cpuref_rope_angle.argtypes = [ctypes.c_int64, ctypes.c_size_t, ctypes.c_size_t]
        L.cpuref_rope_angle.restype = ctypes.c_float
        L.cpuref_rope_inplace.argtypes = [_u16p, ctypes.c_size_t, ctypes.c_int64, ctypes.c_size_t]
        L.cpuref_rope_inplace.restype = None
        L.cpuref_kv_quant.argtypes = [_u16p, ctypes.c_size_t, _u8p]
        L.cpuref_kv_quant.restype = ctypes.c_size_t
        L.cpuref_kv_dequant.argtypes = [_u8p, ctypes.c_size_t, ctypes.c_size_t, _u16p]
        L.cpuref_kv_dequant.restype = None
        L.cpuref_attention.argtypes = [_u16p, _u16p, _u16p, ctypes.c_size_t, ctypes.c_size_t, ctypes.c_size_t,
                                       ctypes.c_size_t, _u16p]
        L.cpuref_attention.restype = None
        L.cpuref_decode_step.argtypes = [ctypes.POINTER(ctypes.c_uint32), ctypes.c_float, _u8p,
                                         ctypes.POINTER(ctypes.c_void_p), ctypes.POINTER(ctypes.c_void_p),
                                         ctypes.POINTER(ctypes.c_void_p), ctypes.POINTER(ctypes.c_size_t),
                                         ctypes.c_uint32, ctypes.c_int64, _u16p, ctypes.c_int]
        L.cpuref_decode_step.restype = ctypes.c_int
        L.cpuref_set_fold_mode.argtypes = [ctypes.c_int]
        L.cpuref_set_fold_mode.restype = None
        L.cpuref_fold_overflowed.argtypes = []
        L.cpuref_fold_overflowed.restype = ctypes.c_int
        _f32p = ctypes.POINTER(ctypes.c_float)
        L.cpuref_fit_palette.argtypes = [_f32p, ctypes.c_size_t, ctypes.c_size_t, ctypes.c_size_t, _f32p]
        L.cpuref_fit_palette.restype = ctypes.c_size_t
        L.cpuref_encode_channel.argtypes = [_f32p, ctypes.c_size_t, _f32p, ctypes.c_size_t, _u8p]
        L.cpuref_encode_channel.restype = ctypes.c_float
        L.cpuref_palettize_payload.argtypes = [_f32p, ctypes.c_size_t, ctypes.c_size_t, ctypes.c_size_t,
                                               ctypes.c_size_t, _u8p, _f32p]
        L.cpuref_palettize_payload.restype = ctypes.c_int
        L.cpuref_fit_palette_seeded.argtypes = [_f32p, ctypes.c_size_t, ctypes.c_size_t, ctypes.c_size_t, _f32p,
                                                ctypes.c_size_t, _f32p]
        L.cpuref_fit_palette_seeded.restype = ctypes.c_size_t
        L.cpuref_palettize_payload_seeded.argtypes = [_f32p, ctypes.c_size_t, ctypes.c_size_t, ctypes.c_size_t,
                                                      ctypes.c_size_t, _f32p, ctypes.c_size_t, _u8p, _f32p]
        L.cpuref_palettize_payload_seeded.restype = ctypes.c_int
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


# ---- decode step (prism_cpuref_step.c) -------------------------------------

def rms_norm(x, eps: float) -> np.ndarray:
    """rms_norm_inplace (evaluator.rs:49-64), on a copy."""
    x = _bits16(x).copy()
    lib().cpuref_rms_norm_inplace(_p16(x), x.size, ctypes.c_float(eps))
    return x


def vec_add(a, b) -> np.ndarray:
    """vec_add_inplace (evaluator.rs:67-73), on a copy of a."""
    a = _bits16(a).copy()
    b = _bits16(b)
    assert a.size == b.size
    lib().cpuref_vec_add_inplace(_p16(a), _p16(b), a.size)
    return a


def rope_angle(pos: int, j: int, hd: int) -> float:
    return float(lib().cpuref_rope_angle(pos, j, hd))


def rope(x, pos: int, hd: int) -> np.ndarray:
    """rope_inplace (evaluator.rs:154-166), on a copy; theta is not an
    argument because the reference ignores it (base 10000)."""
    x = _bits16(x).copy()
    lib().cpuref_rope_inplace(_p16(x), x.size, pos, hd)
    return x


def kv_quant(data) -> np.ndarray:
    """One INT8 KV token block [scale f32 LE][n x i8] (engine_impl.rs:532-556)."""
    data = _bits16(data)
    out = np.zeros(4 + data.size, dtype=np.uint8)
    n = lib().cpuref_kv_quant(_p16(data), data.size, _p8(out))
    return out[:n]


def kv_dequant(blocks, ntok: int, kv_dim: int) -> np.ndarray:
    """dequant_inline (engine_impl.rs:569-584) -> [ntok x kv_dim] fp16 bits."""
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
    assert blocks.size >= ntok * (kv_dim + 4)
    out = np.zeros((ntok, kv_dim), dtype=np.uint16)
    lib().cpuref_kv_dequant(_p8(blocks), ntok, kv_dim, _p16(out))
    return out


def attention(q, kc, vc, nh: int, nkv: int, hd: int, sl: int) -> np.ndarray:
    """attention_cpu (evaluator.rs:104-146); kc, vc [sl x nkv*hd] fp16 bits."""
    q, kc, vc = _bits16(q), _bits16(kc), _bits16(vc)
    out = np.zeros(nh * hd, dtype=np.uint16)
    lib().cpuref_attention(_p16(q), _p16(kc), _p16(vc), nh, nkv, hd, sl, _p16(out))
    return out


class KVState:
    """The reference's KVCache (engine_impl.rs:514-584): per layer, INT8
    token blocks of (4 + kv_dim) bytes for K and for V."""

    def __init__(self, n_layers: int, kv_dim: int, capacity: int):
        self.kv_dim = kv_dim
        self.capacity = capacity
        ts = kv_dim + 4
        self.k = [np.zeros(capacity * ts, dtype=np.uint8) for _ in range(n_layers)]
        self.v = [np.zeros(capacity * ts, dtype=np.uint8) for _ in range(n_layers)]
        self.len = np.zeros(n_layers, dtype=np.uintp)

    def append(self, layer: int, k, v) -> None:
        """KVCache::append(l, k, v) with both slices given: one block each."""
        ts = self.kv_dim + 4
        n = int(self.len[layer])
        assert n < self.capacity
        self.k[layer][n * ts:(n + 1) * ts] = kv_quant(k)
        self.v[layer][n * ts:(n + 1) * ts] = kv_quant(v)
        self.len[layer] = n + 1

    def dequant(self, layer: int):
        n = int(self.len[layer])
        return (kv_dequant(self.k[layer], n, self.kv_dim), kv_dequant(self.v[layer], n, self.kv_dim))

    def copy(self) -> "KVState":
        c = KVState.__new__(KVState)
        c.kv_dim, c.capacity = self.kv_dim, self.capacity
        c.k = [a.copy() for a in self.k]
        c.v = [a.copy() for a in self.v]
        c.len = self.len.copy()
        return c


def decode_step(dims, eps: float, embed, layers, kv: KVState, token: int, pos: int,
                threads: int = 1, fold: int = 0) -> np.ndarray:
    """PrismEngine::step (engine_impl.rs:1076-1405) for a Qwen2 graph.

    dims = (n_layers, hidden, n_heads, n_kv_heads, head_dim, intermediate,
    vocab, bits); `layers` is a list of 7-payload tuples (q, k, v, o, gate,
    up, down); `embed` the [vocab x hidden] 4-bit embedding (tied LM head).
    Advances `kv` by one token per layer and returns the fp16 logits.

    fold=1 runs the order-perturbed variant (prism_cpuref.c: every long sum
    in 64-term blocks added as a tree) -- test support for measuring
    summation-order drift, not the reference's arithmetic."""
    L = int(dims[0])
    assert len(layers) == L and len(kv.k) == L
    d = (ctypes.c_uint32 * 8)(*[int(v) for v in dims])
    ws = [np.ascontiguousarray(w, dtype=np.uint8) for lw in layers for w in lw]
    wp = (ctypes.c_void_p * max(1, len(ws)))(*[w.ctypes.data for w in ws])
    kp = (ctypes.c_void_p * max(1, L))(*[a.ctypes.data for a in kv.k])
    vp = (ctypes.c_void_p * max(1, L))(*[a.ctypes.data for a in kv.v])
    for l in range(L):
        assert int(kv.len[l]) < kv.capacity
    lens = (ctypes.c_size_t * max(1, L))(*[int(v) for v in kv.len])
    embed = np.ascontiguousarray(embed, dtype=np.uint8)
    logits = np.zeros(int(dims[6]), dtype=np.uint16)
    L_ = lib()
    # the fold mode is a process-wide switch of the C library: one call at a
    # time holds it
    with FOLD_LOCK:
        L_.cpuref_set_fold_mode(int(fold))
        try:
            rc = L_.cpuref_decode_step(d, ctypes.c_float(eps), _p8(embed), wp, kp, vp, lens, token, pos,
                                       _p16(logits), threads)
        finally:
            L_.cpuref_set_fold_mode(0)
            overflow = L_.cpuref_fold_overflowed()
    if overflow:
        raise ValueError("fold mode 1: a sum of more than 131072 terms (2048 blocks of 64) has no blocked order here")
    assert rc == 0, rc
    for l in range(L):
        kv.len[l] = lens[l]
    return logits


# ---- palette compiler (prism_cpuref_palette.c) -----------------------------

def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def fit_palette(channel, k: int = 16, max_iter: int = 50, seeds=None) -> np.ndarray:
    """fit_palette (palette.rs:75-183): min(k, n) centroids, |c| descending.
    seeds: compute-core's seeded variant (compute-core/src/quantization/
    palette.rs:94-201), the first min(len, k) centroids."""
    ch = _f32(channel)
    out = np.zeros(max(k, 1), dtype=np.float32)
    fp = ctypes.POINTER(ctypes.c_float)
    if seeds is None:
        sp, ns = None, 0
    else:
        sd = _f32(seeds)
        if sd.size == 0:
            raise ValueError("empty seed list (the reference indexes centroids[-1])")
        sp, ns = sd.ctypes.data_as(fp), sd.size
    kc = lib().cpuref_fit_palette_seeded(ch.ctypes.data_as(fp), ch.size, k, max_iter, sp, ns,
                                         out.ctypes.data_as(fp))
    return out[:kc].copy()


def encode_channel(channel, codebook):
    """encode_channel (palette.rs:198-228): (packed indices, MSE)."""
    ch = _f32(channel)
    cb = _f32(codebook)
    packed = np.zeros((ch.size + 1) // 2, dtype=np.uint8)
    mse = lib().cpuref_encode_channel(ch.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), ch.size,
                                      cb.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), cb.size, _p8(packed))
    return packed, float(mse)


def palettize_payload(weights, k: int = 16, max_iter: int = 50, threads: int = 1, seeds=None):
    """palettize_matrix + compile_to_cimage's payload (compiler.rs:47-60) for a
    [out_dim, in_dim] f32 matrix: (payload bytes, per-row MSE).  seeds: the
    calibration seeds of compute-core's palettize_matrix_phased, shared by
    every row."""
    w = _f32(weights)
    assert w.ndim == 2
    out_dim, in_dim = w.shape
    payload = np.zeros(out_dim * 32 + out_dim * ((in_dim + 1) // 2), dtype=np.uint8)
    mse = np.zeros(out_dim, dtype=np.float32)
    fp = ctypes.POINTER(ctypes.c_float)
    sd = None if seeds is None else _f32(seeds)
    if sd is not None and sd.size == 0:
        raise ValueError("empty seed list (the reference indexes centroids[-1])")
    if threads <= 1 or out_dim < 2 * threads:
        rc = lib().cpuref_palettize_payload_seeded(w.ctypes.data_as(fp), out_dim, in_dim, k, max_iter,
                                                   None if sd is None else sd.ctypes.data_as(fp),
                                                   0 if sd is None else sd.size, _p8(payload),
                                                   mse.ctypes.data_as(fp))
        assert rc == 0
        return payload, mse
    # rows are independent: split them over host threads (identical bytes)
    from concurrent.futures import ThreadPoolExecutor
    bounds = np.linspace(0, out_dim, threads + 1).astype(int)

    def run(a, b):
        p, e = palettize_payload(w[a:b], k, max_iter, 1, sd)
        return a, b, p, e

    with ThreadPoolExecutor(threads) as ex:
        parts = list(ex.map(lambda ab: run(*ab), zip(bounds[:-1], bounds[1:])))
    rb = (in_dim + 1) // 2
    for a, b, p, e in parts:
        payload[a * 32:b * 32] = p[:(b - a) * 32]
        payload[out_dim * 32 + a * rb:out_dim * 32 + b * rb] = p[(b - a) * 32:]
        mse[a:b] = e
    return payload, mse
