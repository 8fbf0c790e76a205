"""Host-side mirror of the reference's backend surface over the HIP C ABI.

* :class:`Context` / :class:`Weight` wrap ``prism_hip_ctx`` /
  ``prism_hip_weight`` (host- and device-pointer entry points).
* :class:`HipBackend` mirrors ``MetalBackend`` (src/lut/engine_impl.rs:31-490)
  method for method: ``new(tensors)``, ``gemv(key, inp, out)``,
  ``fused_gate_up(gate_key, up_key, input, output)``, plus ``gemm`` and
  ``embed``.  Where the reference returns ``Err(String)`` this raises
  :class:`PrismHipError` with the same text ("miss <key>", ...).
* :class:`Model` wraps ``prism_hip_model``: the GPU-resident decode step
  (PrismEngine::step, engine_impl.rs:1076-1405) with its INT8 KV cache.
* :func:`load_cimage` uploads every palettized tensor of a `.cimage` file
  (the weight half of ``PrismEngine::load`` + ``MetalBackend::new``,
  engine_impl.rs:597-636,124-133).

Nothing here computes on the CPU: a missing library or a device error
raises; there is no fallback path.
"""
from __future__ import annotations

import ctypes
import sys

import numpy as np

from . import _native
from ._native import PrismHipError, ptr
from .palette import PalettizedTensor


def _u16(a) -> np.ndarray:
    a = np.ascontiguousarray(a)
    if a.dtype == np.float16:
        a = a.view(np.uint16)
    if a.dtype != np.uint16:
        raise TypeError(f"expected fp16 bits (uint16), got {a.dtype}")
    return a


def _stream_handle(stream) -> int | None:
    if stream is None:
        return None
    if hasattr(stream, "cuda_stream"):
        return stream.cuda_stream
    return int(stream)


class Context:
    """One device + one HIP stream (prism_hip_ctx)."""

    def __init__(self, device: int = 0):
        self.lib = _native.load()
        self.h = self.lib.prism_hip_ctx_create(device)
        if not self.h:
            raise PrismHipError(_native.ERR_DEVICE, self.lib.prism_hip_last_error(None).decode())
        self.device = device

    def error(self) -> str:
        return self.lib.prism_hip_last_error(self.h).decode()

    def check(self, rc: int) -> None:
        if rc != _native.OK:
            raise PrismHipError(rc, self.error())

    def last_kernels(self) -> str:
        """The kernels the dispatch launched in this context's most recent
        compute call, e.g. "k_gemv_lpr<8, 1, 1, 0, 16>" (prism_hip_last_kernels)."""
        return self.lib.prism_hip_last_kernels(self.h).decode()

    def upload(self, payload: np.ndarray, dim_m: int, dim_n: int, bits: int) -> "Weight":
        payload = np.ascontiguousarray(payload, dtype=np.uint8)
        h = self.lib.prism_hip_weight_upload(self.h, payload.ctypes.data, payload.size, dim_m, dim_n, bits,
                                             _native.LAYOUT_SPLIT_BLOCK)
        if not h:
            raise PrismHipError(_native.ERR_SHAPE, self.error())
        return Weight(self, h, dim_m, dim_n, bits, payload.size)

    def upload_async(self, payload: np.ndarray, dim_m: int, dim_n: int, bits: int) -> "Weight":
        """upload() without the final wait (the payload is consumed before
        return; the device copy is ordered on the context stream).  Call
        synchronize() before using the weight on another stream."""
        payload = np.ascontiguousarray(payload, dtype=np.uint8)
        h = self.lib.prism_hip_weight_upload_async(self.h, payload.ctypes.data, payload.size, dim_m, dim_n, bits,
                                                   _native.LAYOUT_SPLIT_BLOCK)
        if not h:
            raise PrismHipError(_native.ERR_SHAPE, self.error())
        return Weight(self, h, dim_m, dim_n, bits, payload.size)

    def synchronize(self) -> None:
        self.check(self.lib.prism_hip_ctx_synchronize(self.h))

    def upload_tensor(self, t: PalettizedTensor) -> "Weight":
        return self.upload(t.payload, t.dim_m, t.dim_n, t.bits)

    def upload_dev(self, d_payload, dim_m: int, dim_n: int, bits: int) -> "Weight":
        """Upload from a device buffer (a torch tensor or an address) holding a split-block payload."""
        nbytes = d_payload.numel() * d_payload.element_size() if hasattr(d_payload, "numel") else None
        if nbytes is None:
            raise ValueError("pass a torch tensor")
        h = self.lib.prism_hip_weight_upload_dev(self.h, ptr(d_payload), nbytes, dim_m, dim_n, bits,
                                                 _native.LAYOUT_SPLIT_BLOCK)
        if not h:
            raise PrismHipError(_native.ERR_SHAPE, self.error())
        return Weight(self, h, dim_m, dim_n, bits, nbytes)

    # -- host-pointer, synchronous
    def gemv(self, w: "Weight", x) -> np.ndarray:
        x = _u16(x)
        batch = x.size // w.dim_n
        if batch * w.dim_n != x.size:
            raise ValueError("x size is not a multiple of dim_n")
        y = np.empty((batch, w.dim_m), dtype=np.uint16)
        self.check(self.lib.prism_hip_gemv(self.h, w.h, x.ctypes.data, batch, y.ctypes.data))
        return y

    def gateup_swiglu(self, gate: "Weight", up: "Weight", x) -> np.ndarray:
        x = _u16(x)
        y = np.empty(gate.dim_m, dtype=np.uint16)
        self.check(self.lib.prism_hip_gateup_swiglu(self.h, gate.h, up.h, x.ctypes.data, y.ctypes.data))
        return y

    def gate_up(self, gate: "Weight", up: "Weight", x) -> tuple[np.ndarray, np.ndarray]:
        """The raw gate and up outputs in one pass (fused_gate_up.metal's two outputs)."""
        x = _u16(x)
        yg = np.empty(gate.dim_m, dtype=np.uint16)
        yu = np.empty(gate.dim_m, dtype=np.uint16)
        self.check(self.lib.prism_hip_gate_up(self.h, gate.h, up.h, x.ctypes.data, yg.ctypes.data, yu.ctypes.data))
        return yg, yu

    def gemm(self, w: "Weight", X) -> np.ndarray:
        X = _u16(X)
        M = X.size // w.dim_n
        Y = np.empty((M, w.dim_m), dtype=np.uint16)
        self.check(self.lib.prism_hip_gemm(self.h, w.h, X.ctypes.data, M, Y.ctypes.data))
        return Y

    def lut_embed(self, w: "Weight", token: int) -> np.ndarray:
        out = np.empty(w.dim_n, dtype=np.uint16)
        self.check(self.lib.prism_hip_lut_embed(self.h, w.h, token, out.ctypes.data))
        return out

    # -- device-pointer, asynchronous on `stream` (torch stream or handle)
    def gemv_dev(self, w: "Weight", d_x, batch: int, d_y, stream=None) -> None:
        self.check(self.lib.prism_hip_gemv_dev(self.h, w.h, ptr(d_x), batch, ptr(d_y), _stream_handle(stream)))

    def gateup_swiglu_dev(self, gate: "Weight", up: "Weight", d_x, d_y, stream=None) -> None:
        self.check(self.lib.prism_hip_gateup_swiglu_dev(self.h, gate.h, up.h, ptr(d_x), ptr(d_y),
                                                        _stream_handle(stream)))

    def gate_up_dev(self, gate: "Weight", up: "Weight", d_x, d_gate, d_up, stream=None) -> None:
        self.check(self.lib.prism_hip_gate_up_dev(self.h, gate.h, up.h, ptr(d_x), ptr(d_gate), ptr(d_up),
                                                  _stream_handle(stream)))

    def stream_read_dev(self, d_buf, nbytes: int, d_sink, stream=None) -> None:
        """The read floor: read nbytes of d_buf once (measure_kernels.hpp)."""
        self.check(self.lib.prism_hip_stream_read_dev(self.h, ptr(d_buf), nbytes, ptr(d_sink),
                                                      _stream_handle(stream)))

    def launch_empty_dev(self, stream=None) -> None:
        """One launch of an empty kernel (measure_kernels.hpp)."""
        self.check(self.lib.prism_hip_launch_empty_dev(self.h, _stream_handle(stream)))

    def mfma_probe_dev(self, groups: int, iters: int, d_sink, stream=None) -> None:
        """`groups` workgroups of register-only MFMA rounds (measure_kernels.hpp)."""
        self.check(self.lib.prism_hip_mfma_probe_dev(self.h, groups, iters, ptr(d_sink), _stream_handle(stream)))

    def issue_probe_dev(self, op: int, groups: int, waves_per_simd: int, iters: int, d_sink, stream=None) -> None:
        """Issue-rate probe (measure_kernels.hpp k_issue_probe): op 0 v_fma_f32,
        1 v_dot2_f32_f16, 2 v_perm_b32, 3 v_mfma_f32_4x4x4f16."""
        self.check(self.lib.prism_hip_issue_probe_dev(self.h, op, groups, waves_per_simd, iters, ptr(d_sink),
                                                      _stream_handle(stream)))

    def gemm_dev(self, w: "Weight", d_X, M: int, d_Y, stream=None) -> None:
        self.check(self.lib.prism_hip_gemm_dev(self.h, w.h, ptr(d_X), M, ptr(d_Y), _stream_handle(stream)))

    def gemm_dev_noalloc(self, w: "Weight", d_X, M: int, d_Y, stream=None) -> None:
        """gemm_dev with its split-K partials in the library's static per-GPU
        scratch: allocates nothing; overlapping calls on one GPU race."""
        self.check(self.lib.prism_hip_gemm_dev_noalloc(self.h, w.h, ptr(d_X), M, ptr(d_Y), _stream_handle(stream)))

    def decode_rows_dev(self, w: "Weight", row0: int, nrows: int, d_out, stream=None) -> None:
        self.check(self.lib.prism_hip_decode_rows_dev(self.h, w.h, row0, nrows, ptr(d_out),
                                                      _stream_handle(stream)))

    # -- palette compiler (palettize_matrix + compile_to_cimage's payload)
    def palettize_bytes(self, out_dim: int, in_dim: int) -> int:
        return int(self.lib.prism_hip_palettize_bytes(out_dim, in_dim))

    @staticmethod
    def _seeds(seeds):
        if seeds is None:
            return None, None, 0
        s = np.ascontiguousarray(seeds, dtype=np.float32).reshape(-1)
        return s, s.ctypes.data, s.size

    def palettize(self, w, k: int = 16, max_iter: int = 50, seeds=None) -> np.ndarray:
        """fp32 [out_dim, in_dim] weights -> the split-block payload (uint8),
        byte-identical to the reference compiler's (k=16, max_iter=50 there).
        seeds: compute-core's calibration seeds (first centroids of every row)."""
        w = np.ascontiguousarray(w, dtype=np.float32)
        if w.ndim != 2:
            raise ValueError(f"weights must be 2-D [out_dim, in_dim], got shape {w.shape}")
        out_dim, in_dim = w.shape
        out = np.empty(self.palettize_bytes(out_dim, in_dim), dtype=np.uint8)
        keep, sp, ns = self._seeds(seeds)
        self.check(self.lib.prism_hip_palettize(self.h, w.ctypes.data if w.size else None, out_dim, in_dim, k,
                                                max_iter, sp, ns, out.ctypes.data))
        return out

    def palettize_dev(self, d_w, out_dim: int, in_dim: int, d_payload, k: int = 16, max_iter: int = 50,
                      stream=None, seeds=None) -> None:
        keep, sp, ns = self._seeds(seeds)
        self.check(self.lib.prism_hip_palettize_dev(self.h, ptr(d_w), out_dim, in_dim, k, max_iter, sp, ns,
                                                    ptr(d_payload), _stream_handle(stream)))

    def close(self) -> None:
        if self.h:
            self.lib.prism_hip_ctx_destroy(self.h)
            self.h = None

    def __del__(self):
        # no HIP calls while the interpreter tears down (the runtime may be gone)
        if sys.is_finalizing():
            return
        try:
            self.close()
        except Exception:
            pass


class Weight:
    """A device copy of one palettized payload (prism_hip_weight)."""

    def __init__(self, ctx: Context, h, dim_m: int, dim_n: int, bits: int, nbytes: int):
        self.ctx, self.h = ctx, h
        self.dim_m, self.dim_n, self.bits, self.nbytes = dim_m, dim_n, bits, nbytes

    def free(self) -> None:
        if self.h:
            self.ctx.lib.prism_hip_weight_free(self.h)
            self.h = None

    def __del__(self):
        if sys.is_finalizing():
            return
        try:
            self.free()
        except Exception:
            pass


class Model:
    """prism_hip_model: one decode step per call, KV cache in HBM."""

    def __init__(self, ctx: Context, cfg, max_seq: int = 4096):
        self.ctx, self.cfg, self.max_seq = ctx, cfg, max_seq
        c = _native.ModelConfig(cfg.n_layers, cfg.hidden, cfg.n_heads, cfg.n_kv_heads, cfg.head_dim,
                                cfg.intermediate, cfg.vocab, max_seq, cfg.rms_eps, cfg.rope_theta)
        self.h = ctx.lib.prism_hip_model_create(ctx.h, ctypes.byref(c))
        if not self.h:
            raise PrismHipError(_native.ERR_SHAPE, ctx.error())

    @classmethod
    def from_tensors(cls, ctx: Context, cfg, embed: PalettizedTensor, layers, max_seq: int = 4096) -> "Model":
        """Upload `embed` and the per-layer tensors (7 per layer, q k v o gate
        up down); the model keeps its own copies."""
        m = cls(ctx, cfg, max_seq)
        w = ctx.upload_tensor(embed)
        m.set_embedding(w)
        w.free()
        for l, lw in enumerate(layers):
            ws = [ctx.upload_tensor(t) for t in lw]
            m.set_layer(l, ws)
            for x in ws:
                x.free()
        return m

    def set_embedding(self, w: "Weight") -> None:
        self.ctx.check(self.ctx.lib.prism_hip_model_set_embedding(self.h, w.h))

    def set_layer(self, layer: int, ws) -> None:
        assert len(ws) == 7
        self.ctx.check(self.ctx.lib.prism_hip_model_set_layer(self.h, layer, *[w.h for w in ws]))

    def kv_append(self, layer: int, k, v) -> None:
        """KVCache::append for rows of kv_dim fp16 values (k, v: [n, kv_dim])."""
        k, v = _u16(k), _u16(v)
        n = k.size // self.cfg.kv_dim
        assert k.size == v.size == n * self.cfg.kv_dim
        self.ctx.check(self.ctx.lib.prism_hip_model_kv_append(self.h, layer, k.ctypes.data, v.ctypes.data, n))

    def kv_len(self, layer: int) -> int:
        n = ctypes.c_uint32(0)
        self.ctx.check(self.ctx.lib.prism_hip_model_kv_len(self.h, layer, ctypes.byref(n)))
        return int(n.value)

    def kv_read(self, layer: int):
        """(K blocks, V blocks) in the reference's byte format."""
        n = self.kv_len(layer)
        kb = np.zeros(n * (self.cfg.kv_dim + 4), dtype=np.uint8)
        vb = np.zeros_like(kb)
        self.ctx.check(self.ctx.lib.prism_hip_model_kv_read(self.h, layer, kb.ctypes.data, vb.ctypes.data))
        return kb, vb

    def kv_reset(self) -> None:
        self.ctx.check(self.ctx.lib.prism_hip_model_kv_reset(self.h))

    def kv_truncate(self, n: int) -> None:
        """Drop every layer's tokens past n (host bookkeeping only)."""
        self.ctx.check(self.ctx.lib.prism_hip_model_kv_truncate(self.h, n))

    def step(self, token: int, pos: int) -> np.ndarray:
        """PrismEngine::step(token, pos): fp16 logits [vocab] (host)."""
        out = np.empty(self.cfg.vocab, dtype=np.uint16)
        self.ctx.check(self.ctx.lib.prism_hip_model_step(self.h, token, pos, out.ctypes.data))
        return out

    def step_dev(self, token: int, pos: int, stream=None) -> None:
        """Enqueue one step on `stream`; logits stay in logits_dev()."""
        self.ctx.check(self.ctx.lib.prism_hip_model_step_dev(self.h, token, pos, _stream_handle(stream)))

    def logits_dev(self) -> int:
        return int(self.ctx.lib.prism_hip_model_logits_dev(self.h) or 0)

    def close(self) -> None:
        if self.h:
            self.ctx.lib.prism_hip_model_free(self.h)
            self.h = None

    def __del__(self):
        if sys.is_finalizing():
            return
        try:
            self.close()
        except Exception:
            pass


class HipBackend:
    """MetalBackend's surface (src/lut/engine_impl.rs:31-490) on MI355X."""

    def __init__(self, device: int = 0):
        self.lib = _native.load()
        self.h = self.lib.prism_hip_backend_new(device)
        if not self.h:
            raise PrismHipError(_native.ERR_DEVICE, self.lib.prism_hip_backend_last_error(None).decode())

    @classmethod
    def new(cls, tensors, device: int = 0) -> "HipBackend":
        """MetalBackend::new (engine_impl.rs:51-154): uploads every tensor.
        `tensors` maps key -> PalettizedTensor (or an iterable of them)."""
        b = cls(device)
        items = tensors.values() if isinstance(tensors, dict) else tensors
        for t in items:
            b.add_tensor(t.key, t.payload, t.dim_m, t.dim_n, t.bits)
        b.synchronize()
        return b

    def _check(self, rc: int) -> None:
        if rc != _native.OK:
            raise PrismHipError(rc, self.lib.prism_hip_backend_last_error(self.h).decode())

    def __len__(self) -> int:
        return int(self.lib.prism_hip_backend_len(self.h))

    def synchronize(self) -> None:
        """Wait for every add_tensor upload (they are asynchronous)."""
        self._check(self.lib.prism_hip_backend_synchronize(self.h))

    def add_tensor(self, key: str, payload, dim_m: int, dim_n: int, bits: int = 4) -> None:
        payload = np.ascontiguousarray(payload, dtype=np.uint8)
        self._check(self.lib.prism_hip_backend_add_tensor(self.h, key.encode(), payload.ctypes.data, payload.size,
                                                          dim_m, dim_n, bits))

    def gemv(self, key: str, inp, out: np.ndarray | None = None, dim_m: int | None = None) -> np.ndarray:
        """MetalBackend::gemv(key, inp, out) (engine_impl.rs:155-190)."""
        inp = _u16(inp)
        if out is None:
            if dim_m is None:
                raise ValueError("pass `out` or `dim_m`")
            out = np.empty(dim_m * max(1, inp.size // max(1, inp.shape[-1])), dtype=np.uint16)
        self._check(self.lib.prism_hip_backend_gemv(self.h, key.encode(), inp.ctypes.data, inp.size,
                                                    out.ctypes.data, out.size))
        return out

    def fused_gate_up(self, gate_key: str, up_key: str, inp, out: np.ndarray) -> np.ndarray:
        """MetalBackend::fused_gate_up (engine_impl.rs:443-490)."""
        inp = _u16(inp)
        self._check(self.lib.prism_hip_backend_fused_gate_up(self.h, gate_key.encode(), up_key.encode(),
                                                             inp.ctypes.data, inp.size, out.ctypes.data,
                                                             out.size))
        return out

    def gemm(self, key: str, X, out: np.ndarray) -> np.ndarray:
        X = _u16(X)
        M = out.shape[0]
        self._check(self.lib.prism_hip_backend_gemm(self.h, key.encode(), X.ctypes.data, M, out.ctypes.data))
        return out

    def embed(self, key: str, token: int, out: np.ndarray) -> np.ndarray:
        """lut_embed through a keyed tensor (engine_impl.rs:1407-1446)."""
        self._check(self.lib.prism_hip_backend_embed(self.h, key.encode(), token, out.ctypes.data, out.size))
        return out

    def close(self) -> None:
        if self.h:
            self.lib.prism_hip_backend_free(self.h)
            self.h = None

    def __del__(self):
        if sys.is_finalizing():
            return
        try:
            self.close()
        except Exception:
            pass


def load_cimage(path: str, device: int = 0, populate: bool = True) -> HipBackend:
    """Upload every palettized tensor of a `.cimage` file into a HipBackend
    (engine_impl.rs:597-636 + MetalBackend::new's upload, :124-133).  The
    payloads are memory-mapped, not read whole; each goes through the
    context's pinned staging ring without a wait, and one wait at the end
    makes them all usable from any stream."""
    from .cimage import CImageReader, bits_of
    b = HipBackend(device)
    with CImageReader(path, populate=populate) as r:
        for name, rec in r.tensors.items():
            if rec["tensor_type"] not in ("Palettized4Bit", "Palettized8Bit"):
                continue
            b.add_tensor(name, r.payload(name), rec["dim_m"], rec["dim_n"], bits_of(rec["tensor_type"]))
        b.synchronize()
    return b
