"""Palettized weight format: producers, unpackers and seeded synthetic data.

Byte layout (split-block, the `.cimage` payload of src/lut/compiler.rs:50-61):

* 4-bit: ``[dim_m x 16 fp16 LUT, little-endian][dim_m x dim_n/2 packed
  nibbles]``; element ``2i`` is the low nibble of byte ``i`` and ``2i+1`` the
  high nibble (src/quantization/palette.rs:207-212).
* 8-bit (build extension, the format of
  compute-core/tests/palettized_vs_direct.rs:108-135 laid out split-block):
  ``[dim_m x 256 fp16 LUT][dim_m x dim_n index bytes]``.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

# Seeds of the BASELINE configurations (numpy PCG64); recorded in every
# bench and test record.
SEEDS = {"cfg1": 1001, "cfg2": 1002, "cfg3": 1003, "cfg4": 1004, "cfg5": 1005, "hero": 1000,
         "palettize": 1006}


def lut_entries(bits: int) -> int:
    if bits not in (4, 8):
        raise ValueError(f"bits must be 4 or 8, got {bits}")
    return 1 << bits


def row_index_bytes(dim_n: int, bits: int) -> int:
    """Index bytes per row; 4-bit rows are dim_n/2 bytes apart (evaluator.rs:31)."""
    return dim_n // 2 if bits == 4 else dim_n


def payload_bytes(dim_m: int, dim_n: int, bits: int) -> int:
    return dim_m * lut_entries(bits) * 2 + dim_m * row_index_bytes(dim_n, bits)


def pack_nibbles(idx: np.ndarray) -> np.ndarray:
    """[N, K] indices (0..15) -> [N, ceil(K/2)] bytes, element 2i in the low
    nibble (src/quantization/palette.rs:207-212)."""
    idx = np.asarray(idx, dtype=np.uint8)
    n, k = idx.shape
    if idx.size and int(idx.max()) > 15:
        raise ValueError("4-bit index out of range")
    pad = np.zeros((n, k + (k & 1)), dtype=np.uint8)
    pad[:, :k] = idx
    return (pad[:, 0::2] | (pad[:, 1::2] << 4)).astype(np.uint8)


def unpack_nibbles(packed: np.ndarray, k: int) -> np.ndarray:
    packed = np.asarray(packed, dtype=np.uint8)
    out = np.empty((packed.shape[0], packed.shape[1] * 2), dtype=np.uint8)
    out[:, 0::2] = packed & 0x0F
    out[:, 1::2] = packed >> 4
    return out[:, :k]


def encode_channel(channel: np.ndarray, codebook: np.ndarray) -> tuple[np.ndarray, float]:
    """Nearest-codebook encoding of one row, packed 2 per byte; returns
    (packed bytes, MSE).  Restates encode_channel
    (src/quantization/palette.rs:189-217): squared distance in f32 against
    the first 16 entries, the first minimum wins, (n+1)/2 output bytes."""
    ch = np.asarray(channel, dtype=np.float32)
    cb = np.asarray(codebook, dtype=np.float32)[:16]
    d = (ch[:, None] - cb[None, :]) ** 2
    best = np.argmin(d, axis=1).astype(np.uint8)  # argmin returns the first minimum
    mse = float(np.sum(d[np.arange(ch.size), best], dtype=np.float32) / np.float32(max(ch.size, 1)))
    return pack_nibbles(best[None, :])[0], mse


def split_block_payload(lut_f16: np.ndarray, idx: np.ndarray, bits: int) -> np.ndarray:
    """All rows' fp16 LUTs, then all rows' indices (src/lut/compiler.rs:50-61).

    lut_f16: [N, 2^bits] float16 (or uint16 bits); idx: [N, K] uint8 indices.
    """
    n = idx.shape[0]
    lut = np.ascontiguousarray(lut_f16)
    if lut.dtype == np.float16:
        lut = lut.view(np.uint16)
    if lut.shape != (n, lut_entries(bits)):
        raise ValueError(f"LUT shape {lut.shape} != ({n}, {lut_entries(bits)})")
    lut_bytes = lut.astype("<u2").view(np.uint8).reshape(-1)
    if bits == 4:
        k = idx.shape[1]
        packed = pack_nibbles(idx)[:, : k // 2]  # rows are K/2 bytes apart
        ib = packed.reshape(-1)
    else:
        ib = np.ascontiguousarray(idx, dtype=np.uint8).reshape(-1)
    return np.concatenate([lut_bytes, ib]).astype(np.uint8)


def unpack_payload(payload: np.ndarray, dim_m: int, dim_n: int, bits: int):
    """Split-block payload -> (lut uint16 [N, 2^bits], idx uint8 [N, K'])
    where K' = dim_n for 8-bit and 2*(dim_n//2) for 4-bit."""
    payload = np.asarray(payload, dtype=np.uint8)
    t = lut_entries(bits)
    lb = dim_m * t * 2
    if payload.size != payload_bytes(dim_m, dim_n, bits):
        raise ValueError("payload size does not match the shape")
    lut = payload[:lb].view("<u2").reshape(dim_m, t).astype(np.uint16)
    rb = row_index_bytes(dim_n, bits)
    ib = payload[lb:].reshape(dim_m, rb)
    idx = unpack_nibbles(ib, 2 * rb) if bits == 4 else ib.copy()
    return lut, idx


def dequantize(payload: np.ndarray, dim_m: int, dim_n: int, bits: int) -> np.ndarray:
    """Dense fp32 weights [N, K] (4-bit: elements past (K//8)*8 are zero,
    matching lut_gemv_cpu's word loop)."""
    lut, idx = unpack_payload(payload, dim_m, dim_n, bits)
    w = np.take_along_axis(lut.view(np.float16), idx.astype(np.int64), axis=1).astype(np.float32)
    out = np.zeros((dim_m, dim_n), dtype=np.float32)
    keff = (dim_n // 8) * 8 if bits == 4 else dim_n
    out[:, :keff] = w[:, :keff]
    return out


@dataclass
class PalettizedTensor:
    """A CompiledTensor (src/lut/compiler.rs:14-20) plus its bit width."""
    key: str
    dim_m: int
    dim_n: int
    bits: int
    payload: np.ndarray


def synth_tensor(dim_m: int, dim_n: int, bits: int, seed: int, key: str = "w",
                 lut_sigma: float = 0.02) -> PalettizedTensor:
    """Seeded synthetic palettized weights: per-row LUT = sorted draws from
    N(0, lut_sigma) cast to fp16, indices uniform over 0..2^bits-1."""
    rng = np.random.Generator(np.random.PCG64(seed))
    t = lut_entries(bits)
    lut = np.sort(rng.normal(0.0, lut_sigma, size=(dim_m, t)).astype(np.float32), axis=1).astype(np.float16)
    idx = rng.integers(0, t, size=(dim_m, dim_n), dtype=np.uint8)
    return PalettizedTensor(key, dim_m, dim_n, bits, split_block_payload(lut, idx, bits))


def synth_x(batch: int, dim_n: int, seed: int) -> np.ndarray:
    """Activations ~ N(0, 1) cast to fp16 (round-to-nearest-even); uint16 bits [batch, dim_n]."""
    rng = np.random.Generator(np.random.PCG64(seed + 7919))
    return rng.standard_normal(size=(batch, dim_n)).astype(np.float32).astype(np.float16).view(np.uint16)


def rel_err(y, ref) -> float:
    """max_i |y_i - ref_i| / max_i |ref_i| over one output vector (fp16 bits in)."""
    a = np.asarray(y).view(np.float16).astype(np.float64)
    b = np.asarray(ref).view(np.float16).astype(np.float64)
    den = np.max(np.abs(b)) if b.size else 0.0
    num = np.max(np.abs(a - b)) if b.size else 0.0
    if den == 0.0:
        return 0.0 if num == 0.0 else float("inf")
    return float(num / den)
