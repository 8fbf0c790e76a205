"""Format producers and consumers: split-block packing, nibble order,
`.cimage` container (src/quantization/cimage.rs, palette.rs, compiler.rs)."""
import json
import os
import struct

import numpy as np
from hypothesis import given, settings, strategies as st


@settings(max_examples=60, deadline=None)
@given(st.integers(1, 9), st.integers(1, 70), st.sampled_from([4, 8]), st.integers(0, 2**31 - 1))
def test_payload_roundtrip(pe, n, k, bits, seed):
    rng = np.random.default_rng(seed)
    t = 1 << bits
    lut = rng.standard_normal((n, t)).astype(np.float16)
    idx = rng.integers(0, t, size=(n, k), dtype=np.uint8)
    p = pe.split_block_payload(lut, idx, bits)
    assert p.size == pe.payload_bytes(n, k, bits)
    lut2, idx2 = pe.unpack_payload(p, n, k, bits)
    assert np.array_equal(lut2, lut.view(np.uint16))
    keep = 2 * (k // 2) if bits == 4 else k
    assert np.array_equal(idx2[:, :keep], idx[:, :keep])


def test_nibble_layout_closed_form(pe):
    """element 8w+j is bits 4j..4j+3 of the little-endian u32 word w
    (compute-core/src/lut/evaluator.rs:33-38)."""
    rng = np.random.default_rng(1)
    idx = rng.integers(0, 16, size=(3, 64), dtype=np.uint8)
    packed = pe.pack_nibbles(idx)
    words = packed.view("<u4")
    for r in range(3):
        for w in range(8):
            for j in range(8):
                assert (int(words[r, w]) >> (4 * j)) & 15 == idx[r, 8 * w + j]


def test_encode_channel_odd_length(pe):
    """encode_channel packs (n+1)/2 bytes (palette.rs:219-247)."""
    packed, _ = pe.encode_channel(np.array([0.1, 0.2, 0.3]), np.linspace(0, 1.5, 16))
    assert packed.size == 2


def test_cimage_roundtrip(pe, tmp_path):
    """cimage.rs:360-392: write/read, 16 KB-aligned offsets, header parse."""
    path = str(tmp_path / "t.cimage")
    w = pe.CImageWriter(path)
    payload = np.arange(2 * 32 + 2 * 4, dtype=np.uint8)
    w.append_palettized("layer.0.wq", payload, 2, 8)
    t8 = pe.synth_tensor(3, 16, 8, seed=1)
    w.append_palettized("layer.0.w8", t8.payload, 3, 16, bits=8)
    w.set_execution_plan('{"assignments":[]}')
    w.finalize()
    with open(path, "rb") as f:
        assert f.read(8) == b"TRB_CIMG"
        (hs,) = struct.unpack("<Q", f.read(8))
        hdr = json.loads(f.read(hs))
    assert hdr["tensors"]["layer.0.wq"]["tensor_type"] == "Palettized4Bit"
    with pe.CImageReader(path) as r:
        rec = r.tensor("layer.0.wq")
        assert rec["dim_m"] == 2 and rec["dim_n"] == 8 and rec["offset"] % 16384 == 0
        assert np.array_equal(r.payload("layer.0.wq"), payload)
        assert np.array_equal(r.payload("layer.0.w8"), t8.payload)
        assert r.tensor("layer.0.w8")["tensor_type"] == "Palettized8Bit"
        assert r.execution_plan == '{"assignments":[]}'
    assert os.path.getsize(path) >= 8 * 16384


def test_cimage_header_fits_50_tensors(pe, tmp_path):
    """cimage.rs:394-411."""
    path = str(tmp_path / "h.cimage")
    w = pe.CImageWriter(path)
    for i in range(50):
        w.append_fp16(f"layer.{i}.wq", np.zeros(64, dtype=np.uint8), 1, 1)
    w.finalize()
    with pe.CImageReader(path) as r:
        assert len(r.tensors) == 50


def test_cimage_bad_magic(pe, tmp_path):
    path = tmp_path / "bad.cimage"
    path.write_bytes(b"NOTCIMG!" + bytes(100))
    import pytest
    with pytest.raises(ValueError, match="magic"):
        pe.CImageReader(str(path))


def test_synth_is_seeded(pe):
    a = pe.synth_tensor(8, 64, 4, seed=5)
    b = pe.synth_tensor(8, 64, 4, seed=5)
    assert np.array_equal(a.payload, b.payload)
    lut, idx = pe.unpack_payload(a.payload, 8, 64, 4)
    v = lut.view(np.float16).astype(np.float32)
    assert np.all(np.diff(v, axis=1) >= 0)  # sorted per row
