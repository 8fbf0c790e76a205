"""prism-engine_amd -- MI355X (gfx950) palettized-LUT weight contraction.

The product is ``libprism_hip.so`` (C ABI: ``include/prism_hip.h``), built
from ``csrc/``: hand-written HIP kernels for the palettized decode GEMV
(4/8-bit, any batch), the fused gate_up + SwiGLU GEMV, the prefill GEMM
(LUT decode feeding fp16 MFMA), the GPU-resident decode step and the palette
compiler.  This package is the host-side mirror of the reference's backend
surface over that ABI.

The directory name is not a Python identifier; import it with
``importlib.import_module("prism-engine_amd")``.
"""
from ._native import PrismHipError, header_functions, load as load_library  # noqa: F401
from .backend import Context, HipBackend, Model, Weight, load_cimage  # noqa: F401
from .model import Qwen2Config, synth_kv, synth_weights, tensor_names  # noqa: F401
from .cimage import CImageReader, CImageWriter  # noqa: F401
from .palette import (  # noqa: F401
    SEEDS,
    PalettizedTensor,
    dequantize,
    encode_channel,
    pack_nibbles,
    payload_bytes,
    rel_err,
    split_block_payload,
    synth_tensor,
    synth_x,
    unpack_nibbles,
    unpack_payload,
)

__version__ = "0.1.0"
