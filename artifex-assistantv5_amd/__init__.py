"""MI355X-native GGUF dequant-matmul for the 16 quantized types of the
reference's ``dequantGGML``: Q8_0 / Q4_K / Q5_K / Q6_K / Q2_K / Q3_K / Q4_0 /
Q5_0 / IQ4_NL / IQ4_XS and the grid-codebook types IQ2_XXS / IQ2_XS / IQ2_S /
IQ3_XXS / IQ3_S / IQ1_M.

Python host side of ``libgguf_hip.so`` (hand-written HIP kernels for gfx950
behind a C ABI, ``include/gguf_hip.h``).  The per-layer API mirrors the
reference's WebGPU engine (``webgpu/src/engine/forward-pass.ts``):

* ``GGUFWeight``            — a quantized matrix resident in HBM (forward-pass.ts:89-98)
* ``repack_gguf_for_gpu``   — raw GGUF bytes -> HBM row-tile layout (gguf-dequant.ts:809-840)
* ``dispatch_matmul_gguf``  — ``C[M,N] = A[M,K] @ dequant(W)^T`` (forward-pass.ts:1496-1544)
* ``dispatch_projection``   — per-layer projection lookup (forward-pass.ts:1576-1629)
* ``dequant_ggml``          — dequantize to f32 on the GPU (gguf-dequant.ts:844-868)
* ``qlinear``               — functional form returning a new tensor
* ``QuantEmbedding``        — raw GGUF rows in HBM, gathered per token (forward-pass.ts:2171-2186)
* ``parse_gguf``            — GGUF header / KV / tensor table (gguf.ts:241-299)
* ``load_gguf_model``       — place a GGUF file's tensors in HBM (gguf-loader.ts:166-460)
* ``load_decoder``          — a llama-architecture GGUF file as a ``QuantDecoder``

Importing this package does not touch the GPU; the native library is loaded
on first use and a missing or unbuilt library raises immediately.
"""

from . import ggml, quantize  # noqa: F401
from .ggml import (GGML_TYPES, GGMLTypeError, ggml_tensor_bytes, ggml_type_traits,  # noqa: F401
                   raw_row_bytes, tile_row_bytes, tiled_bytes)
from .linear import (GGUFWeight, LayerWeights, QuantEmbedding, concat_rows,  # noqa: F401
                     dequant_ggml, dequant_raw, dispatch_matmul_gguf, dispatch_projection,
                     interleave_tiles, qlinear, repack_gguf_for_gpu, split_interleaved)
from .gguf_file import parse_gguf, parse_gguf_path, write_gguf  # noqa: F401
from .gguf_loader import load_gguf_model  # noqa: F401
from .gguf_model import load_decoder  # noqa: F401
from ._native import GGUFHipError, load_library  # noqa: F401

__all__ = [
    "GGML_TYPES", "GGMLTypeError", "GGUFHipError", "GGUFWeight", "LayerWeights",
    "QuantEmbedding", "load_decoder", "load_gguf_model", "parse_gguf", "parse_gguf_path",
    "write_gguf",
    "concat_rows", "interleave_tiles", "split_interleaved", "dequant_ggml", "dequant_raw", "dispatch_matmul_gguf",
    "dispatch_projection", "ggml_tensor_bytes", "ggml_type_traits", "load_library",
    "qlinear", "raw_row_bytes", "repack_gguf_for_gpu", "tile_row_bytes", "tiled_bytes",
]

