"""GGML type ids, block traits and the HBM row layout of quantized weights.

Type ids and (block elements, block bytes) follow the GGUF spec as the
reference tabulates it in ``webgpu/src/model/gguf.ts:24-35`` (``GGML_TYPES``)
and ``:39-73`` (``TYPE_TRAITS``); ``ggml_type_traits`` and
``ggml_tensor_bytes`` mirror ``gguf.ts:75-92`` including their errors.

The row-tile layout is this library's own (the reference pads blocks to
4-byte strides for WGSL, ``gguf-dequant.ts:655-672``).  Rows are grouped in
tiles of 16 consecutive rows (row-major weight, ``matmul_gguf.wgsl:5-8``;
the last tile is zero-padded).  For each unit of K -- a 256-element
superblock (Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, IQ4_XS) or a 32-element block (Q4_0, Q5_0,
Q8_0, IQ4_NL) -- a tile stores the 16 rows' GGUF blocks interleaved at 16-byte
granularity (8 bytes for Q8_0 quants, 4 for the nibble codes of the other
32-element types and of each IQ4_XS sub-block, regrouped per lane), so that one wave-wide load of a
matrix-core operand reads contiguous HBM.  No bytes are added: a weight of ``N`` rows takes
``round_up(N, 16) * raw_row_bytes(type, K)`` bytes.  The byte order inside a
tile-unit is defined in ``csrc/common.hpp`` (and modelled in
``tests/tile_model.py``).

Row ranges that start on a multiple of 16 are weights of their own (byte
offset ``start * raw_row_bytes``): gate/up concatenation and row sharding
stay byte-range operations.
"""

from __future__ import annotations

# gguf.ts:24-35
GGML_TYPES = {
    "F32": 0, "F16": 1,
    "Q4_0": 2, "Q4_1": 3,
    "Q5_0": 6, "Q5_1": 7,
    "Q8_0": 8, "Q8_1": 9,
    "Q2_K": 10, "Q3_K": 11, "Q4_K": 12, "Q5_K": 13, "Q6_K": 14, "Q8_K": 15,
    "IQ2_XXS": 16, "IQ2_XS": 17, "IQ3_XXS": 18, "IQ1_S": 19, "IQ4_NL": 20,
    "IQ3_S": 21, "IQ2_S": 22, "IQ4_XS": 23,
    "I8": 24, "I16": 25, "I32": 26, "I64": 27, "F64": 28, "IQ1_M": 29,
    "BF16": 30,
}
GGML_TYPE_NAMES = {v: k for k, v in GGML_TYPES.items()}

F32 = GGML_TYPES["F32"]
F16 = GGML_TYPES["F16"]
BF16 = GGML_TYPES["BF16"]
Q4_0 = GGML_TYPES["Q4_0"]
Q5_0 = GGML_TYPES["Q5_0"]
Q8_0 = GGML_TYPES["Q8_0"]
Q4_K = GGML_TYPES["Q4_K"]
Q5_K = GGML_TYPES["Q5_K"]
Q6_K = GGML_TYPES["Q6_K"]
IQ4_NL = GGML_TYPES["IQ4_NL"]
IQ4_XS = GGML_TYPES["IQ4_XS"]
Q2_K = GGML_TYPES["Q2_K"]
Q3_K = GGML_TYPES["Q3_K"]

# gguf.ts:39-73 — [elements per block, bytes per block]
_TYPE_TRAITS = {
    0: (1, 4), 1: (1, 2), 30: (1, 2), 24: (1, 1), 25: (1, 2), 26: (1, 4),
    27: (1, 8), 28: (1, 8),
    2: (32, 18), 3: (32, 20), 6: (32, 22), 7: (32, 24), 8: (32, 34), 9: (32, 36),
    10: (256, 84), 11: (256, 110), 12: (256, 144), 13: (256, 176), 14: (256, 210),
    15: (256, 292),
    16: (256, 66), 17: (256, 74), 18: (256, 98), 19: (256, 50), 20: (32, 18),
    21: (256, 110), 22: (256, 82), 23: (256, 136), 29: (256, 56),
}

IQ2_XXS = GGML_TYPES["IQ2_XXS"]
IQ2_XS = GGML_TYPES["IQ2_XS"]
IQ2_S = GGML_TYPES["IQ2_S"]
IQ3_XXS = GGML_TYPES["IQ3_XXS"]
IQ3_S = GGML_TYPES["IQ3_S"]
IQ1_M = GGML_TYPES["IQ1_M"]

# The grid-codebook types (codebook entries, sign patterns and odd scale factors
# per 8 values).
GRID_TYPES = (IQ2_XXS, IQ2_XS, IQ2_S, IQ3_XXS, IQ3_S, IQ1_M)

# Types the HIP kernels of this library decode.
KERNEL_TYPES = (Q4_0, Q5_0, Q8_0, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, IQ4_NL, IQ4_XS) + GRID_TYPES

# Types with fused decode-step kernels (gguf_hip_matmul_fused / _attn_merge): all.
FUSED_TYPES = KERNEL_TYPES


class GGMLTypeError(NotImplementedError):
    """Unsupported ggml type (gguf.ts:75-79, gguf-dequant.ts:837,866)."""


def ggml_type_traits(ggml_type: int) -> tuple[int, int, str]:
    """``(block_size, type_size, name)``; raises for unknown types (gguf.ts:75-79)."""
    t = _TYPE_TRAITS.get(int(ggml_type))
    if t is None:
        raise GGMLTypeError(f"[GGUF] Unsupported ggml type {ggml_type}")
    return t[0], t[1], GGML_TYPE_NAMES[int(ggml_type)]


def ggml_tensor_bytes(ggml_type: int, ne: list[int] | tuple[int, ...]) -> int:
    """Raw GGUF bytes of a tensor with dims ``ne`` (innermost first), gguf.ts:82-92."""
    block, tsize, _ = ggml_type_traits(ggml_type)
    ne0 = int(ne[0]) if len(ne) else 1
    if ne0 % block != 0:
        raise ValueError(
            f"[GGUF] ne[0]={ne0} not divisible by block size {block} for type {ggml_type}")
    outer = 1
    for d in ne[1:]:
        outer *= int(d)
    return (ne0 // block) * tsize * outer


def check_kernel_type(ggml_type: int) -> None:
    if int(ggml_type) not in KERNEL_TYPES:
        ggml_type_traits(ggml_type)  # unknown ids raise the gguf.ts error
        raise GGMLTypeError(
            f"[gguf-hip] no kernel for ggml type {ggml_type} "
            f"({GGML_TYPE_NAMES.get(int(ggml_type), '?')})")


def raw_row_bytes(ggml_type: int, k: int) -> int:
    """GGUF bytes of one row of ``k`` elements."""
    return ggml_tensor_bytes(ggml_type, [k])


TILE_ROWS = 16


def tile_row_bytes(ggml_type: int, k: int) -> int:
    """Bytes per row in the row-tile layout (equal to the raw GGUF row bytes)."""
    check_kernel_type(ggml_type)
    block, tsize, _ = ggml_type_traits(ggml_type)
    if k <= 0 or k % block != 0:
        raise ValueError(f"[gguf-hip] K={k} not a positive multiple of block size {block}")
    return tsize * (k // block)


def tiled_rows(n: int) -> int:
    """Rows a weight of ``n`` rows occupies (whole tiles of 16)."""
    return -(-int(n) // TILE_ROWS) * TILE_ROWS


def tiled_bytes(ggml_type: int, n: int, k: int) -> int:
    """Bytes of an ``[n, k]`` weight in the row-tile layout."""
    return tiled_rows(n) * tile_row_bytes(ggml_type, k)
