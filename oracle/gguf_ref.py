"""CPU oracle for the GGUF Q4_0 / Q5_0 / Q8_0 / IQ4_NL / IQ4_XS / Q2_K / Q3_K / Q4_K / Q5_K /
Q6_K dequant-matmul path (and, through ``oracle/gguf_iq.py``, the grid-codebook
IQ types IQ2_XXS / IQ2_XS / IQ2_S / IQ3_XXS / IQ3_S / IQ1_M).

TEST INFRASTRUCTURE ONLY.  This module is the oracle: only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it, and only to check or to time the CPU baseline.  The product path
(the HIP library and its Python host code) never calls it.

It restates the reference's CPU dequantization
(``webgpu/src/model/gguf-dequant.ts``) twice:

* ``*_loop`` functions follow the TypeScript loops line for line, computing in
  Python floats (IEEE f64, like JavaScript numbers) and rounding once to f32
  on store, as the reference's ``Float32Array`` store does.  Pure Python;
  use them on small inputs only.
* the vectorised numpy functions compute in f32.  They are bit-identical to
  the loops because every product in these formats is exact in f32 (Q8_0
  ``d*q`` needs <= 18 significant bits, Q4_0 / Q5_0 ``d*(q-8)`` / ``d*(q-16)``
  <= 15 / 16, IQ4_NL ``d*kvalues[q]`` <= 18, IQ4_XS ``d*(ls-32)*kvalues[q]``
  <= 23, Q2_K ``d*sc*q`` <= 17 and ``dmin*m`` <= 15, Q3_K ``d*(sc-32)*(q-4)`` <= 20, Q6_K ``d*sc*q`` <= 23, Q4_K
  ``d*sc*q`` <= 21, Q5_K ``d*sc*q`` <= 22 and ``dmin*m`` <= 17) and the only
  rounding left is the final Q2_K / Q4_K / Q5_K subtraction, which f32 and
  f64-then-f32 both round correctly (the exact difference is a multiple of
  2**-24 below 2**27, so it fits in f64's 53 bits).

Parity pins (all in ``tests/test_oracle.py``):
* the reference's gguf-py golden vectors (``webgpu/test-fixtures/gguf-*.json``
  ``dequant_samples``: 1 Q8_0, 2 Q4_K, 2 Q5_K, 3 Q6_K samples) — bit-exact;
* exact rational arithmetic (``fractions.Fraction``) on random blocks;
* an independently written encoder (the packing side of the 6-bit scale/min
  and the Q6_K ql/qh split, in the package quantizer) round-tripping through
  the decoders, exhaustively over each scale slot;
* special values: d = 0, f16 subnormal and Inf/NaN scales, Q6_K sc = -128.
Q4_0, Q5_0 and IQ4_NL have no reference fixture: they are pinned by exact
rational arithmetic over every code value, closed-form blocks (each element
equal to d times a known integer), the nibble order checked element by
element against the reference's documented rule (element j in the low
nibble of ``qs[j]``, element j + 16 in its high nibble; Q5_0's fifth bit of
element j in bit j of ``qh``), the package quantizer's round trip, and
IQ4_NL's codebook cross-checked as the 16 values Q4_0-style code points take
(kvalues_iq4nl, ``gguf-dequant.ts:29``).  IQ4_XS (no fixture either) is pinned
by exact rational arithmetic, a closed-form superblock that sets each 6-bit
sub-block scale through its scales_l nibble and scales_h bit pair
separately, its equality with eight IQ4_NL blocks of scale d * (ls - 32)
where that scale is an f16, and the quantizer's round trip.  Q2_K (no
fixture) is pinned by exact rational arithmetic, a closed-form superblock
whose every element sits in its own (group, code) cell, and the quantizer's
round trip.  Q3_K likewise (exact rationals with the scale bits read as
fields of a 96-bit integer, a closed-form superblock, the quantizer's round
trip).
``matmul_bt`` is pinned against numpy float64 products and linearity.
"""

from __future__ import annotations

import math

import numpy as np

T_F32, T_F16, T_Q8_0, T_Q4_K, T_Q5_K, T_Q6_K, T_BF16 = 0, 1, 8, 12, 13, 14, 30
T_Q4_0, T_Q5_0, T_IQ4_NL, T_IQ4_XS, T_Q2_K, T_Q3_K = 2, 6, 20, 23, 10, 11
# the grid-codebook IQ types, restated in oracle/gguf_iq.py
_IQ_TYPES = (16, 17, 18, 21, 22, 29)

# kvalues_iq4nl, gguf-dequant.ts:29 (shared by IQ4_NL and IQ4_XS)
KVALUES_IQ4NL = (-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113)

# ---------------------------------------------------------------------------
# Literal restatement (pure Python, f64 arithmetic, f32 store)
# ---------------------------------------------------------------------------


def f16_to_f32(h: int) -> float:
    """IEEE half bits -> value; gguf-dequant.ts:64-71."""
    sign = -1.0 if (h & 0x8000) else 1.0
    exp = (h >> 10) & 0x1F
    frac = h & 0x3FF
    if exp == 0:
        return sign * frac * 2.0 ** -24
    if exp == 0x1F:
        return math.nan if frac else sign * math.inf
    return sign * (1 + frac / 1024) * 2.0 ** (exp - 15)


def _u16(b: bytes, off: int) -> int:
    return b[off] | (b[off + 1] << 8)


def _i8(v: int) -> int:
    return v - 256 if v >= 128 else v


def get_scale_min_k4(j: int, q: bytes, base: int) -> tuple[int, int]:
    """6-bit (scale, min) pair ``j`` of a Q4_K superblock; gguf-dequant.ts:169-176."""
    if j < 4:
        return q[base + j] & 63, q[base + j + 4] & 63
    sc = (q[base + j + 4] & 0x0F) | ((q[base + j - 4] >> 6) << 4)
    m = (q[base + j + 4] >> 4) | ((q[base + j] >> 6) << 4)
    return sc, m


def dequant_q8_0_loop(data: bytes, n: int) -> np.ndarray:
    """gguf-dequant.ts:152-166."""
    if n % 32 != 0:
        raise ValueError(f"[Q8_0] n={n} not divisible by 32")
    out = np.zeros(n, np.float32)
    for b in range(n // 32):
        base = b * 34
        d = f16_to_f32(_u16(data, base))
        for i in range(32):
            out[b * 32 + i] = d * _i8(data[base + 2 + i])
    return out


def dequant_q4_0_loop(data: bytes, n: int) -> np.ndarray:
    """gguf-dequant.ts:110-127."""
    if n % 32 != 0:
        raise ValueError(f"[Q4_0] n={n} not divisible by 32")
    out = np.zeros(n, np.float32)
    for b in range(n // 32):
        base = b * 18
        d = f16_to_f32(_u16(data, base))
        for j in range(16):
            q = data[base + 2 + j]
            out[b * 32 + j] = d * ((q & 0xF) - 8)
            out[b * 32 + j + 16] = d * ((q >> 4) - 8)
    return out


def dequant_q5_0_loop(data: bytes, n: int) -> np.ndarray:
    """gguf-dequant.ts:130-149."""
    if n % 32 != 0:
        raise ValueError(f"[Q5_0] n={n} not divisible by 32")
    out = np.zeros(n, np.float32)
    for b in range(n // 32):
        base = b * 22
        d = f16_to_f32(_u16(data, base))
        qh = _u16(data, base + 2) | (_u16(data, base + 4) << 16)
        for j in range(16):
            q = data[base + 6 + j]
            lo = (q & 0xF) | (((qh >> j) & 1) << 4)
            hi = (q >> 4) | (((qh >> (j + 16)) & 1) << 4)
            out[b * 32 + j] = d * (lo - 16)
            out[b * 32 + j + 16] = d * (hi - 16)
    return out


def dequant_iq4_nl_loop(data: bytes, n: int) -> np.ndarray:
    """gguf-dequant.ts:321-341."""
    if n % 32 != 0:
        raise ValueError(f"[IQ4_NL] n={n} not divisible by 32")
    out = np.zeros(n, np.float32)
    for b in range(n // 32):
        base = b * 18
        d = f16_to_f32(_u16(data, base))
        for j in range(16):
            q = data[base + 2 + j]
            out[b * 32 + j] = d * KVALUES_IQ4NL[q & 0xF]
            out[b * 32 + j + 16] = d * KVALUES_IQ4NL[q >> 4]
    return out


def dequant_q2_k_loop(data: bytes, n: int) -> np.ndarray:
    """gguf-dequant.ts:181-206."""
    if n % 256 != 0:
        raise ValueError(f"[Q2_K] n={n} not divisible by 256")
    out = np.zeros(n, np.float32)
    for b in range(n // 256):
        base = b * 84
        d = f16_to_f32(_u16(data, base + 80))
        mn = f16_to_f32(_u16(data, base + 82))
        oi, is_ = b * 256, 0
        for nn in (0, 128):
            q_base = base + 16 + (nn // 128) * 32
            shift = 0
            for _j in range(4):
                for half in (0, 16):
                    sc = data[base + is_]
                    is_ += 1
                    dl, ml = d * (sc & 0xF), mn * (sc >> 4)
                    for l in range(16):
                        out[oi] = dl * ((data[q_base + half + l] >> shift) & 3) - ml
                        oi += 1
                shift += 2
    return out


def dequant_q3_k_loop(data: bytes, n: int) -> np.ndarray:
    """gguf-dequant.ts:213-252."""
    if n % 256 != 0:
        raise ValueError(f"[Q3_K] n={n} not divisible by 256")
    km1, km2 = 0x03030303, 0x0F0F0F0F
    out = np.zeros(n, np.float32)
    for b in range(n // 256):
        base = b * 110
        d_all = f16_to_f32(_u16(data, base + 108))
        s0 = int.from_bytes(data[base + 96:base + 100], "little")
        s1 = int.from_bytes(data[base + 100:base + 104], "little")
        tmp = int.from_bytes(data[base + 104:base + 108], "little")
        aux2 = ((s0 >> 4) & km2) | (((tmp >> 4) & km1) << 4)
        aux3 = ((s1 >> 4) & km2) | (((tmp >> 6) & km1) << 4)
        aux0 = (s0 & km2) | (((tmp >> 0) & km1) << 4)
        aux1 = (s1 & km2) | (((tmp >> 2) & km1) << 4)
        aux = b"".join(v.to_bytes(4, "little") for v in (aux0, aux1, aux2, aux3))
        oi, is_, m = b * 256, 0, 1
        for nn in (0, 128):
            q_base = base + 32 + (nn // 128) * 32
            shift = 0
            for _j in range(4):
                for half in (0, 16):
                    dl = d_all * (aux[is_] - 32)
                    is_ += 1
                    for l in range(16):
                        q3 = (data[q_base + half + l] >> shift) & 3
                        out[oi] = dl * (q3 - (0 if data[base + half + l] & m else 4))
                        oi += 1
                shift += 2
                m <<= 1
    return out


def dequant_iq4_xs_loop(data: bytes, n: int) -> np.ndarray:
    """gguf-dequant.ts:344-366."""
    if n % 256 != 0:
        raise ValueError(f"[IQ4_XS] n={n} not divisible by 256")
    out = np.zeros(n, np.float32)
    for b in range(n // 256):
        base = b * 136
        d = f16_to_f32(_u16(data, base))
        sh = _u16(data, base + 2)
        y, qs = b * 256, base + 8
        for ib in range(8):
            ls = ((data[base + 4 + (ib >> 1)] >> (4 * (ib & 1))) & 0xF) | (((sh >> (2 * ib)) & 3) << 4)
            dl = d * (ls - 32)
            for j in range(16):
                out[y + j] = dl * KVALUES_IQ4NL[data[qs + j] & 0xF]
                out[y + j + 16] = dl * KVALUES_IQ4NL[data[qs + j] >> 4]
            y += 32
            qs += 16
    return out


def dequant_q4_k_loop(data: bytes, n: int) -> np.ndarray:
    """gguf-dequant.ts:255-281."""
    if n % 256 != 0:
        raise ValueError(f"[Q4_K] n={n} not divisible by 256")
    out = np.zeros(n, np.float32)
    for b in range(n // 256):
        base = b * 144
        d = f16_to_f32(_u16(data, base))
        dmin = f16_to_f32(_u16(data, base + 2))
        scales_base = base + 4
        y = b * 256
        qs = base + 16
        is_ = 0
        for _ in range(0, 256, 64):
            sc1, m1 = get_scale_min_k4(is_ + 0, data, scales_base)
            sc2, m2 = get_scale_min_k4(is_ + 1, data, scales_base)
            d1, min1 = d * sc1, dmin * m1
            d2, min2 = d * sc2, dmin * m2
            for l in range(32):
                out[y + l] = d1 * (data[qs + l] & 0x0F) - min1
            for l in range(32):
                out[y + 32 + l] = d2 * (data[qs + l] >> 4) - min2
            y += 64
            qs += 32
            is_ += 2
    return out


def dequant_q5_k_loop(data: bytes, n: int) -> np.ndarray:
    """gguf-dequant.ts:283-314."""
    if n % 256 != 0:
        raise ValueError(f"[Q5_K] n={n} not divisible by 256")
    out = np.zeros(n, np.float32)
    for b in range(n // 256):
        base = b * 176
        d = f16_to_f32(_u16(data, base))
        dmin = f16_to_f32(_u16(data, base + 2))
        scales_base, qh_base = base + 4, base + 16
        y, ql, is_ = b * 256, base + 48, 0
        u1, u2 = 1, 2
        for _ in range(0, 256, 64):
            sc1, m1 = get_scale_min_k4(is_ + 0, data, scales_base)
            sc2, m2 = get_scale_min_k4(is_ + 1, data, scales_base)
            d1, min1 = d * sc1, dmin * m1
            d2, min2 = d * sc2, dmin * m2
            for l in range(32):
                out[y + l] = d1 * ((data[ql + l] & 0x0F)
                                   + (16 if data[qh_base + l] & u1 else 0)) - min1
            for l in range(32):
                out[y + 32 + l] = d2 * ((data[ql + l] >> 4)
                                        + (16 if data[qh_base + l] & u2 else 0)) - min2
            y += 64
            ql += 32
            is_ += 2
            u1 <<= 2
            u2 <<= 2
    return out


def dequant_q6_k_loop(data: bytes, n: int) -> np.ndarray:
    """gguf-dequant.ts:369-399."""
    if n % 256 != 0:
        raise ValueError(f"[Q6_K] n={n} not divisible by 256")
    out = np.zeros(n, np.float32)
    for b in range(n // 256):
        base = b * 210
        d = f16_to_f32(_u16(data, base + 208))
        y, ql, qh, sc = b * 256, base, base + 128, base + 192
        for _half in range(2):
            for l in range(32):
                is_ = l // 16
                q1 = ((data[ql + l] & 0x0F) | (((data[qh + l] >> 0) & 3) << 4)) - 32
                q2 = ((data[ql + l + 32] & 0x0F) | (((data[qh + l] >> 2) & 3) << 4)) - 32
                q3 = ((data[ql + l] >> 4) | (((data[qh + l] >> 4) & 3) << 4)) - 32
                q4 = ((data[ql + l + 32] >> 4) | (((data[qh + l] >> 6) & 3) << 4)) - 32
                out[y + l] = d * _i8(data[sc + is_]) * q1
                out[y + l + 32] = d * _i8(data[sc + is_ + 2]) * q2
                out[y + l + 64] = d * _i8(data[sc + is_ + 4]) * q3
                out[y + l + 96] = d * _i8(data[sc + is_ + 6]) * q4
            y += 128
            ql += 64
            qh += 32
            sc += 8
    return out


def dequant_ggml_loop(ggml_type: int, data: bytes, n: int) -> np.ndarray:
    """Type switch of gguf-dequant.ts:844-868 (the in-scope types)."""
    data = bytes(data)
    if ggml_type == T_F32:
        return np.frombuffer(data, "<f4", n).astype(np.float32)
    if ggml_type == T_F16:
        return np.array([f16_to_f32(_u16(data, 2 * i)) for i in range(n)], np.float32)
    if ggml_type == T_BF16:
        u = np.frombuffer(data, "<u2", n).astype(np.uint32) << 16
        return u.view(np.float32).copy()
    if ggml_type == T_Q8_0:
        return dequant_q8_0_loop(data, n)
    if ggml_type == T_Q4_0:
        return dequant_q4_0_loop(data, n)
    if ggml_type == T_Q5_0:
        return dequant_q5_0_loop(data, n)
    if ggml_type == T_IQ4_NL:
        return dequant_iq4_nl_loop(data, n)
    if ggml_type == T_IQ4_XS:
        return dequant_iq4_xs_loop(data, n)
    if ggml_type == T_Q2_K:
        return dequant_q2_k_loop(data, n)
    if ggml_type == T_Q3_K:
        return dequant_q3_k_loop(data, n)
    if ggml_type == T_Q4_K:
        return dequant_q4_k_loop(data, n)
    if ggml_type == T_Q5_K:
        return dequant_q5_k_loop(data, n)
    if ggml_type == T_Q6_K:
        return dequant_q6_k_loop(data, n)
    if ggml_type in _IQ_TYPES:
        from oracle import gguf_iq
        return gguf_iq.LOOPS[ggml_type](data, n)
    raise NotImplementedError(f"[GGUF-dequant] No CPU reference for ggml type {ggml_type}")


# ---------------------------------------------------------------------------
# Vectorised restatement (numpy, f32 arithmetic; bit-identical to the loops)
# ---------------------------------------------------------------------------

Q8_0_BLOCK = np.dtype([("d", "<f2"), ("qs", "i1", 32)])
Q4_K_BLOCK = np.dtype([("d", "<f2"), ("dmin", "<f2"), ("scales", "u1", 12), ("qs", "u1", 128)])
Q5_K_BLOCK = np.dtype([("d", "<f2"), ("dmin", "<f2"), ("scales", "u1", 12), ("qh", "u1", 32),
                       ("qs", "u1", 128)])
Q6_K_BLOCK = np.dtype([("ql", "u1", 128), ("qh", "u1", 64), ("sc", "i1", 16), ("d", "<f2")])
assert Q8_0_BLOCK.itemsize == 34 and Q4_K_BLOCK.itemsize == 144 and Q6_K_BLOCK.itemsize == 210
assert Q5_K_BLOCK.itemsize == 176
Q4_0_BLOCK = np.dtype([("d", "<f2"), ("qs", "u1", 16)])           # also IQ4_NL
Q5_0_BLOCK = np.dtype([("d", "<f2"), ("qh", "<u4"), ("qs", "u1", 16)])
Q2_K_BLOCK = np.dtype([("scales", "u1", 16), ("qs", "u1", 64), ("d", "<f2"), ("dmin", "<f2")])
Q3_K_BLOCK = np.dtype([("hmask", "u1", 32), ("qs", "u1", 64), ("scales", "u1", 12), ("d", "<f2")])
IQ4_XS_BLOCK = np.dtype([("d", "<f2"), ("scales_h", "<u2"), ("scales_l", "u1", 4), ("qs", "u1", 128)])
assert Q4_0_BLOCK.itemsize == 18 and Q5_0_BLOCK.itemsize == 22


def _blocks(data, dtype: np.dtype, n: int, block: int, name: str) -> np.ndarray:
    if n % block != 0:
        raise ValueError(f"[{name}] n={n} not divisible by {block}")
    buf = np.frombuffer(data, np.uint8) if not isinstance(data, np.ndarray) else data.reshape(-1)
    nb = n // block
    if buf.size < nb * dtype.itemsize:
        raise ValueError(f"[{name}] byteLength {buf.size} < expected {nb * dtype.itemsize}")
    return buf[: nb * dtype.itemsize].view(dtype)


def q4_k_scale_min(scales: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Vectorised get_scale_min_k4 for all j: ``scales`` (..., 12) u8 -> (sc, m) (..., 8)."""
    s = scales.astype(np.uint8)
    sc = np.empty(s.shape[:-1] + (8,), np.uint8)
    m = np.empty_like(sc)
    sc[..., :4] = s[..., 0:4] & 63
    m[..., :4] = s[..., 4:8] & 63
    sc[..., 4:] = (s[..., 8:12] & 0x0F) | ((s[..., 0:4] >> 6) << 4)
    m[..., 4:] = (s[..., 8:12] >> 4) | ((s[..., 4:8] >> 6) << 4)
    return sc, m


def dequant_q8_0(data, n: int) -> np.ndarray:
    blk = _blocks(data, Q8_0_BLOCK, n, 32, "Q8_0")
    d = blk["d"].astype(np.float32)[:, None]
    return (d * blk["qs"].astype(np.float32)).reshape(-1)


def nibbles32(qs: np.ndarray) -> np.ndarray:
    """4-bit codes of 32-element blocks in element order, (nb, 32): element j < 16 is the
    low nibble of qs[j], element j + 16 the high nibble."""
    return np.concatenate([qs & 0x0F, qs >> 4], axis=1)


def dequant_q4_0(data, n: int) -> np.ndarray:
    blk = _blocks(data, Q4_0_BLOCK, n, 32, "Q4_0")
    d = blk["d"].astype(np.float32)[:, None]
    return (d * (nibbles32(blk["qs"]).astype(np.float32) - 8)).reshape(-1)


def q5_0_values(blk: np.ndarray) -> np.ndarray:
    """Unsigned 5-bit codes of Q5_0 blocks in element order, (nb, 32)."""
    bits = (blk["qh"][:, None] >> np.arange(32, dtype=np.uint32)[None, :]) & 1
    return nibbles32(blk["qs"]).astype(np.uint32) | (bits << 4)


def dequant_q5_0(data, n: int) -> np.ndarray:
    blk = _blocks(data, Q5_0_BLOCK, n, 32, "Q5_0")
    d = blk["d"].astype(np.float32)[:, None]
    return (d * (q5_0_values(blk).astype(np.float32) - 16)).reshape(-1)


def dequant_iq4_nl(data, n: int) -> np.ndarray:
    blk = _blocks(data, Q4_0_BLOCK, n, 32, "IQ4_NL")
    d = blk["d"].astype(np.float32)[:, None]
    table = np.array(KVALUES_IQ4NL, np.float32)
    return (d * table[nibbles32(blk["qs"])]).reshape(-1)


def q2_k_codes(blk: np.ndarray) -> np.ndarray:
    """2-bit codes of Q2_K superblocks in element order, (nb, 256): element
    128 h + 32 j + 16 s + l is bits 2 j of qs[32 h + 16 s + l]."""
    qs = blk["qs"].reshape(-1, 2, 1, 32)                          # (nb, h, 1, 16 s + l)
    shifts = (2 * np.arange(4, dtype=np.uint8)).reshape(1, 1, 4, 1)
    return ((qs >> shifts) & 3).reshape(-1, 256)


def dequant_q2_k(data, n: int) -> np.ndarray:
    blk = _blocks(data, Q2_K_BLOCK, n, 256, "Q2_K")
    d = blk["d"].astype(np.float32)[:, None]
    dmin = blk["dmin"].astype(np.float32)[:, None]
    sc = blk["scales"]
    dl = np.repeat(d * (sc & 0xF).astype(np.float32), 16, axis=1)   # group e // 16
    ml = np.repeat(dmin * (sc >> 4).astype(np.float32), 16, axis=1)
    return (dl * q2_k_codes(blk).astype(np.float32) - ml).reshape(-1)


def q3_k_scales(blk: np.ndarray) -> np.ndarray:
    """The 16 6-bit scales (stored + 32) of Q3_K superblocks, (nb, 16): low nibbles
    are the low / high nibbles of bytes 0-7 (scales 0-7 / 8-15), bits 4-5 of scale i
    are bits 2 (i // 4) of byte 8 + i % 4."""
    a = blk["scales"]
    lo = np.concatenate([a[:, :8] & 15, a[:, :8] >> 4], axis=1)
    i = np.arange(16)
    hi = (a[:, 8 + i % 4] >> (2 * (i // 4))) & 3
    return lo.astype(np.int32) | (hi.astype(np.int32) << 4)


def dequant_q3_k(data, n: int) -> np.ndarray:
    blk = _blocks(data, Q3_K_BLOCK, n, 256, "Q3_K")
    d = blk["d"].astype(np.float32)[:, None]
    dl = np.repeat(d * (q3_k_scales(blk) - 32).astype(np.float32), 16, axis=1)
    low = q2_k_codes(blk)
    hb = (blk["hmask"].reshape(-1, 1, 1, 32) >>
          (4 * np.arange(2, dtype=np.uint8).reshape(1, 2, 1, 1) +
           np.arange(4, dtype=np.uint8).reshape(1, 1, 4, 1))) & 1
    q3 = low.astype(np.int32) + 4 * hb.reshape(-1, 256).astype(np.int32) - 4
    return (dl * q3.astype(np.float32)).reshape(-1)


def iq4_xs_scales(blk: np.ndarray) -> np.ndarray:
    """The eight 6-bit sub-block scales ``ls`` of IQ4_XS superblocks, (nb, 8)."""
    ib = np.arange(8)
    lo = (blk["scales_l"][:, ib >> 1] >> (4 * (ib & 1))) & 0xF
    hi = (blk["scales_h"][:, None].astype(np.uint32) >> (2 * ib)) & 3
    return lo.astype(np.int32) | (hi.astype(np.int32) << 4)


def dequant_iq4_xs(data, n: int) -> np.ndarray:
    blk = _blocks(data, IQ4_XS_BLOCK, n, 256, "IQ4_XS")
    nb = blk.shape[0]
    dl = blk["d"].astype(np.float32)[:, None] * (iq4_xs_scales(blk) - 32).astype(np.float32)
    codes = nibbles32(blk["qs"].reshape(nb * 8, 16)).reshape(nb, 8, 32)
    table = np.array(KVALUES_IQ4NL, np.float32)
    return (dl[:, :, None] * table[codes]).reshape(-1)


def dequant_q4_k(data, n: int) -> np.ndarray:
    blk = _blocks(data, Q4_K_BLOCK, n, 256, "Q4_K")
    nb = blk.shape[0]
    d = blk["d"].astype(np.float32)[:, None]
    dmin = blk["dmin"].astype(np.float32)[:, None]
    sc, m = q4_k_scale_min(blk["scales"])
    d1 = (d * sc.astype(np.float32))[:, :, None]        # exact
    m1 = (dmin * m.astype(np.float32))[:, :, None]      # exact
    qs = blk["qs"].reshape(nb, 4, 1, 32)
    q = np.concatenate([qs & 0x0F, qs >> 4], axis=2).reshape(nb, 8, 32)
    return (d1 * q.astype(np.float32) - m1).reshape(-1)


def q5_k_values(blk: np.ndarray) -> np.ndarray:
    """Unsigned 5-bit codes of Q5_K blocks in element order, shape (nb, 8, 32): sub-block
    2c holds the low nibbles of qs[32c..32c+31] plus 16 x bit 2c of qh[l], sub-block
    2c + 1 the high nibbles plus 16 x bit 2c + 1."""
    nb = blk.shape[0]
    qs = blk["qs"].reshape(nb, 4, 1, 32)
    nib = np.concatenate([qs & 0x0F, qs >> 4], axis=2).reshape(nb, 8, 32)
    bits = (blk["qh"][:, None, :] >> np.arange(8, dtype=np.uint8)[None, :, None]) & 1
    return nib + (bits << 4)


def dequant_q5_k(data, n: int) -> np.ndarray:
    blk = _blocks(data, Q5_K_BLOCK, n, 256, "Q5_K")
    d = blk["d"].astype(np.float32)[:, None]
    dmin = blk["dmin"].astype(np.float32)[:, None]
    sc, m = q4_k_scale_min(blk["scales"])
    d1 = (d * sc.astype(np.float32))[:, :, None]        # exact
    m1 = (dmin * m.astype(np.float32))[:, :, None]      # exact
    return (d1 * q5_k_values(blk).astype(np.float32) - m1).reshape(-1)


def q6_k_values(blk: np.ndarray) -> np.ndarray:
    """Signed 6-bit values (q - 32) of Q6_K blocks in element order, shape (nb, 256)."""
    nb = blk.shape[0]
    ql = blk["ql"].reshape(nb, 2, 64).astype(np.int16)
    qh = blk["qh"].reshape(nb, 2, 32).astype(np.int16)
    lo, hi = ql[:, :, :32], ql[:, :, 32:]
    q = np.stack([
        (lo & 0x0F) | (((qh >> 0) & 3) << 4),
        (hi & 0x0F) | (((qh >> 2) & 3) << 4),
        (lo >> 4) | (((qh >> 4) & 3) << 4),
        (hi >> 4) | (((qh >> 6) & 3) << 4),
    ], axis=2)                                            # (nb, half, t, l)
    return (q - 32).reshape(nb, 256)


def dequant_q6_k(data, n: int) -> np.ndarray:
    blk = _blocks(data, Q6_K_BLOCK, n, 256, "Q6_K")
    nb = blk.shape[0]
    d = blk["d"].astype(np.float32)[:, None]
    # element e of a superblock uses scale index e // 16 (half*8 + 2t + l//16)
    sc = np.repeat(blk["sc"].astype(np.float32), 16, axis=1)   # (nb, 256)
    return ((d * sc) * q6_k_values(blk).astype(np.float32)).reshape(-1)


def dequant_ggml(ggml_type: int, data, n: int) -> np.ndarray:
    """Vectorised dequantization of raw GGUF bytes to f32 (gguf-dequant.ts:844-868)."""
    if ggml_type == T_Q8_0:
        return dequant_q8_0(data, n)
    if ggml_type == T_Q4_0:
        return dequant_q4_0(data, n)
    if ggml_type == T_Q5_0:
        return dequant_q5_0(data, n)
    if ggml_type == T_IQ4_NL:
        return dequant_iq4_nl(data, n)
    if ggml_type == T_IQ4_XS:
        return dequant_iq4_xs(data, n)
    if ggml_type == T_Q2_K:
        return dequant_q2_k(data, n)
    if ggml_type == T_Q3_K:
        return dequant_q3_k(data, n)
    if ggml_type == T_Q4_K:
        return dequant_q4_k(data, n)
    if ggml_type == T_Q5_K:
        return dequant_q5_k(data, n)
    if ggml_type == T_Q6_K:
        return dequant_q6_k(data, n)
    if ggml_type in _IQ_TYPES:
        from oracle import gguf_iq
        return gguf_iq.VECTORISED[ggml_type](data, n)
    if ggml_type in (T_F32, T_F16, T_BF16):
        return dequant_ggml_loop(ggml_type, bytes(np.frombuffer(data, np.uint8)), n)
    raise NotImplementedError(f"[GGUF-dequant] No CPU reference for ggml type {ggml_type}")


def dequant_rows(ggml_type: int, raw: np.ndarray, n_rows: int, k: int) -> np.ndarray:
    """Dequantize a row-major [n_rows, k] weight from its raw GGUF bytes."""
    return dequant_ggml(ggml_type, raw, n_rows * k).reshape(n_rows, k)


# ---------------------------------------------------------------------------
# Matmul reference and the parity gate
# ---------------------------------------------------------------------------


def matmul_bt(a: np.ndarray, w: np.ndarray) -> np.ndarray:
    """``C[m, n] = sum_k a[m, k] * w[n, k]`` accumulated in f64 (kernel-tests.ts:98-110).

    Returns the f64 result; the reference stores it to f32, ``.astype(np.float32)``.
    """
    return np.asarray(a, np.float64) @ np.asarray(w, np.float64).T


def matmul_bt_abs(a: np.ndarray, w: np.ndarray) -> np.ndarray:
    """``sum_k |a[m, k] * w[n, k]|`` — the scale of the per-element error bound."""
    return np.abs(np.asarray(a, np.float64)) @ np.abs(np.asarray(w, np.float64)).T


REL_TOL = 1e-3


def parity_metrics(y, y_ref, sum_abs) -> dict:
    """Both gates of the path: normwise and per-element relative error.

    normwise  = ||y - y_ref||_2 / ||y_ref||_2                       (<= 1e-3)
    elemwise  = max |y - y_ref| / sum_k |x_k w_nk|                  (<= 1e-3)
    """
    y = np.asarray(y, np.float64)
    y_ref = np.asarray(y_ref, np.float64)
    sum_abs = np.asarray(sum_abs, np.float64)
    err = np.abs(y - y_ref)
    denom = np.linalg.norm(y_ref)
    normwise = float(np.linalg.norm(y - y_ref) / denom) if denom > 0 else float(np.linalg.norm(y - y_ref))
    with np.errstate(divide="ignore", invalid="ignore"):
        ratio = np.where(sum_abs > 0, err / sum_abs, np.where(err > 0, np.inf, 0.0))
    finite = bool(np.all(np.isfinite(y)))
    return {
        "normwise": normwise,
        "elemwise": float(ratio.max()) if ratio.size else 0.0,
        "max_abs": float(err.max()) if err.size else 0.0,
        "finite": finite,
        "ok": finite and normwise <= REL_TOL and (float(ratio.max()) if ratio.size else 0.0) <= REL_TOL,
    }


def same_bits(a: np.ndarray, b: np.ndarray) -> bool:
    """Bitwise f32 equality, NaN == NaN (any payload), +0 != -0."""
    a = np.ascontiguousarray(a, np.float32).reshape(-1)
    b = np.ascontiguousarray(b, np.float32).reshape(-1)
    if a.shape != b.shape:
        return False
    na, nb_ = np.isnan(a), np.isnan(b)
    if not np.array_equal(na, nb_):
        return False
    return bool(np.array_equal(a.view(np.uint32)[~na], b.view(np.uint32)[~nb_]))
