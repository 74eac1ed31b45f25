"""CPU oracle for the grid-codebook IQ types: IQ2_XXS, IQ2_XS, IQ2_S, IQ3_XXS,
IQ3_S and IQ1_M.

TEST INFRASTRUCTURE ONLY, like ``gguf_ref`` (which dispatches to this module):
only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import it.  The product path never calls it.

It restates the reference's CPU dequantization of these types
(``webgpu/src/model/gguf-dequant.ts:406-672``) twice:

* ``*_loop``: the TypeScript loops line for line, in Python floats (IEEE f64,
  as JavaScript numbers), rounded once to f32 on store.  Small inputs only.
* vectorised numpy, in f64 and rounded once to f32.

Every value of these formats is exact in f32: a superblock scale d (an f16,
11 significant bits) times a sub-block factor with at most 6 significant bits
(IQ2 (0.5 + ls) / 4, IQ3_XXS (0.5 + ls) / 2, IQ3_S 1 + 2 s, IQ1_M 2 s + 1),
times a grid magnitude of at most 6 bits (IQ2 {8, 25, 43}, IQ3_XXS
{4, 12, ..., 62}, IQ3_S odd values up to 15) or, for IQ1_M, an int8 grid
value in {-1, 0, 1} plus the +-1/8 delta.
So the loops and the vectorised functions agree bit for bit, and both agree
bit for bit with gguf-py.

The grids and the ksigns table are data: ``tests/golden/iq_grids.json``,
extracted from the byte arrays of the reference's CPU dequant (they restate
the ``iq2xxs_grid`` ... ``iq1s_grid`` and ``ksigns_iq2xs`` tables of ggml's
``ggml-common.h``).

Parity pins (``tests/test_oracle_iq.py``): the reference's IQ parity fixture
(``webgpu/scripts/iq_parity_fixture.json``, gguf-py output on four random
blocks of each type) bit for bit, for both restatements; the loops against the
vectorised functions on further random blocks; closed-form blocks whose
elements are known products; the grids' shapes and value sets and the
ksigns parity rule.
"""

from __future__ import annotations

import json
import os

import numpy as np

T_IQ2_XXS, T_IQ2_XS, T_IQ3_XXS, T_IQ3_S, T_IQ2_S, T_IQ1_M = 16, 17, 18, 21, 22, 29
IQ_TYPES = (T_IQ2_XXS, T_IQ2_XS, T_IQ2_S, T_IQ3_XXS, T_IQ3_S, T_IQ1_M)
BLOCK_BYTES = {T_IQ2_XXS: 66, T_IQ2_XS: 74, T_IQ2_S: 82, T_IQ3_XXS: 98, T_IQ3_S: 110, T_IQ1_M: 56}
NAMES = {T_IQ2_XXS: "IQ2_XXS", T_IQ2_XS: "IQ2_XS", T_IQ2_S: "IQ2_S", T_IQ3_XXS: "IQ3_XXS",
         T_IQ3_S: "IQ3_S", T_IQ1_M: "IQ1_M"}

_GRIDS_JSON = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))),
                           "tests", "golden", "iq_grids.json")


def load_grids(path: str = _GRIDS_JSON) -> dict:
    """The codebooks as numpy arrays: ``iq2xxs`` (256, 8) u8, ``iq2xs`` (512, 8),
    ``iq2s`` (1024, 8), ``iq3xxs`` (256, 4), ``iq3s`` (512, 4), ``iq1s``
    (2048, 8) i8, ``ksigns`` (128,) u8, and ``delta`` (IQ1 grid shift)."""
    with open(path, encoding="utf-8") as f:
        fx = json.load(f)
    g = fx["grids"]

    def arr(key, width, dtype):
        return np.asarray(g[key]["values"], dtype).reshape(-1, width)
    return {
        "iq2xxs": arr("iq2xxs_grid", 8, np.uint8), "iq2xs": arr("iq2xs_grid", 8, np.uint8),
        "iq2s": arr("iq2s_grid", 8, np.uint8), "iq3xxs": arr("iq3xxs_grid", 4, np.uint8),
        "iq3s": arr("iq3s_grid", 4, np.uint8), "iq1s": arr("iq1s_grid", 8, np.int8),
        "ksigns": np.asarray(g["ksigns_iq2xs"]["values"], np.uint8),
        "delta": float(fx["iq1_delta"]),
    }


_G = None


def grids() -> dict:
    global _G
    if _G is None:
        _G = load_grids()
    return _G


def _f16(b: bytes, off: int) -> float:
    return float(np.frombuffer(b[off:off + 2], "<f2")[0])


def _u16(b: bytes, off: int) -> int:
    return b[off] | (b[off + 1] << 8)


def _u32(b: bytes, off: int) -> int:
    return b[off] | (b[off + 1] << 8) | (b[off + 2] << 16) | (b[off + 3] << 24)


def _check(name: str, n: int, data: bytes, bs: int) -> int:
    if n % 256 != 0:
        raise ValueError(f"[{name}] n={n} not divisible by 256")
    nb = n // 256
    if len(data) < nb * bs:
        raise ValueError(f"[{name}] byteLength {len(data)} < expected {nb * bs}")
    return nb


# ---------------------------------------------------------------------------
# Literal restatement (pure Python, f64 arithmetic, f32 store)
# ---------------------------------------------------------------------------


def dequant_iq2_xxs_loop(data: bytes, n: int) -> np.ndarray:
    """gguf-dequant.ts:406-431."""
    G, data = grids(), bytes(data)
    nb = _check("IQ2_XXS", n, data, 66)
    out = np.zeros(n, np.float32)
    for b in range(nb):
        base = b * 66
        d = _f16(data, base)
        for ib in range(8):
            g = base + 2 + ib * 8
            aux1 = _u32(data, g + 4)
            db = d * (0.5 + (aux1 >> 28)) * 0.25
            y = b * 256 + ib * 32
            for l in range(4):
                idx = data[g + l]
                signs = int(G["ksigns"][(aux1 >> (7 * l)) & 127])
                for j in range(8):
                    sign = -1 if (signs >> j) & 1 else 1
                    out[y + l * 8 + j] = db * int(G["iq2xxs"][idx, j]) * sign
    return out


def dequant_iq2_xs_loop(data: bytes, n: int) -> np.ndarray:
    """gguf-dequant.ts:440-470."""
    G, data = grids(), bytes(data)
    nb = _check("IQ2_XS", n, data, 74)
    out = np.zeros(n, np.float32)
    for b in range(nb):
        base = b * 74
        d = _f16(data, base)
        for ib in range(8):
            sc = data[base + 66 + ib]
            db0 = d * (0.5 + (sc & 0xF)) * 0.25
            db1 = d * (0.5 + (sc >> 4)) * 0.25
            y = b * 256 + ib * 32
            for l in range(4):
                q = _u16(data, base + 2 + 2 * (4 * ib + l))
                idx, signs = q & 511, int(G["ksigns"][q >> 9])
                dl = db0 if l < 2 else db1
                for j in range(8):
                    sign = -1 if signs & (1 << j) else 1
                    out[y + l * 8 + j] = dl * int(G["iq2xs"][idx, j]) * sign
    return out


def dequant_iq1_m_loop(data: bytes, n: int) -> np.ndarray:
    """gguf-dequant.ts:478-524."""
    G, data = grids(), bytes(data)
    nb = _check("IQ1_M", n, data, 56)
    delta0 = G["delta"]
    out = np.zeros(n, np.float32)
    for b in range(nb):
        base = b * 56
        sc = [_u16(data, base + 48 + 2 * i) for i in range(4)]
        bits = ((sc[0] >> 12) | ((sc[1] >> 8) & 0x00F0) | ((sc[2] >> 4) & 0x0F00)
                | (sc[3] & 0xF000)) & 0xFFFF
        d = float(np.array([bits], np.uint16).view(np.float16)[0])
        for ib in range(8):
            w = sc[ib >> 1]
            sh = 6 * (ib & 1)
            dl1 = d * (2 * ((w >> sh) & 7) + 1)
            dl2 = d * (2 * ((w >> (sh + 3)) & 7) + 1)
            qs = base + ib * 4
            qh0, qh1 = data[base + 32 + ib * 2], data[base + 32 + ib * 2 + 1]
            idx = [data[qs] | ((qh0 << 8) & 0x700), data[qs + 1] | ((qh0 << 4) & 0x700),
                   data[qs + 2] | ((qh1 << 8) & 0x700), data[qs + 3] | ((qh1 << 4) & 0x700)]
            delta = [-delta0 if qh0 & 0x08 else delta0, -delta0 if qh0 & 0x80 else delta0,
                     -delta0 if qh1 & 0x08 else delta0, -delta0 if qh1 & 0x80 else delta0]
            y = b * 256 + ib * 32
            for l in range(4):
                dl = dl1 if l < 2 else dl2
                for j in range(8):
                    out[y + l * 8 + j] = dl * (int(G["iq1s"][idx[l], j]) + delta[l])
    return out


def dequant_iq3_xxs_loop(data: bytes, n: int) -> np.ndarray:
    """gguf-dequant.ts:532-561."""
    G, data = grids(), bytes(data)
    nb = _check("IQ3_XXS", n, data, 98)
    out = np.zeros(n, np.float32)
    for b in range(nb):
        base = b * 98
        d = _f16(data, base)
        for ib in range(8):
            aux32 = _u32(data, base + 66 + 4 * ib)
            db = d * (0.5 + (aux32 >> 28)) * 0.5
            y = b * 256 + ib * 32
            q = base + 2 + ib * 8
            for l in range(4):
                signs = int(G["ksigns"][(aux32 >> (7 * l)) & 127])
                g1, g2 = data[q + 2 * l], data[q + 2 * l + 1]
                for j in range(4):
                    s1 = -1 if signs & (1 << j) else 1
                    s2 = -1 if signs & (1 << (j + 4)) else 1
                    out[y + j] = db * int(G["iq3xxs"][g1, j]) * s1
                    out[y + j + 4] = db * int(G["iq3xxs"][g2, j]) * s2
                y += 8
    return out


def dequant_iq3_s_loop(data: bytes, n: int) -> np.ndarray:
    """gguf-dequant.ts:569-613."""
    G, data = grids(), bytes(data)
    nb = _check("IQ3_S", n, data, 110)
    out = np.zeros(n, np.float32)
    for b in range(nb):
        base = b * 110
        d = _f16(data, base)
        y = b * 256
        for p in range(4):
            sc = data[base + 106 + p]
            for half, (db, qh, qs, sg) in enumerate((
                    (d * (1 + 2 * (sc & 0xF)), data[base + 66 + 2 * p], base + 2 + p * 16,
                     base + 74 + p * 8),
                    (d * (1 + 2 * (sc >> 4)), data[base + 66 + 2 * p + 1], base + 2 + p * 16 + 8,
                     base + 74 + p * 8 + 4))):
                for l in range(4):
                    g1 = data[qs + 2 * l] | ((qh << (8 - 2 * l)) & 256)
                    g2 = data[qs + 2 * l + 1] | ((qh << (7 - 2 * l)) & 256)
                    s = data[sg + l]
                    for j in range(4):
                        out[y + j] = db * int(G["iq3s"][g1, j]) * (-1 if s & (1 << j) else 1)
                        out[y + j + 4] = db * int(G["iq3s"][g2, j]) * (-1 if s & (1 << (j + 4)) else 1)
                    y += 8
    return out


def dequant_iq2_s_loop(data: bytes, n: int) -> np.ndarray:
    """gguf-dequant.ts:621-648."""
    G, data = grids(), bytes(data)
    nb = _check("IQ2_S", n, data, 82)
    out = np.zeros(n, np.float32)
    for b in range(nb):
        base = b * 82
        d = _f16(data, base)
        for ib in range(8):
            sc = data[base + 74 + ib]
            db0 = d * (0.5 + (sc & 0xF)) * 0.25
            db1 = d * (0.5 + (sc >> 4)) * 0.25
            qh = data[base + 66 + ib]
            y = b * 256 + ib * 32
            for l in range(4):
                dl = db0 if l < 2 else db1
                g = data[base + 2 + ib * 4 + l] | ((qh << (8 - 2 * l)) & 0x300)
                sg = data[base + 34 + ib * 4 + l]
                for j in range(8):
                    out[y + l * 8 + j] = dl * int(G["iq2s"][g, j]) * (-1 if sg & (1 << j) else 1)
    return out


LOOPS = {T_IQ2_XXS: dequant_iq2_xxs_loop, T_IQ2_XS: dequant_iq2_xs_loop,
         T_IQ2_S: dequant_iq2_s_loop, T_IQ3_XXS: dequant_iq3_xxs_loop,
         T_IQ3_S: dequant_iq3_s_loop, T_IQ1_M: dequant_iq1_m_loop}


# ---------------------------------------------------------------------------
# Vectorised restatement (numpy, f64 then one rounding to f32)
# ---------------------------------------------------------------------------


def _raw_blocks(data, ggml_type: int, n: int) -> np.ndarray:
    bs = BLOCK_BYTES[ggml_type]
    buf = np.frombuffer(bytes(data), np.uint8) if not isinstance(data, np.ndarray) else data.reshape(-1)
    nb = _check(NAMES[ggml_type], n, buf, bs)
    return buf[:nb * bs].reshape(nb, bs)


def _f16_col(blk: np.ndarray, off: int) -> np.ndarray:
    return np.ascontiguousarray(blk[:, off:off + 2]).view("<f2")[:, 0].astype(np.float64)


def _u32_cols(blk: np.ndarray, off: int, count: int) -> np.ndarray:
    return np.ascontiguousarray(blk[:, off:off + 4 * count]).view("<u4").astype(np.int64)


def _sign_bits(signs: np.ndarray, width: int = 8) -> np.ndarray:
    """(..., ) sign bytes -> (..., width) of +-1 (bit j set -> -1)."""
    bits = (signs[..., None].astype(np.int64) >> np.arange(width)) & 1
    return 1 - 2 * bits


def dequant_iq2_xxs(data, n: int) -> np.ndarray:
    G = grids()
    blk = _raw_blocks(data, T_IQ2_XXS, n)
    d = _f16_col(blk, 0)
    qs = blk[:, 2:66].reshape(-1, 8, 8)                               # (nb, ib, 8 bytes)
    aux1 = np.ascontiguousarray(qs[:, :, 4:8]).view("<u4")[..., 0].astype(np.int64)   # (nb, ib)
    db = d[:, None] * (0.5 + (aux1 >> 28)) * 0.25
    sidx = (aux1[..., None] >> (7 * np.arange(4))) & 127                # (nb, ib, l)
    sg = _sign_bits(G["ksigns"][sidx])                                 # (nb, ib, l, 8)
    mag = G["iq2xxs"][qs[:, :, 0:4]].astype(np.float64)                # (nb, ib, l, 8)
    return (db[:, :, None, None] * mag * sg).astype(np.float32).reshape(-1)


def dequant_iq2_xs(data, n: int) -> np.ndarray:
    G = grids()
    blk = _raw_blocks(data, T_IQ2_XS, n)
    d = _f16_col(blk, 0)
    q = np.ascontiguousarray(blk[:, 2:66]).view("<u2").astype(np.int64).reshape(-1, 8, 4)
    sc = blk[:, 66:74].astype(np.int64)                                # (nb, ib)
    nib = np.stack([sc & 0xF, sc & 0xF, sc >> 4, sc >> 4], axis=2)     # (nb, ib, l)
    dl = d[:, None, None] * (0.5 + nib) * 0.25
    mag = G["iq2xs"][q & 511].astype(np.float64)
    sg = _sign_bits(G["ksigns"][q >> 9])
    return (dl[..., None] * mag * sg).astype(np.float32).reshape(-1)


def dequant_iq2_s(data, n: int) -> np.ndarray:
    G = grids()
    blk = _raw_blocks(data, T_IQ2_S, n)
    d = _f16_col(blk, 0)
    qs = blk[:, 2:34].astype(np.int64).reshape(-1, 8, 4)
    sgn = blk[:, 34:66].reshape(-1, 8, 4)
    qh = blk[:, 66:74].astype(np.int64)
    sc = blk[:, 74:82].astype(np.int64)
    l = np.arange(4)
    idx = qs | ((qh[..., None] << (8 - 2 * l)) & 0x300)
    nib = np.stack([sc & 0xF, sc & 0xF, sc >> 4, sc >> 4], axis=2)
    dl = d[:, None, None] * (0.5 + nib) * 0.25
    mag = G["iq2s"][idx].astype(np.float64)
    return (dl[..., None] * mag * _sign_bits(sgn)).astype(np.float32).reshape(-1)


def dequant_iq3_xxs(data, n: int) -> np.ndarray:
    G = grids()
    blk = _raw_blocks(data, T_IQ3_XXS, n)
    d = _f16_col(blk, 0)
    qs = blk[:, 2:66].reshape(-1, 8, 4, 2)                             # (nb, ib, l, two indices)
    aux = _u32_cols(blk, 66, 8)                                        # (nb, ib)
    db = d[:, None] * (0.5 + (aux >> 28)) * 0.5
    sidx = (aux[..., None] >> (7 * np.arange(4))) & 127
    sg = _sign_bits(G["ksigns"][sidx])                                 # (nb, ib, l, 8)
    mag = G["iq3xxs"][qs].astype(np.float64).reshape(-1, 8, 4, 8)      # two entries of 4
    return (db[:, :, None, None] * mag * sg).astype(np.float32).reshape(-1)


def dequant_iq3_s(data, n: int) -> np.ndarray:
    G = grids()
    blk = _raw_blocks(data, T_IQ3_S, n)
    d = _f16_col(blk, 0)
    qs = blk[:, 2:66].astype(np.int64).reshape(-1, 8, 4, 2)            # ib = 2p + half
    qh = blk[:, 66:74].astype(np.int64)                                # (nb, ib)
    sgn = blk[:, 74:106].reshape(-1, 8, 4)
    sc = blk[:, 106:110].astype(np.int64)
    l = np.arange(4)
    g1 = qs[..., 0] | ((qh[..., None] << (8 - 2 * l)) & 256)
    g2 = qs[..., 1] | ((qh[..., None] << (7 - 2 * l)) & 256)
    mag = np.concatenate([G["iq3s"][g1], G["iq3s"][g2]], axis=-1).astype(np.float64)
    nib = np.stack([sc & 0xF, sc >> 4], axis=2).reshape(-1, 8)         # (nb, ib)
    db = d[:, None] * (1 + 2 * nib)
    return (db[:, :, None, None] * mag * _sign_bits(sgn)).astype(np.float32).reshape(-1)


def dequant_iq1_m(data, n: int) -> np.ndarray:
    G = grids()
    blk = _raw_blocks(data, T_IQ1_M, n)
    sc = np.ascontiguousarray(blk[:, 48:56]).view("<u2").astype(np.int64)   # (nb, 4)
    bits = ((sc[:, 0] >> 12) | ((sc[:, 1] >> 8) & 0x00F0) | ((sc[:, 2] >> 4) & 0x0F00)
            | (sc[:, 3] & 0xF000)) & 0xFFFF
    d = bits.astype(np.uint16).view(np.float16).astype(np.float64)
    ib = np.arange(8)
    w = sc[:, ib >> 1]                                                 # (nb, ib)
    sh = 6 * (ib & 1)
    s = np.stack([(w >> sh) & 7, (w >> sh) & 7, (w >> (sh + 3)) & 7, (w >> (sh + 3)) & 7], axis=2)
    dl = d[:, None, None] * (2 * s + 1)                                # (nb, ib, l)
    qs = blk[:, 0:32].astype(np.int64).reshape(-1, 8, 4)
    qh = blk[:, 32:48].astype(np.int64).reshape(-1, 8, 2)
    hi = np.stack([(qh[..., 0] << 8) & 0x700, (qh[..., 0] << 4) & 0x700,
                   (qh[..., 1] << 8) & 0x700, (qh[..., 1] << 4) & 0x700], axis=2)
    neg = np.stack([qh[..., 0] & 0x08, qh[..., 0] & 0x80, qh[..., 1] & 0x08, qh[..., 1] & 0x80],
                   axis=2) != 0
    delta = np.where(neg, -G["delta"], G["delta"])
    val = G["iq1s"][qs | hi].astype(np.float64) + delta[..., None]
    return (dl[..., None] * val).astype(np.float32).reshape(-1)


VECTORISED = {T_IQ2_XXS: dequant_iq2_xxs, T_IQ2_XS: dequant_iq2_xs, T_IQ2_S: dequant_iq2_s,
              T_IQ3_XXS: dequant_iq3_xxs, T_IQ3_S: dequant_iq3_s, T_IQ1_M: dequant_iq1_m}


def random_blocks(ggml_type: int, n_blocks: int, seed: int, d: float = 0.0625) -> np.ndarray:
    """Random valid blocks (every bit pattern is a legal code) with the
    superblock scale set to the f16 ``d`` (for IQ1_M, whose scale is spread
    over the top nibbles of its four scale words: those nibbles), so that no
    block decodes to Inf / NaN.  Follows the reference's fixture recipe
    (webgpu/scripts/gen_iq_parity_fixture.py:39-57)."""
    bs = BLOCK_BYTES[ggml_type]
    rng = np.random.default_rng(seed)
    raw = rng.integers(0, 256, size=(n_blocks, bs), dtype=np.uint8)
    dh = np.array([d], np.float16).view(np.uint16)[0]
    if ggml_type != T_IQ1_M:
        raw[:, 0] = dh & 0xFF
        raw[:, 1] = dh >> 8
    else:
        words = raw[:, 48:56].copy().view("<u2").astype(np.int64)
        for k in range(4):
            words[:, k] = (words[:, k] & 0x0FFF) | (((int(dh) >> (4 * k)) & 0xF) << 12)
        raw[:, 48:56] = words.astype("<u2").view(np.uint8).reshape(n_blocks, 8)
    return raw.reshape(-1)
