"""numpy model of the HBM row-tile layout (test helper; the layout is defined
in ``artifex-assistantv5_amd/csrc/common.hpp`` and ``include/gguf_hip.h``).

Rows are grouped in tiles of 16; per unit of K (Q4_K / Q6_K superblock, Q8_0
block) a tile stores the 16 rows' GGUF blocks interleaved:

* Q4_K: [header of row r at 16 r] then piece (cp, g, r) at 256 + ((4 cp + g) 16 + r) 16
  = qs[64 cp + 8 g, +8) | qs[64 cp + 32 + 8 g, +8)
* Q5_K: as Q4_K (qs from byte 48 of the block), then piece (g, r) at 2304 + (16 g + r) 8
  = qh[8 g, +8)
* Q6_K: piece (v, g, r) at ((4 v + g) 16 + r) 16 = the lane's quant dwords 4v..4v+3,
  dword 3i = ql[64 hf + 16 lh + 4 g, +4), 3i+1 = ql[64 hf + 32 + 16 lh + 4 g, +4),
  3i+2 = qh[32 hf + 16 lh + 4 g, +4) for i = 2 hf + lh; scales at 3072 + 16 r; d at 3328 + 2 r
* Q8_0: d at 2 r, then piece (g, r) at 32 + (16 g + r) 8 = qs[8 g, +8)
* Q4_0 / IQ4_NL: d at 2 r, then word (g, r) at 32 + (16 g + r) 4 whose byte i holds the
  codes of block elements 8 g + i (low nibble) and 8 g + 4 + i (high nibble); element j
  of a GGUF block is the low nibble of qs[j] (j < 16) or the high nibble of qs[j - 16]
* Q5_0: d at 2 r, qh at 32 + 4 r, then the code words at 96 + (16 g + r) 4 as Q4_0
* Q2_K: scales[16] at 16 r, d | dmin at 256 + 4 r, then piece (g, r) at 320 + (16 g + r) 16
  = qs[8 g, +8) | qs[32 + 8 g, +8)
* Q3_K: scales[12] at 12 r, d at 192 + 2 r, hmask piece (g, r) at 224 + (16 g + r) 8 =
  hmask[8 g, +8), qs piece (g, r) at 736 + (16 g + r) 16 as Q2_K
* IQ4_XS: header (d, scales_h, scales_l) at 8 r, then piece (g, r) at 128 + (16 g + r) 32
  whose word j holds sub-block j's codes 8 g .. 8 g + 7 as Q4_0 (sub-block j's 16 code
  bytes start at byte 8 + 16 j of the GGUF block)
* IQ2_XXS, IQ2_XS, IQ2_S, IQ3_XXS, IQ3_S (block bytes BS, f16 d first): d at 2 r, then
  the block's bytes 2 .. BS - 1 at 32 + r (BS - 2)
* IQ1_M (no d field): row r's block at 56 r
"""

import numpy as np

BLOCK = {8: (32, 34), 12: (256, 144), 13: (256, 176), 14: (256, 210), 2: (32, 18), 6: (32, 22),
         20: (32, 18), 23: (256, 136), 10: (256, 84), 11: (256, 110),
         16: (256, 66), 17: (256, 74), 22: (256, 82), 18: (256, 98), 21: (256, 110),
         29: (256, 56)}
GRID = (16, 17, 22, 18, 21, 29)
SMALL = (2, 6, 20, 23)      # nibble codes regrouped per lane (not a byte permutation)


def tile_row_bytes(t, k):
    block, size = BLOCK[t]
    return size * (k // block)


def tiled_rows(n):
    return -(-n // 16) * 16


def tiled_bytes(t, n, k):
    return tiled_rows(n) * tile_row_bytes(t, k)


def _unit_maps(t):
    """(dst, src) byte index arrays: tile-unit byte dst[i] = row r's block byte src[i], as
    arrays of shape (16, UB) giving the tile-unit offset of each (row, block byte)."""
    block, ub = BLOCK[t]
    pos = np.zeros((16, ub), np.int64)
    for r in range(16):
        if t == 29:
            pos[r] = ub * r + np.arange(ub)
        elif t in GRID:
            pos[r, 0:2] = 2 * r + np.arange(2)
            pos[r, 2:] = 32 + r * (ub - 2) + np.arange(ub - 2)
        elif t in (12, 13):
            qs = 16 if t == 12 else 48
            pos[r, 0:16] = 16 * r + np.arange(16)
            for cp in range(2):
                for g in range(4):
                    base = 256 + ((4 * cp + g) * 16 + r) * 16
                    pos[r, qs + 64 * cp + 8 * g + np.arange(8)] = base + np.arange(8)
                    pos[r, qs + 64 * cp + 32 + 8 * g + np.arange(8)] = base + 8 + np.arange(8)
            if t == 13:
                for g in range(4):
                    pos[r, 16 + 8 * g + np.arange(8)] = 2304 + (16 * g + r) * 8 + np.arange(8)
        elif t == 11:
            pos[r, 96:108] = 12 * r + np.arange(12)                     # scales
            pos[r, 108:110] = 192 + 2 * r + np.arange(2)                # d
            for g in range(4):
                pos[r, 8 * g + np.arange(8)] = 224 + (16 * g + r) * 8 + np.arange(8)   # hmask
                base = 736 + (16 * g + r) * 16
                pos[r, 32 + 8 * g + np.arange(8)] = base + np.arange(8)
                pos[r, 32 + 32 + 8 * g + np.arange(8)] = base + 8 + np.arange(8)
        elif t == 10:
            pos[r, 0:16] = 16 * r + np.arange(16)                       # scales
            pos[r, 80:84] = 256 + 4 * r + np.arange(4)                  # d, dmin
            for g in range(4):
                base = 320 + (16 * g + r) * 16
                pos[r, 16 + 8 * g + np.arange(8)] = base + np.arange(8)
                pos[r, 16 + 32 + 8 * g + np.arange(8)] = base + 8 + np.arange(8)
        elif t == 14:
            for g in range(4):
                for i in range(4):
                    hf, lh = i >> 1, i & 1
                    srcs = [64 * hf + 16 * lh + 4 * g, 64 * hf + 32 + 16 * lh + 4 * g,
                            128 + 32 * hf + 16 * lh + 4 * g]
                    for j, src in enumerate(srcs):
                        dwi = 3 * i + j
                        base = ((4 * (dwi // 4) + g) * 16 + r) * 16 + 4 * (dwi % 4)
                        pos[r, src + np.arange(4)] = base + np.arange(4)
            pos[r, 192:208] = 3072 + 16 * r + np.arange(16)
            pos[r, 208:210] = 3328 + 2 * r + np.arange(2)
        else:
            pos[r, 0:2] = 2 * r + np.arange(2)
            for g in range(4):
                pos[r, 2 + 8 * g + np.arange(8)] = 32 + (16 * g + r) * 8 + np.arange(8)
    assert np.array_equal(np.sort(pos.reshape(-1)), np.arange(16 * ub))
    return pos


def _word(codes, g):
    """Byte i of lane group g's word: codes 8 g + i (low nibble), 8 g + 4 + i (high)."""
    return [codes[..., 8 * g + i] | (codes[..., 8 * g + 4 + i] << 4) for i in range(4)]


def _small_to_unit(t, blk):
    """(..., 16 rows, UB) raw blocks -> (..., 16 * UB) tile-unit bytes."""
    sh = blk.shape[:-2]
    out = np.zeros(sh + (16 * BLOCK[t][1],), np.uint8)
    if t == 23:
        for r in range(16):
            out[..., 8 * r:8 * r + 8] = blk[..., r, 0:8]
            for j in range(8):
                qs = blk[..., r, 8 + 16 * j:24 + 16 * j]
                codes = np.concatenate([qs & 15, qs >> 4], axis=-1)
                for g in range(4):
                    base = 128 + (16 * g + r) * 32 + 4 * j
                    for i, b in enumerate(_word(codes, g)):
                        out[..., base + i] = b
        return out
    qs = blk[..., 6:] if t == 6 else blk[..., 2:]
    codes = np.concatenate([qs & 15, qs >> 4], axis=-1)          # (..., 16, 32) element order
    off = 96 if t == 6 else 32
    for r in range(16):
        out[..., 2 * r:2 * r + 2] = blk[..., r, 0:2]
        if t == 6:
            out[..., 32 + 4 * r:36 + 4 * r] = blk[..., r, 2:6]
        for g in range(4):
            base = off + (16 * g + r) * 4
            for i in range(4):
                out[..., base + i] = codes[..., r, 8 * g + i] | (codes[..., r, 8 * g + 4 + i] << 4)
    return out


def _small_from_unit(t, tu):
    """Inverse of _small_to_unit: (..., 16 * UB) -> (..., 16, UB)."""
    sh = tu.shape[:-1]
    ub = BLOCK[t][1]
    blk = np.zeros(sh + (16, ub), np.uint8)
    if t == 23:
        for r in range(16):
            blk[..., r, 0:8] = tu[..., 8 * r:8 * r + 8]
            for j in range(8):
                codes = np.zeros(sh + (32,), np.uint8)
                for g in range(4):
                    base = 128 + (16 * g + r) * 32 + 4 * j
                    for i in range(4):
                        b = tu[..., base + i]
                        codes[..., 8 * g + i] = b & 15
                        codes[..., 8 * g + 4 + i] = b >> 4
                blk[..., r, 8 + 16 * j:24 + 16 * j] = codes[..., :16] | (codes[..., 16:] << 4)
        return blk
    off = 96 if t == 6 else 32
    for r in range(16):
        blk[..., r, 0:2] = tu[..., 2 * r:2 * r + 2]
        if t == 6:
            blk[..., r, 2:6] = tu[..., 32 + 4 * r:36 + 4 * r]
        codes = np.zeros(sh + (32,), np.uint8)
        for g in range(4):
            base = off + (16 * g + r) * 4
            for i in range(4):
                b = tu[..., base + i]
                codes[..., 8 * g + i] = b & 15
                codes[..., 8 * g + 4 + i] = b >> 4
        q0 = 6 if t == 6 else 2
        blk[..., r, q0:q0 + 16] = codes[..., :16] | (codes[..., 16:] << 4)
    return blk


def to_tiles(t, raw, n, k):
    """Raw GGUF bytes of an [n, k] tensor -> row-tile layout bytes."""
    block, ub = BLOCK[t]
    if t in SMALL:
        nu = k // block
        npad = tiled_rows(n)
        rows = np.zeros((npad, nu, ub), np.uint8)
        rows[:n] = np.asarray(raw, np.uint8).reshape(n, nu, ub)
        grp = rows.reshape(npad // 16, 16, nu, ub).transpose(0, 2, 1, 3)   # (tiles, nu, 16, ub)
        return _small_to_unit(t, grp).reshape(-1)
    nu = k // block
    npad = tiled_rows(n)
    rows = np.zeros((npad, nu, ub), np.uint8)
    rows[:n] = np.asarray(raw, np.uint8).reshape(n, nu, ub)
    pos = _unit_maps(t)
    out = np.zeros((npad // 16, nu, 16 * ub), np.uint8)
    for r in range(16):
        out[:, :, pos[r]] = rows[r::16]
    return out.reshape(-1)


def from_tiles(t, tiles, n, k):
    """Inverse of ``to_tiles`` (drops the padding rows)."""
    block, ub = BLOCK[t]
    if t in SMALL:
        nu = k // block
        npad = tiled_rows(n)
        tl = np.asarray(tiles, np.uint8).reshape(npad // 16, nu, 16 * ub)
        rows = _small_from_unit(t, tl).transpose(0, 2, 1, 3).reshape(npad, nu, ub)
        return rows[:n].reshape(-1)
    nu = k // block
    npad = tiled_rows(n)
    tl = np.asarray(tiles, np.uint8).reshape(npad // 16, nu, 16 * ub)
    pos = _unit_maps(t)
    rows = np.zeros((npad, nu, ub), np.uint8)
    for r in range(16):
        rows[r::16] = tl[:, :, pos[r]]
    return rows[:n].reshape(-1)


def random_blocks(t, n, k, seed, specials=False):
    """Random block bytes with finite, moderate f16 scales (optionally a sprinkling
    of zero / subnormal / Inf / NaN scales)."""
    rng = np.random.default_rng(seed)
    block, size = BLOCK[t]
    nb = n * (k // block)
    raw = rng.integers(0, 256, (nb, size), dtype=np.uint8)
    offs = {8: [0], 12: [0, 2], 13: [0, 2], 14: [208], 2: [0], 6: [0], 20: [0], 23: [0],
            10: [80, 82], 11: [108], 16: [0], 17: [0], 22: [0], 18: [0], 21: [0], 29: [None]}[t]
    for o in offs:
        vals = (rng.uniform(-0.01, 0.01, nb) if t not in (12, 13) or o == 0
                else rng.uniform(0, 0.005, nb))
        h = vals.astype(np.float16)
        if specials:
            pick = rng.random(nb)
            h = np.where(pick < 0.03, np.float16(0), h)
            h = np.where((pick >= 0.03) & (pick < 0.06), np.float16(6e-8), h)
            h = np.where((pick >= 0.06) & (pick < 0.07), np.float16(np.inf), h)
            h = np.where((pick >= 0.07) & (pick < 0.08), np.float16(np.nan), h)
            h = np.where((pick >= 0.08) & (pick < 0.10), np.float16(-3.0e4), h)
        if o is None:  # IQ1_M: the f16 d in the top nibbles of the four scale words
            dh = h.astype(np.float16).view(np.uint16).astype(np.int64)
            w = raw[:, 48:56].copy().view("<u2").astype(np.int64)
            for i in range(4):
                w[:, i] = (w[:, i] & 0x0FFF) | (((dh >> (4 * i)) & 0xF) << 12)
            raw[:, 48:56] = w.astype("<u2").view(np.uint8).reshape(nb, 8)
        else:
            raw[:, o:o + 2] = h.astype(np.float16).view(np.uint8).reshape(nb, 2)
    return raw.reshape(-1)
