"""numpy model of the HBM row layout (test helper; the layout is defined in
``artifex-assistantv5_amd/ggml.py`` and ``include/gguf_hip.h``)."""

import numpy as np

BLOCK = {8: (32, 34), 12: (256, 144), 14: (256, 210)}


def _align16(x):
    return (x + 15) & ~15


def tile_row_bytes(t, k):
    block, size = BLOCK[t]
    nb = k // block
    return 144 * nb if t == 12 else _align16(size * nb)


def to_tiles(t, raw, n, k):
    """Raw GGUF bytes of an [n, k] tensor -> HBM row layout bytes."""
    block, size = BLOCK[t]
    nb = k // block
    raw = np.asarray(raw, np.uint8).reshape(n, nb, size)
    trb = tile_row_bytes(t, k)
    out = np.zeros((n, trb), np.uint8)
    if t == 12:
        out[:] = raw.reshape(n, -1)
    elif t == 8:
        out[:, :k] = raw[:, :, 2:].reshape(n, k)
        out[:, k:k + 2 * nb] = raw[:, :, :2].reshape(n, 2 * nb)
    else:
        out[:, :k // 2] = raw[:, :, :128].reshape(n, -1)
        out[:, k // 2:k // 2 + k // 4] = raw[:, :, 128:192].reshape(n, -1)
        o = k // 2 + k // 4
        out[:, o:o + k // 16] = raw[:, :, 192:208].reshape(n, -1)
        out[:, o + k // 16:o + k // 16 + 2 * nb] = raw[:, :, 208:210].reshape(n, -1)
    return out.reshape(-1)


def from_tiles(t, tiles, n, k):
    """Inverse of ``to_tiles``."""
    block, size = BLOCK[t]
    nb = k // block
    tiles = np.asarray(tiles, np.uint8).reshape(n, tile_row_bytes(t, k))
    raw = np.zeros((n, nb, size), np.uint8)
    if t == 12:
        raw[:] = tiles[:, :144 * nb].reshape(n, nb, 144)
    elif t == 8:
        raw[:, :, 2:] = tiles[:, :k].reshape(n, nb, 32)
        raw[:, :, :2] = tiles[:, k:k + 2 * nb].reshape(n, nb, 2)
    else:
        o = k // 2 + k // 4
        raw[:, :, :128] = tiles[:, :k // 2].reshape(n, nb, 128)
        raw[:, :, 128:192] = tiles[:, k // 2:o].reshape(n, nb, 64)
        raw[:, :, 192:208] = tiles[:, o:o + k // 16].reshape(n, nb, 16)
        raw[:, :, 208:210] = tiles[:, o + k // 16:o + k // 16 + 2 * nb].reshape(n, nb, 2)
    return raw.reshape(-1)


def random_blocks(t, n, k, seed, specials=False):
    """Random block bytes with finite, moderate f16 scales (optionally a sprinkling
    of zero / subnormal / Inf / NaN scales)."""
    rng = np.random.default_rng(seed)
    block, size = BLOCK[t]
    nb = n * (k // block)
    raw = rng.integers(0, 256, (nb, size), dtype=np.uint8)
    offs = {8: [0], 12: [0, 2], 14: [208]}[t]
    for o in offs:
        vals = (rng.uniform(-0.01, 0.01, nb) if t != 12 or o == 0 else rng.uniform(0, 0.005, nb))
        h = vals.astype(np.float16)
        if specials:
            pick = rng.random(nb)
            h = np.where(pick < 0.03, np.float16(0), h)
            h = np.where((pick >= 0.03) & (pick < 0.06), np.float16(6e-8), h)
            h = np.where((pick >= 0.06) & (pick < 0.07), np.float16(np.inf), h)
            h = np.where((pick >= 0.07) & (pick < 0.08), np.float16(np.nan), h)
            h = np.where((pick >= 0.08) & (pick < 0.10), np.float16(-3.0e4), h)
        raw[:, o:o + 2] = h.astype(np.float16).view(np.uint8).reshape(nb, 2)
    return raw.reshape(-1)
