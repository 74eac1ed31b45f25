"""Deterministic CPU quantizers that produce raw GGUF blocks (host-side input
generation; the reference ships none — it only decodes).

The decode side of each format is fixed by the reference
(``webgpu/src/model/gguf-dequant.ts:152-166,169-176,255-281,369-399``); any
block bytes are valid input to the kernels, so the quantizers only need to be
deterministic and sensible.  They follow the packing conventions of
llama.cpp's ``quantize_row_*_ref`` (6-bit scale/min packing of Q4_K, ql/qh
split of Q6_K) with simpler scale searches:

* Q8_0: ``d = max|w| / 127`` per 32 elements, stored as f16; ``q = rint(w / d)``.
* Q4_K: per 32-element sub-block ``scale = (max - min(0, min)) / 15`` and
  ``min = -min(0, min)``; per superblock ``d = max scale / 63``,
  ``dmin = max min / 63`` (f16); 6-bit ``sc, m`` then 4-bit ``q``.
* Q5_K: as Q4_K with ``/ 31`` and 5-bit ``q``: low nibble into ``qs`` as Q4_K
  does, the fifth bit of sub-block j into bit j of ``qh[l]`` (element l of
  the sub-block).
* Q6_K: per 16-element sub-block ``scale = max|w| / 31``; ``d = max|scale| /
  127`` (f16); int8 ``sc`` then ``q - 32`` in [-32, 31].
* Q4_0 / Q5_0: ``d = v / -8`` (``/ -16``) per 32 elements, ``v`` the element
  of largest magnitude (so that it maps to code 0); ``q = rint(w / d) + 8``
  (``+ 16``) clipped to 4 (5) bits; element ``j`` of the block goes to the low
  nibble of ``qs[j]`` for ``j < 16`` and to the high nibble of ``qs[j - 16]``
  above, Q5_0's fifth bit of element ``j`` to bit ``j`` of ``qh``.
* IQ4_NL: ``d = v / -127`` per 32 elements; each element takes the nearest
  entry of the 16-value codebook (ties to the lower index); packed as Q4_0.
* IQ4_XS: per 32-element sub-block the IQ4_NL scale ``s = v / -127``; per
  superblock ``d = max|s| / 31`` (f16) and ``ls - 32 = rint(s / d)``; each
  element takes the nearest codebook entry of ``w / (d (ls - 32))``; ``ls``
  packed as nibble ``j`` of ``scales_l`` and bits ``2j, 2j + 1`` of
  ``scales_h``, each sub-block's codes as a Q4_0 block.
* Q2_K: per 16-element group ``m = -min(0, min)`` and ``s = (max + m) / 3``;
  per superblock ``d = max s / 15``, ``dmin = max m / 15`` (f16); 4-bit
  ``sc, mn`` packed as ``sc | mn << 4``; ``q = rint((w + dmin mn) / (d sc))``
  clipped to 2 bits; element ``128 h + 32 j + 16 s + l`` goes to bits ``2 j``
  of ``qs[32 h + 16 s + l]``.
* Q3_K: per 16-element group ``s = v / -4``; per superblock ``d = max|s| / 31``
  (f16), ``sc - 32 = rint(s / d)``; ``q3 = rint(w / (d (sc - 32))) + 4`` clipped
  to 3 bits: bits 0-1 into ``qs`` as Q2_K, bit 2 into bit ``4 h + j`` of
  ``hmask[16 s + l]``; the 6-bit ``sc`` packed as low nibbles (scales 0-7 in the
  low, 8-15 in the high nibbles of bytes 0-7) and 2-bit fields (scale ``i`` in
  bits ``2 (i // 4)`` of byte ``8 + i % 4``).

All arithmetic is numpy f32; results depend only on the input values.
"""

from __future__ import annotations

import numpy as np

from .ggml import IQ4_NL, IQ4_XS, Q2_K, Q3_K, Q4_0, Q4_K, Q5_0, Q5_K, Q6_K, Q8_0

_CHUNK_ROWS = 4096


def _f16(x: np.ndarray) -> np.ndarray:
    return x.astype(np.float16)


def _safe_div(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    out = np.zeros(np.broadcast(a, b).shape, np.float32)
    np.divide(a, b, out=out, where=(b != 0))
    return out


def pack_q4_k_scales(sc: np.ndarray, m: np.ndarray) -> np.ndarray:
    """Pack 8 six-bit (scale, min) pairs per superblock into 12 bytes.

    ``sc``, ``m``: (..., 8) integers in [0, 63].  Slot j < 4 keeps the low six
    bits of byte j (scale) and byte j + 4 (min); slot j >= 4 stores its low
    nibbles in byte j + 4 and its top two bits in bits 6-7 of bytes j - 4
    (scale) and j (min).
    """
    sc = np.asarray(sc, np.uint8)
    m = np.asarray(m, np.uint8)
    out = np.zeros(sc.shape[:-1] + (12,), np.uint8)
    out[..., 0:4] = (sc[..., 0:4] & 63) | ((sc[..., 4:8] >> 4) << 6)
    out[..., 4:8] = (m[..., 0:4] & 63) | ((m[..., 4:8] >> 4) << 6)
    out[..., 8:12] = (sc[..., 4:8] & 0x0F) | ((m[..., 4:8] & 0x0F) << 4)
    return out


def pack_q6_k(q: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Split unsigned 6-bit values (nb, 256) in element order into ``ql[128]``, ``qh[64]``.

    Element ``128*h + 32*t + l`` (half h, quarter t, lane l < 32) puts its low
    nibble in ``ql[64h + l]`` (t = 0 low, t = 2 high nibble) or
    ``ql[64h + 32 + l]`` (t = 1 low, t = 3 high) and its top two bits in bits
    ``2t..2t+1`` of ``qh[32h + l]``.
    """
    q = np.asarray(q, np.uint8).reshape(-1, 2, 4, 32)
    lo = q & 0x0F
    hi = q >> 4
    ql = np.empty((q.shape[0], 2, 2, 32), np.uint8)
    ql[:, :, 0, :] = lo[:, :, 0, :] | (lo[:, :, 2, :] << 4)
    ql[:, :, 1, :] = lo[:, :, 1, :] | (lo[:, :, 3, :] << 4)
    qh = hi[:, :, 0, :] | (hi[:, :, 1, :] << 2) | (hi[:, :, 2, :] << 4) | (hi[:, :, 3, :] << 6)
    return ql.reshape(-1, 128), qh.reshape(-1, 64)


def _quantize_q8_0(w: np.ndarray) -> np.ndarray:
    blocks = w.reshape(-1, 32)
    amax = np.abs(blocks).max(axis=1)
    d = (amax / np.float32(127)).astype(np.float32)
    inv = _safe_div(np.float32(1), d)
    q = np.clip(np.rint(blocks * inv[:, None]), -127, 127).astype(np.int8)
    out = np.empty((blocks.shape[0], 34), np.uint8)
    out[:, 0:2] = _f16(d).view(np.uint8).reshape(-1, 2)
    out[:, 2:34] = q.view(np.uint8)
    return out.reshape(-1)


def _k_scales(w: np.ndarray, levels: int):
    """Per-sub-block scale / min codes of Q4_K / Q5_K and the integer codes q."""
    sub = w.reshape(-1, 8, 32)
    wmin = np.minimum(sub.min(axis=2), np.float32(0))
    wmax = sub.max(axis=2)
    scale = (wmax - wmin) / np.float32(levels)
    mins = -wmin
    d16 = _f16(scale.max(axis=1) / np.float32(63))
    dmin16 = _f16(mins.max(axis=1) / np.float32(63))
    d = d16.astype(np.float32)[:, None]
    dmin = dmin16.astype(np.float32)[:, None]
    sc = np.clip(np.rint(_safe_div(scale, d)), 0, 63).astype(np.uint8)
    m = np.clip(np.rint(_safe_div(mins, dmin)), 0, 63).astype(np.uint8)
    d1 = (d * sc)[:, :, None]
    m1 = (dmin * m)[:, :, None]
    q = np.clip(np.rint(_safe_div(sub + m1, d1)), 0, levels).astype(np.uint8)   # (nb, 8, 32)
    return d16, dmin16, sc, m, q


def _quantize_q5_k(w: np.ndarray) -> np.ndarray:
    d16, dmin16, sc, m, q = _k_scales(w, 31)
    nb = q.shape[0]
    qs = (q[:, 0::2, :] & 0x0F) | ((q[:, 1::2, :] & 0x0F) << 4)          # (nb, 4, 32)
    qh = ((q >> 4) << np.arange(8, dtype=np.uint8)[None, :, None]).sum(axis=1, dtype=np.uint8)
    out = np.empty((nb, 176), np.uint8)
    out[:, 0:2] = d16.view(np.uint8).reshape(-1, 2)
    out[:, 2:4] = dmin16.view(np.uint8).reshape(-1, 2)
    out[:, 4:16] = pack_q4_k_scales(sc, m)
    out[:, 16:48] = qh
    out[:, 48:176] = qs.reshape(nb, 128)
    return out.reshape(-1)


def _quantize_q4_k(w: np.ndarray) -> np.ndarray:
    sub = w.reshape(-1, 8, 32)
    nb = sub.shape[0]
    wmin = np.minimum(sub.min(axis=2), np.float32(0))
    wmax = sub.max(axis=2)
    scale = (wmax - wmin) / np.float32(15)
    mins = -wmin
    d16 = _f16(scale.max(axis=1) / np.float32(63))
    dmin16 = _f16(mins.max(axis=1) / np.float32(63))
    d = d16.astype(np.float32)[:, None]
    dmin = dmin16.astype(np.float32)[:, None]
    sc = np.clip(np.rint(_safe_div(scale, d)), 0, 63).astype(np.uint8)
    m = np.clip(np.rint(_safe_div(mins, dmin)), 0, 63).astype(np.uint8)
    d1 = (d * sc)[:, :, None]
    m1 = (dmin * m)[:, :, None]
    q = np.clip(np.rint(_safe_div(sub + m1, d1)), 0, 15).astype(np.uint8)   # (nb, 8, 32)
    qs = q[:, 0::2, :] | (q[:, 1::2, :] << 4)                              # (nb, 4, 32)
    out = np.empty((nb, 144), np.uint8)
    out[:, 0:2] = d16.view(np.uint8).reshape(-1, 2)
    out[:, 2:4] = dmin16.view(np.uint8).reshape(-1, 2)
    out[:, 4:16] = pack_q4_k_scales(sc, m)
    out[:, 16:144] = qs.reshape(nb, 128)
    return out.reshape(-1)


def _quantize_q6_k(w: np.ndarray) -> np.ndarray:
    sub = w.reshape(-1, 16, 16)
    nb = sub.shape[0]
    scale = np.abs(sub).max(axis=2) / np.float32(31)                        # (nb, 16)
    d16 = _f16(scale.max(axis=1) / np.float32(127))
    d = d16.astype(np.float32)[:, None]
    sc = np.clip(np.rint(_safe_div(scale, d)), -128, 127).astype(np.int8)
    ds = (d * sc.astype(np.float32))[:, :, None]
    q = np.clip(np.rint(_safe_div(sub, ds)), -32, 31).astype(np.int16) + 32   # 0..63
    ql, qh = pack_q6_k(q.reshape(nb, 256))
    out = np.empty((nb, 210), np.uint8)
    out[:, 0:128] = ql
    out[:, 128:192] = qh
    out[:, 192:208] = sc.view(np.uint8)
    out[:, 208:210] = d16.view(np.uint8).reshape(-1, 2)
    return out.reshape(-1)


# IQ4_NL codebook (kvalues_iq4nl; gguf-dequant.ts:29).
IQ4NL_VALUES = np.array([-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113],
                        np.int8)


def _signed_absmax(b: np.ndarray) -> np.ndarray:
    """The element of largest magnitude of each row (first on ties), keeping its sign."""
    idx = np.abs(b).argmax(axis=1)
    return b[np.arange(b.shape[0]), idx]


def pack_nibbles32(q: np.ndarray) -> np.ndarray:
    """4-bit codes (nb, 32) -> qs (nb, 16): element j < 16 in the low nibble of byte j,
    element j + 16 in its high nibble."""
    q = np.asarray(q, np.uint8)
    return (q[:, :16] & 0x0F) | ((q[:, 16:] & 0x0F) << 4)


def _quantize_q4_0(w: np.ndarray) -> np.ndarray:
    b = w.reshape(-1, 32)
    d16 = _f16(_signed_absmax(b) / np.float32(-8))
    d = d16.astype(np.float32)[:, None]
    q = np.clip(np.rint(_safe_div(b, d)) + 8, 0, 15).astype(np.uint8)
    out = np.empty((b.shape[0], 18), np.uint8)
    out[:, 0:2] = d16.view(np.uint8).reshape(-1, 2)
    out[:, 2:18] = pack_nibbles32(q)
    return out.reshape(-1)


def _quantize_q5_0(w: np.ndarray) -> np.ndarray:
    b = w.reshape(-1, 32)
    d16 = _f16(_signed_absmax(b) / np.float32(-16))
    d = d16.astype(np.float32)[:, None]
    q = np.clip(np.rint(_safe_div(b, d)) + 16, 0, 31).astype(np.uint32)
    qh = ((q >> 4) << np.arange(32, dtype=np.uint32)[None, :]).sum(axis=1, dtype=np.uint64)
    out = np.empty((b.shape[0], 22), np.uint8)
    out[:, 0:2] = d16.view(np.uint8).reshape(-1, 2)
    out[:, 2:6] = qh.astype("<u4").view(np.uint8).reshape(-1, 4)
    out[:, 6:22] = pack_nibbles32(q & 0x0F)
    return out.reshape(-1)


def _quantize_iq4_nl(w: np.ndarray) -> np.ndarray:
    b = w.reshape(-1, 32)
    d16 = _f16(_signed_absmax(b) / np.float32(-127))
    d = d16.astype(np.float32)[:, None]
    t = _safe_div(b, d)
    q = np.abs(t[:, :, None] - IQ4NL_VALUES.astype(np.float32)[None, None, :]).argmin(axis=2)
    out = np.empty((b.shape[0], 18), np.uint8)
    out[:, 0:2] = d16.view(np.uint8).reshape(-1, 2)
    out[:, 2:18] = pack_nibbles32(q)
    return out.reshape(-1)


def _quantize_iq4_xs(w: np.ndarray) -> np.ndarray:
    sb = w.reshape(-1, 8, 32)
    nb = sb.shape[0]
    s = _signed_absmax(sb.reshape(-1, 32)).reshape(nb, 8) / np.float32(-127)   # per sub-block
    d16 = _f16(np.abs(s).max(axis=1) / np.float32(31))
    d = d16.astype(np.float32)[:, None]
    l = np.clip(np.rint(_safe_div(s, d)), -32, 31).astype(np.int32)            # ls - 32
    ls = (l + 32).astype(np.uint32)
    dl = (d * l.astype(np.float32))[:, :, None]
    t = _safe_div(sb, dl)
    q = np.abs(t[..., None] - IQ4NL_VALUES.astype(np.float32)).argmin(axis=-1)
    out = np.empty((nb, 136), np.uint8)
    out[:, 0:2] = d16.view(np.uint8).reshape(-1, 2)
    sh = (((ls >> 4) & 3) << (2 * np.arange(8, dtype=np.uint32))).sum(axis=1, dtype=np.uint32)
    out[:, 2:4] = sh.astype("<u2").view(np.uint8).reshape(-1, 2)
    out[:, 4:8] = ((ls[:, 0::2] & 0xF) | ((ls[:, 1::2] & 0xF) << 4)).astype(np.uint8)
    out[:, 8:136] = pack_nibbles32(q.reshape(-1, 32)).reshape(nb, 128)
    return out.reshape(-1)


def _quantize_q2_k(w: np.ndarray) -> np.ndarray:
    g = w.reshape(-1, 16, 16)                                   # (nb, group, element)
    nb = g.shape[0]
    mn = -np.minimum(g.min(axis=2), 0)
    sc = (g.max(axis=2) + mn) / np.float32(3)
    d16 = _f16(sc.max(axis=1) / np.float32(15))
    m16 = _f16(mn.max(axis=1) / np.float32(15))
    d, dm = d16.astype(np.float32)[:, None], m16.astype(np.float32)[:, None]
    isc = np.clip(np.rint(_safe_div(sc, d)), 0, 15).astype(np.uint8)
    imn = np.clip(np.rint(_safe_div(mn, dm)), 0, 15).astype(np.uint8)
    dl = (d * isc.astype(np.float32))[:, :, None]
    ml = (dm * imn.astype(np.float32))[:, :, None]
    q = np.clip(np.rint(_safe_div(g + ml, dl)), 0, 3).astype(np.uint8)
    # element e = 128 h + 32 j + 16 s + l = group 8 h + 2 j + s, index l
    q = q.reshape(nb, 2, 4, 2, 16)                              # (nb, h, j, s, l)
    qs = np.zeros((nb, 2, 2, 16), np.uint8)                     # (nb, h, s, l)
    for j in range(4):
        qs |= q[:, :, j] << (2 * j)
    out = np.empty((nb, 84), np.uint8)
    out[:, 0:16] = isc | (imn << 4)
    out[:, 16:80] = qs.reshape(nb, 64)
    out[:, 80:82] = d16.view(np.uint8).reshape(-1, 2)
    out[:, 82:84] = m16.view(np.uint8).reshape(-1, 2)
    return out.reshape(-1)


def _quantize_q3_k(w: np.ndarray) -> np.ndarray:
    g = w.reshape(-1, 16, 16)
    nb = g.shape[0]
    s = _signed_absmax(g.reshape(-1, 16)).reshape(nb, 16) / np.float32(-4)
    d16 = _f16(np.abs(s).max(axis=1) / np.float32(31))
    d = d16.astype(np.float32)[:, None]
    l = np.clip(np.rint(_safe_div(s, d)), -32, 31).astype(np.int32)
    dl = (d * l.astype(np.float32))[:, :, None]
    q = (np.clip(np.rint(_safe_div(g, dl)) + 4, 0, 7)).astype(np.uint8)
    q = q.reshape(nb, 2, 4, 2, 16)                              # (nb, h, j, s, l)
    qs = np.zeros((nb, 2, 2, 16), np.uint8)
    hm = np.zeros((nb, 2, 16), np.uint8)                        # (nb, s, l)
    for h in range(2):
        for j in range(4):
            qs[:, h] |= (q[:, h, j] & 3) << (2 * j)
            hm |= ((q[:, h, j] >> 2) & 1) << (4 * h + j)
    sc = (l + 32).astype(np.uint8)                              # (nb, 16), 6 bits
    sb = np.zeros((nb, 12), np.uint8)
    sb[:, 0:8] = (sc[:, 0:8] & 15) | ((sc[:, 8:16] & 15) << 4)
    for i in range(16):
        sb[:, 8 + i % 4] |= ((sc[:, i] >> 4) & 3) << (2 * (i // 4))
    out = np.empty((nb, 110), np.uint8)
    out[:, 0:32] = hm.reshape(nb, 32)
    out[:, 32:96] = qs.reshape(nb, 64)
    out[:, 96:108] = sb
    out[:, 108:110] = d16.view(np.uint8).reshape(-1, 2)
    return out.reshape(-1)


_QUANTIZERS = {Q8_0: (32, 34, _quantize_q8_0), Q4_K: (256, 144, _quantize_q4_k),
               Q5_K: (256, 176, _quantize_q5_k), Q6_K: (256, 210, _quantize_q6_k),
               Q4_0: (32, 18, _quantize_q4_0), Q5_0: (32, 22, _quantize_q5_0),
               IQ4_NL: (32, 18, _quantize_iq4_nl), IQ4_XS: (256, 136, _quantize_iq4_xs),
               Q2_K: (256, 84, _quantize_q2_k), Q3_K: (256, 110, _quantize_q3_k)}


def quantize(w: np.ndarray, ggml_type: int) -> np.ndarray:
    """Quantize a row-major f32 weight ``[N, K]`` to raw GGUF bytes (uint8, N*K/block*size)."""
    if int(ggml_type) not in _QUANTIZERS:
        raise NotImplementedError(f"[gguf-hip] no quantizer for ggml type {ggml_type}")
    block, tsize, fn = _QUANTIZERS[int(ggml_type)]
    w = np.asarray(w, np.float32)
    if w.ndim == 1:
        w = w.reshape(1, -1)
    n, k = w.shape
    if k % block:
        raise ValueError(f"[gguf-hip] K={k} not divisible by block size {block}")
    row_bytes = k // block * tsize
    out = np.empty(n * row_bytes, np.uint8)
    for r0 in range(0, n, _CHUNK_ROWS):
        r1 = min(n, r0 + _CHUNK_ROWS)
        out[r0 * row_bytes:r1 * row_bytes] = fn(np.ascontiguousarray(w[r0:r1]))
    return out


def synthetic_weight(n: int, k: int, seed: int, std: float = 0.02) -> np.ndarray:
    """Seeded f32 weight ``[n, k]`` drawn from N(0, std^2)."""
    rng = np.random.default_rng(seed)
    return rng.standard_normal((n, k), dtype=np.float32) * np.float32(std)


def synthetic_activations(m: int, k: int, seed: int, dtype=np.float32) -> np.ndarray:
    """Seeded activations ``[m, k]`` ~ N(0, 1); fp16 ones are drawn in f32 then rounded."""
    rng = np.random.default_rng(seed)
    return rng.standard_normal((m, k), dtype=np.float32).astype(dtype)
