"""Pins for the CPU oracle (oracle/gguf_ref.py) — CPU only.

* the reference's gguf-py golden vectors (webgpu/test-fixtures/gguf-*.json), bit-exact;
* exact rational arithmetic on random blocks;
* the TS-literal loops vs the vectorised restatement, including special values;
* an independent encoder (package quantizer packing) round-tripped through the decoders;
* mutation checks: plausible oracle mistakes fail at least one pin.
"""

import math
import random
import struct
from fractions import Fraction

import numpy as np
import pytest

IN_SCOPE = (2, 6, 8, 10, 11, 12, 13, 14, 20, 23)
GOLDEN_TYPES = (8, 12, 13, 14)                 # the types the reference's gguf-py fixtures cover
BLOCK = {8: (32, 34), 12: (256, 144), 13: (256, 176), 14: (256, 210), 2: (32, 18), 6: (32, 22),
         20: (32, 18), 23: (256, 136), 10: (256, 84), 11: (256, 110)}
F16_FIELDS = {8: [0], 12: [0, 2], 13: [0, 2], 14: [208], 2: [0], 6: [0], 20: [0], 23: [0],
              10: [80, 82], 11: [108]}


def _samples(golden_samples, types=GOLDEN_TYPES):
    return [s for s in golden_samples if s["ggml_type"] in types]


def test_golden_covers_all_types(golden_samples):
    kinds = sorted(s["ggml_type"] for s in _samples(golden_samples))
    assert kinds == [8, 12, 12, 13, 13, 14, 14, 14]


@pytest.mark.parametrize("loop", [False, True])
def test_golden_vectors_bit_exact(ref, golden_samples, loop):
    for s in _samples(golden_samples):
        raw = bytes.fromhex(s["bytes_hex"])
        want = np.array(s["expected_f32"], np.float64).astype(np.float32)
        fn = ref.dequant_ggml_loop if loop else ref.dequant_ggml
        got = fn(s["ggml_type"], raw, s["n_elements"])
        assert ref.same_bits(got, want), (s["tensor"], s["ggml_type"])


def test_expected_values_are_f32(golden_samples):
    # the fixture stores f32 values through f64 JSON numbers: they must round-trip
    for s in _samples(golden_samples):
        e = np.array(s["expected_f32"], np.float64)
        assert np.array_equal(e.astype(np.float32).astype(np.float64), e)


# ---------------------------------------------------------------------------
# exact rational arithmetic
# ---------------------------------------------------------------------------

def f16_fraction(h: int) -> Fraction:
    sign = -1 if h & 0x8000 else 1
    e, f = (h >> 10) & 0x1F, h & 0x3FF
    assert e != 0x1F
    if e == 0:
        return sign * Fraction(f, 1 << 24)
    return sign * Fraction(1024 + f, 1024) * (Fraction(2) ** (e - 15))


def round_f32(v: Fraction) -> np.float32:
    # v has <= 51 significant bits here, so the f64 conversion is exact and the
    # f32 conversion rounds once (to nearest even)
    return np.float32(float(v))


def random_finite_f16(rng: random.Random) -> int:
    while True:
        h = rng.randrange(0, 1 << 16)
        if ((h >> 10) & 0x1F) != 0x1F:
            return h


def exact_q4_k(raw: bytes) -> list:
    out = []
    for b in range(len(raw) // 144):
        blk = raw[144 * b:144 * (b + 1)]
        d = f16_fraction(blk[0] | blk[1] << 8)
        dmin = f16_fraction(blk[2] | blk[3] << 8)
        sc, q = blk[4:16], blk[16:]
        # bit-level description of the 12-byte packing: slot j < 4 -> bits 0..5 of
        # bytes j (scale) and j+4 (min); slot j >= 4 -> nibbles of byte j+4 with
        # bits 6..7 of bytes j-4 (scale) and j (min) on top
        pairs = []
        for j in range(8):
            if j < 4:
                pairs.append((sc[j] % 64, sc[j + 4] % 64))
            else:
                pairs.append((sc[j + 4] % 16 + 16 * (sc[j - 4] // 64),
                              sc[j + 4] // 16 + 16 * (sc[j] // 64)))
        for j in range(8):
            s, m = pairs[j]
            c, hi = divmod(j, 2)
            for l in range(32):
                qv = q[32 * c + l] // 16 if hi else q[32 * c + l] % 16
                out.append(round_f32(d * s * qv - dmin * m))
    return out


def exact_q5_k(raw: bytes) -> list:
    out = []
    for b in range(len(raw) // 176):
        blk = raw[176 * b:176 * (b + 1)]
        d = f16_fraction(blk[0] | blk[1] << 8)
        dmin = f16_fraction(blk[2] | blk[3] << 8)
        sc, qh, q = blk[4:16], blk[16:48], blk[48:]
        for e in range(256):
            j, l = divmod(e, 32)               # sub-block j, element l
            c, hi = divmod(j, 2)               # 64-element chunk c, nibble
            if j < 4:
                s, m = sc[j] % 64, sc[j + 4] % 64
            else:
                s = sc[j + 4] % 16 + 16 * (sc[j - 4] // 64)
                m = sc[j + 4] // 16 + 16 * (sc[j] // 64)
            nib = q[32 * c + l] // 16 if hi else q[32 * c + l] % 16
            fifth = (qh[l] >> j) % 2           # bit j of qh[l] is the fifth bit of sub-block j
            out.append(round_f32(d * s * (nib + 16 * fifth) - dmin * m))
    return out


def exact_q6_k(raw: bytes) -> list:
    out = []
    for b in range(len(raw) // 210):
        blk = raw[210 * b:210 * (b + 1)]
        d = f16_fraction(blk[208] | blk[209] << 8)
        ql, qh, sc = blk[:128], blk[128:192], blk[192:208]
        vals = [0] * 256
        for e in range(256):
            half, r = divmod(e, 128)
            t, l = divmod(r, 32)
            byte = ql[64 * half + l + (32 if t in (1, 3) else 0)]
            nib = byte // 16 if t >= 2 else byte % 16
            hb = (qh[32 * half + l] >> (2 * t)) % 4
            s = sc[e // 16]
            s = s - 256 if s >= 128 else s
            vals[e] = round_f32(d * s * (nib + 16 * hb - 32))
        out.extend(vals)
    return out


# Q4_0 / Q5_0 / IQ4_NL, from the documented element rule (gguf-dequant.ts:108-109,
# :128-129, :318-320): element j < 16 is the low nibble of qs[j], element j + 16 its
# high nibble; Q5_0's fifth bit of element j is bit j of the 32-bit qh.
def _nib(qs: bytes, j: int) -> int:
    return qs[j] & 15 if j < 16 else qs[j - 16] >> 4


def exact_q4_0(raw: bytes) -> list:
    out = []
    for b in range(len(raw) // 18):
        blk = raw[18 * b:18 * (b + 1)]
        d = f16_fraction(blk[0] | blk[1] << 8)
        out += [round_f32(d * (_nib(blk[2:], j) - 8)) for j in range(32)]
    return out


def exact_q5_0(raw: bytes) -> list:
    out = []
    for b in range(len(raw) // 22):
        blk = raw[22 * b:22 * (b + 1)]
        d = f16_fraction(blk[0] | blk[1] << 8)
        qh = int.from_bytes(blk[2:6], "little")
        out += [round_f32(d * ((_nib(blk[6:], j) | ((qh >> j) & 1) << 4) - 16)) for j in range(32)]
    return out


def exact_iq4_nl(raw: bytes, table=None) -> list:
    table = table or IQ4NL_GOLDEN
    out = []
    for b in range(len(raw) // 18):
        blk = raw[18 * b:18 * (b + 1)]
        d = f16_fraction(blk[0] | blk[1] << 8)
        out += [round_f32(d * table[_nib(blk[2:], j)]) for j in range(32)]
    return out


def _load_codebook():
    import json
    import os
    with open(os.path.join(os.path.dirname(__file__), "golden", "iq4nl_codebook.json")) as f:
        return json.load(f)["kvalues_iq4nl"]


IQ4NL_GOLDEN = _load_codebook()


def exact_iq4_xs(raw: bytes) -> list:
    """IQ4_XS (gguf-dequant.ts:339-343 layout note): the 6-bit scale of sub-block i is
    digit i (base 16) of the 32-bit scales_l plus 16 x digit i (base 4) of the 16-bit
    scales_h; sub-block i's codes are a Q4_0-style nibble block at byte 8 + 16 i."""
    out = []
    for b in range(len(raw) // 136):
        blk = raw[136 * b:136 * (b + 1)]
        d = f16_fraction(blk[0] | blk[1] << 8)
        sh, sl = int.from_bytes(blk[2:4], "little"), int.from_bytes(blk[4:8], "little")
        for i in range(8):
            scale = (sl // 16 ** i) % 16 + 16 * ((sh // 4 ** i) % 4) - 32
            qs = blk[8 + 16 * i:24 + 16 * i]
            out += [round_f32(d * scale * IQ4NL_GOLDEN[_nib(qs, j)]) for j in range(32)]
    return out


def exact_q2_k(raw: bytes) -> list:
    """Q2_K from the element rule (gguf-dequant.ts:186-203 read as a formula): element
    e = 128 h + 32 j + 16 s + l has code floor(qs[32 h + 16 s + l] / 4^j) mod 4 and
    scale byte 8 h + 2 j + s = sc + 16 mn; value d sc q - dmin mn."""
    out = []
    for b in range(len(raw) // 84):
        blk = raw[84 * b:84 * (b + 1)]
        d, dmin = f16_fraction(blk[80] | blk[81] << 8), f16_fraction(blk[82] | blk[83] << 8)
        for e in range(256):
            h, j, s, l = e // 128, (e // 32) % 4, (e // 16) % 2, e % 16
            q = (blk[16 + 32 * h + 16 * s + l] // 4 ** j) % 4
            sb = blk[8 * h + 2 * j + s]
            out.append(round_f32(d * (sb % 16) * q - dmin * (sb // 16)))
    return out


def exact_q3_k(raw: bytes) -> list:
    """Q3_K from the element rule read as a formula: the 12 scale bytes as one 96-bit
    integer S; the low nibble of scale i (0..15) is bits 8 (i % 8) + 4 (i // 8) of S,
    its bits 4-5 are bits 64 + 8 (i % 4) + 2 (i // 4); element e = 128 h + 32 j + 16 s
    + l has code digit j (base 4) of qs[32 h + 16 s + l] plus 4 x bit 4 h + j of
    hmask[16 s + l], value d (scale - 32) (code - 4)."""
    out = []
    for b in range(len(raw) // 110):
        blk = raw[110 * b:110 * (b + 1)]
        d = f16_fraction(blk[108] | blk[109] << 8)
        S = int.from_bytes(blk[96:108], "little")
        sc = []
        for i in range(16):
            lo = (S >> (8 * (i % 8) + 4 * (i // 8))) % 16
            hi = (S >> (64 + 8 * (i % 4) + 2 * (i // 4))) % 4
            sc.append(lo + 16 * hi - 32)
        for e in range(256):
            h, j, s, l = e // 128, (e // 32) % 4, (e // 16) % 2, e % 16
            code = (blk[32 + 32 * h + 16 * s + l] // 4 ** j) % 4 + 4 * ((blk[16 * s + l] >> (4 * h + j)) % 2)
            out.append(round_f32(d * sc[e // 16] * (code - 4)))
    return out


def exact_q8_0(raw: bytes) -> list:
    out = []
    for b in range(len(raw) // 34):
        blk = raw[34 * b:34 * (b + 1)]
        d = f16_fraction(blk[0] | blk[1] << 8)
        for i in range(32):
            q = blk[2 + i]
            out.append(round_f32(d * (q - 256 if q >= 128 else q)))
    return out


def _random_blocks(t: int, nblocks: int, seed: int) -> bytes:
    rng = random.Random(seed)
    block, size = BLOCK[t]
    raw = bytearray(rng.randrange(256) for _ in range(nblocks * size))
    for b in range(nblocks):
        base = b * size
        offs = F16_FIELDS[t]
        for o in offs:
            struct.pack_into("<H", raw, base + o, random_finite_f16(rng))
    return bytes(raw)


@pytest.mark.parametrize("t,exact", [(8, exact_q8_0), (12, exact_q4_k), (13, exact_q5_k),
                                     (14, exact_q6_k), (2, exact_q4_0), (6, exact_q5_0),
                                     (20, exact_iq4_nl), (23, exact_iq4_xs), (10, exact_q2_k),
                                     (11, exact_q3_k)])
def test_exact_rational(ref, t, exact):
    raw = _random_blocks(t, 12, seed=t)
    n = 12 * BLOCK[t][0]
    want = np.array(exact(raw), np.float32)
    # exact rationals carry no sign of zero: compare with -0 folded to +0 (the
    # IEEE zero signs are pinned by the loop-vs-vectorised test)
    assert ref.same_bits(ref.dequant_ggml(t, raw, n) + np.float32(0), want)
    assert ref.same_bits(ref.dequant_ggml_loop(t, raw, n) + np.float32(0), want)


# ---------------------------------------------------------------------------
# loops vs vectorised, with special values
# ---------------------------------------------------------------------------

SPECIAL_F16 = [0x0000, 0x8000, 0x0001, 0x03FF, 0x8001, 0x0400, 0x7BFF, 0xFBFF, 0x7C00, 0xFC00,
               0x7E00, 0x7C01, 0x3C00]


@pytest.mark.parametrize("t", IN_SCOPE)
def test_loop_equals_vectorised_with_special_values(ref, t):
    rng = random.Random(100 + t)
    block, size = BLOCK[t]
    nb = 3 * len(SPECIAL_F16)
    raw = bytearray(rng.randrange(256) for _ in range(nb * size))
    for b in range(nb):
        h = SPECIAL_F16[b % len(SPECIAL_F16)]
        for o in F16_FIELDS[t]:
            struct.pack_into("<H", raw, b * size + o, h if (b // len(SPECIAL_F16)) != 1 or o == F16_FIELDS[t][0] else
                             SPECIAL_F16[(b + 5) % len(SPECIAL_F16)])
    raw = bytes(raw)
    n = nb * block
    a = ref.dequant_ggml_loop(t, raw, n)
    v = ref.dequant_ggml(t, raw, n)
    assert ref.same_bits(a, v)
    assert np.isnan(v).any() and np.isinf(v).any()


def test_special_cases(ref):
    # Q4_K, d = 0: every value is -dmin*m of its sub-block
    blk = bytearray(144)
    struct.pack_into("<HH", blk, 0, 0x0000, 0x3C00)          # d = 0, dmin = 1
    blk[4:16] = bytes([1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12])
    blk[16:] = bytes(range(128))
    v = ref.dequant_ggml(12, bytes(blk), 256)
    sc, m = ref.q4_k_scale_min(np.frombuffer(bytes(blk[4:16]), np.uint8))
    for j in range(8):
        assert np.all(v[32 * j:32 * j + 32] == -float(m[j]))
    # Q6_K: scale -128 with raw 6-bit 0 gives d * (-128) * (-32)
    blk6 = bytearray(210)
    blk6[192:208] = bytes([0x80] * 16)
    struct.pack_into("<H", blk6, 208, 0x3C00)                  # d = 1
    assert np.all(ref.dequant_ggml(14, bytes(blk6), 256) == 4096.0)
    # Q8_0: byte 0x80 is -128
    blk8 = bytearray(34)
    struct.pack_into("<H", blk8, 0, 0x3800)                    # d = 0.5
    blk8[2:] = bytes([0x80] * 32)
    assert np.all(ref.dequant_ggml(8, bytes(blk8), 32) == -64.0)
    # subnormal f16 scale: smallest subnormal times 127 is exact
    struct.pack_into("<H", blk8, 0, 0x0001)
    blk8[2:] = bytes([127] * 32)
    assert np.all(ref.dequant_ggml(8, bytes(blk8), 32) == np.float32(127 * 2.0 ** -24))


def test_f16_decoder_matches_numpy(ref):
    hs = np.arange(1 << 16, dtype=np.uint16)
    want = hs.view(np.float16).astype(np.float64)
    got = np.array([ref.f16_to_f32(int(h)) for h in hs], np.float64)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan], want[~nan])
    assert np.array_equal(np.signbit(got[~nan]), np.signbit(want[~nan]))


# ---------------------------------------------------------------------------
# independent encoder round trips
# ---------------------------------------------------------------------------

def test_q4_k_scale_pack_roundtrip_exhaustive(ref, pkg):
    rng = np.random.default_rng(7)
    for j in range(8):
        for s in range(64):
            sc = rng.integers(0, 64, (64, 8)).astype(np.uint8)
            m = rng.integers(0, 64, (64, 8)).astype(np.uint8)
            sc[:, j] = s
            m[:, j] = np.arange(64)
            packed = pkg.quantize.pack_q4_k_scales(sc, m)
            dsc, dm = ref.q4_k_scale_min(packed)
            assert np.array_equal(dsc, sc) and np.array_equal(dm, m)
            if s % 21 == 0:  # the literal loop too, on a subset
                for r in range(0, 64, 9):
                    assert ref.get_scale_min_k4(j, bytes(packed[r]), 0) == (s, r)


def test_q6_k_pack_roundtrip(ref, pkg):
    rng = np.random.default_rng(8)
    q = rng.integers(0, 64, (5, 256)).astype(np.uint8)
    ql, qh = pkg.quantize.pack_q6_k(q)
    blk = np.zeros(5, ref.Q6_K_BLOCK)
    blk["ql"], blk["qh"] = ql, qh
    assert np.array_equal(ref.q6_k_values(blk) + 32, q)


def test_q5_k_pack_roundtrip(ref, pkg):
    w = pkg.quantize.synthetic_weight(6, 512, seed=9)
    d16, dmin16, sc, m, q = pkg.quantize._k_scales(w, 31)
    assert q.max() > 15                                  # the fifth bit is exercised
    blk = pkg.quantize.quantize(w, 13).view(ref.Q5_K_BLOCK)
    assert np.array_equal(ref.q5_k_values(blk), q)
    dsc, dm = ref.q4_k_scale_min(blk["scales"])
    assert np.array_equal(dsc, sc) and np.array_equal(dm, m)


@pytest.mark.parametrize("t", IN_SCOPE)
def test_quantizer_error_is_bounded(ref, pkg, t):
    w = pkg.quantize.synthetic_weight(4, 512, seed=3)
    raw = pkg.quantize.quantize(w, t)
    assert raw.size == 4 * 512 // BLOCK[t][0] * BLOCK[t][1]
    deq = ref.dequant_rows(t, raw, 4, 512)
    rel = np.linalg.norm(deq - w) / np.linalg.norm(w)
    assert rel < {8: 0.01, 12: 0.12, 13: 0.06, 14: 0.05, 2: 0.12, 6: 0.06, 20: 0.1, 23: 0.1, 10: 0.35, 11: 0.2}[t]


# ---------------------------------------------------------------------------
# matmul reference and the parity gate
# ---------------------------------------------------------------------------

def test_matmul_bt_exactly_rounded_small(ref):
    rng = np.random.default_rng(1)
    a = rng.standard_normal((3, 40)).astype(np.float32)
    w = rng.standard_normal((5, 40)).astype(np.float32)
    y = ref.matmul_bt(a, w)
    for i in range(3):
        for j in range(5):
            exact = math.fsum(float(a[i, k]) * float(w[j, k]) for k in range(40))
            assert abs(y[i, j] - exact) <= 1e-14 * (1 + abs(exact))


def test_matmul_bt_linearity_and_transpose(ref):
    rng = np.random.default_rng(2)
    a1, a2 = rng.standard_normal((2, 4, 64))
    w = rng.standard_normal((7, 64))
    assert np.allclose(ref.matmul_bt(a1 + a2, w), ref.matmul_bt(a1, w) + ref.matmul_bt(a2, w),
                       rtol=1e-12, atol=1e-12)
    assert np.allclose(ref.matmul_bt(a1, w), ref.matmul_bt(w, a1).T, rtol=1e-12, atol=1e-12)


def test_parity_metrics_gate(ref):
    rng = np.random.default_rng(3)
    x = rng.standard_normal((2, 256))
    w = rng.standard_normal((9, 256)) * 0.02
    y = ref.matmul_bt(x, w)
    sa = ref.matmul_bt_abs(x, w)
    assert ref.parity_metrics(y * (1 + 1e-6), y, sa)["ok"]
    assert not ref.parity_metrics(y * (1 + 3e-3), y, sa)["ok"]
    bad = y.copy()
    bad[0, 0] = np.nan
    assert not ref.parity_metrics(bad, y, sa)["ok"]


def test_synthetic_fixture_regression(ref, pkg, synthetic_small):
    for t in IN_SCOPE:
        n, k = synthetic_small[f"t{t}_shape"]
        raw = synthetic_small[f"t{t}_raw"]
        assert ref.same_bits(ref.dequant_rows(t, raw, n, k), synthetic_small[f"t{t}_deq"])
        w = pkg.quantize.synthetic_weight(n, k, seed=1000 + t)
        assert np.array_equal(pkg.quantize.quantize(w, t), raw)
        y = ref.matmul_bt(synthetic_small[f"t{t}_x"], synthetic_small[f"t{t}_deq"])
        assert np.allclose(y, synthetic_small[f"t{t}_y"], rtol=1e-12, atol=1e-12)


# ---------------------------------------------------------------------------
# mutation checks: plausible mistakes in the oracle fail the pins
# ---------------------------------------------------------------------------

def _golden_fails(ref, golden_samples, t, fn) -> bool:
    for s in _samples(golden_samples, (t,)):
        raw = bytes.fromhex(s["bytes_hex"])
        want = np.array(s["expected_f32"], np.float64).astype(np.float32)
        if not ref.same_bits(fn(raw, s["n_elements"]), want):
            return True
    return False


def test_mutations_are_caught(ref, golden_samples):
    def q4_no_min(raw, n):
        blk = ref._blocks(raw, ref.Q4_K_BLOCK, n, 256, "Q4_K")
        d = blk["d"].astype(np.float32)[:, None]
        sc, m = ref.q4_k_scale_min(blk["scales"])
        qs = blk["qs"].reshape(-1, 4, 1, 32)
        q = np.concatenate([qs & 15, qs >> 4], axis=2).reshape(-1, 8, 32)
        return ((d * sc)[:, :, None] * q).reshape(-1).astype(np.float32)

    def q4_swapped_nibbles(raw, n):
        blk = ref._blocks(raw, ref.Q4_K_BLOCK, n, 256, "Q4_K").copy()
        blk["qs"] = (blk["qs"] >> 4) | ((blk["qs"] & 15) << 4)
        return ref.dequant_q4_k(blk.view(np.uint8), n)

    def q6_wrong_qh_shift(raw, n):
        blk = ref._blocks(raw, ref.Q6_K_BLOCK, n, 256, "Q6_K").copy()
        blk["qh"] = ((blk["qh"] & 0x33) << 2) | ((blk["qh"] & 0xCC) >> 2)
        return ref.dequant_q6_k(blk.view(np.uint8), n)

    def q6_unsigned_scale(raw, n):
        blk = ref._blocks(raw, ref.Q6_K_BLOCK, n, 256, "Q6_K")
        d = blk["d"].astype(np.float32)[:, None]
        sc = np.repeat(blk["sc"].view(np.uint8).astype(np.float32), 16, axis=1)
        return ((d * sc) * ref.q6_k_values(blk).astype(np.float32)).reshape(-1)

    def q8_unsigned(raw, n):
        blk = ref._blocks(raw, ref.Q8_0_BLOCK, n, 32, "Q8_0")
        d = blk["d"].astype(np.float32)[:, None]
        return (d * blk["qs"].view(np.uint8).astype(np.float32)).reshape(-1)

    def q5_qh_bit_by_chunk(raw, n):   # fifth bit taken from bit c of qh, not bit 2c + hi
        blk = ref._blocks(raw, ref.Q5_K_BLOCK, n, 256, "Q5_K")
        d = blk["d"].astype(np.float32)[:, None, None]
        dmin = blk["dmin"].astype(np.float32)[:, None, None]
        sc, m = ref.q4_k_scale_min(blk["scales"])
        qs = blk["qs"].reshape(-1, 4, 1, 32)
        nib = np.concatenate([qs & 15, qs >> 4], axis=2).reshape(-1, 8, 32)
        bit = (blk["qh"][:, None, :] >> (np.arange(8) // 2)[None, :, None].astype(np.uint8)) & 1
        q = (nib + (bit << 4)).astype(np.float32)
        return (d * sc[:, :, None] * q - dmin * m[:, :, None]).reshape(-1).astype(np.float32)

    def q5_no_fifth_bit(raw, n):
        blk = ref._blocks(raw, ref.Q5_K_BLOCK, n, 256, "Q5_K").copy()
        blk["qh"] = 0
        return ref.dequant_q5_k(blk.view(np.uint8), n)

    assert _golden_fails(ref, golden_samples, 13, q5_qh_bit_by_chunk)
    assert _golden_fails(ref, golden_samples, 13, q5_no_fifth_bit)
    assert _golden_fails(ref, golden_samples, 12, q4_no_min)
    assert _golden_fails(ref, golden_samples, 12, q4_swapped_nibbles)
    assert _golden_fails(ref, golden_samples, 14, q6_wrong_qh_shift)
    assert _golden_fails(ref, golden_samples, 14, q6_unsigned_scale)
    assert _golden_fails(ref, golden_samples, 8, q8_unsigned)


# ---------------------------------------------------------------------------
# Q4_0 / Q5_0 / IQ4_NL: no reference fixture; pinned by the element rule,
# closed forms, the reference's codebook and the quantizer round trip
# ---------------------------------------------------------------------------

def test_iq4nl_codebook_matches_reference(ref):
    # the fixture is read out of the reference's gguf-dequant.ts by make_golden.py
    assert list(ref.KVALUES_IQ4NL) == IQ4NL_GOLDEN
    assert len(set(IQ4NL_GOLDEN)) == 16 and IQ4NL_GOLDEN == sorted(IQ4NL_GOLDEN)


def _block_with_codes(t, d_bits, codes, fifth=None):
    """One raw block whose element j has 4-bit code codes[j] (and fifth bit fifth[j])."""
    qs = bytes((codes[j] & 15) | ((codes[j + 16] & 15) << 4) for j in range(16))
    head = struct.pack("<H", d_bits)
    if t == 6:
        qh = sum(int(b) << j for j, b in enumerate(fifth))
        return head + struct.pack("<I", qh) + qs
    return head + qs


@pytest.mark.parametrize("t", [2, 6, 20])
def test_small_block_element_order_closed_form(ref, t):
    """Every element position with every code: value = d * (code - offset) (Q4_0, Q5_0) or
    d * kvalues[code] (IQ4_NL), d = 0.5 -- so a swapped nibble, a shifted fifth bit or an
    off-by-one offset moves at least one element."""
    rng = random.Random(t)
    for rep in range(20):
        codes = [rng.randrange(16) for _ in range(32)]
        fifth = [rng.randrange(2) for _ in range(32)]
        raw = _block_with_codes(t, 0x3800, codes, fifth)
        want = []
        for j in range(32):
            if t == 2:
                want.append(0.5 * (codes[j] - 8))
            elif t == 6:
                want.append(0.5 * ((codes[j] | fifth[j] << 4) - 16))
            else:
                want.append(0.5 * IQ4NL_GOLDEN[codes[j]])
        got = ref.dequant_ggml(t, raw, 32)
        assert np.array_equal(got, np.array(want, np.float32)), (t, rep)
        assert np.array_equal(ref.dequant_ggml_loop(t, raw, 32), got)


def test_small_block_extremes(ref):
    # Q4_0 code 0 -> -8 d, code 15 -> 7 d; Q5_0 31 -> 15 d, 0 -> -16 d; IQ4_NL 0 -> -127 d
    one = 0x3C00
    assert np.all(ref.dequant_ggml(2, _block_with_codes(2, one, [0] * 32), 32) == -8)
    assert np.all(ref.dequant_ggml(2, _block_with_codes(2, one, [15] * 32), 32) == 7)
    assert np.all(ref.dequant_ggml(6, _block_with_codes(6, one, [15] * 32, [1] * 32), 32) == 15)
    assert np.all(ref.dequant_ggml(6, _block_with_codes(6, one, [0] * 32, [0] * 32), 32) == -16)
    assert np.all(ref.dequant_ggml(20, _block_with_codes(20, one, [0] * 32), 32) == -127)
    assert np.all(ref.dequant_ggml(20, _block_with_codes(20, one, [15] * 32), 32) == 113)
    # subnormal d times the largest magnitude code is exact
    v = ref.dequant_ggml(20, _block_with_codes(20, 0x0001, [0] * 32), 32)
    assert np.all(v == np.float32(-127 * 2.0 ** -24))


@pytest.mark.parametrize("t", [2, 6, 20])
def test_small_block_quantizer_roundtrip(ref, pkg, t):
    """The package quantizer (an independent encoder: own nibble packing, own qh
    assembly, own codebook search) decodes to d times its chosen integers."""
    w = pkg.quantize.synthetic_weight(3, 256, seed=21 + t)
    raw = pkg.quantize.quantize(w, t)
    b = w.reshape(-1, 32)
    idx = np.abs(b).argmax(axis=1)
    vmax = b[np.arange(b.shape[0]), idx]
    div = {2: -8.0, 6: -16.0, 20: -127.0}[t]
    d = (vmax / np.float32(div)).astype(np.float16).astype(np.float32)[:, None]
    if t == 20:
        tab = np.array(IQ4NL_GOLDEN, np.float32)
        q = np.abs((b / d)[:, :, None] - tab[None, None, :]).argmin(axis=2)
        want = d * tab[q]
    else:
        off = 8 if t == 2 else 16
        q = np.clip(np.rint(b / d) + off, 0, 2 * off - 1)
        want = d * (q - off)
    assert np.array_equal(ref.dequant_rows(t, raw, 3, 256), want.reshape(3, 256).astype(np.float32))


def test_small_block_mutations_are_caught(ref):
    """Plausible oracle mistakes each fail the closed-form element pin."""
    rng = random.Random(7)
    codes = [rng.randrange(16) for _ in range(32)]
    fifth = [rng.randrange(2) for _ in range(32)]

    def fails(t, fn):
        raw = _block_with_codes(t, 0x3800, codes, fifth)
        return not np.array_equal(fn(raw), ref.dequant_ggml(t, raw, 32))

    def q4_interleaved(raw):       # element 2j / 2j + 1 from byte j (llama.cpp-style misread)
        qs = np.frombuffer(raw[2:], np.uint8)
        q = np.stack([qs & 15, qs >> 4], axis=1).reshape(-1).astype(np.float32)
        return np.float32(0.5) * (q - 8)

    def q4_offset_7(raw):
        qs = np.frombuffer(raw[2:], np.uint8)
        return np.float32(0.5) * (ref.nibbles32(qs[None]).reshape(-1).astype(np.float32) - 7)

    def q5_fifth_from_byte(raw):   # fifth bit of element j taken from bit j % 8 of qh byte j // 16
        qh = raw[2:6]
        qs = np.frombuffer(raw[6:], np.uint8)
        nib = ref.nibbles32(qs[None]).reshape(-1)
        bits = np.array([(qh[j // 16] >> (j % 8)) & 1 for j in range(32)])
        return np.float32(0.5) * ((nib | (bits << 4)).astype(np.float32) - 16)

    def iq4_reversed_table(raw):
        qs = np.frombuffer(raw[2:], np.uint8)
        tab = np.array(IQ4NL_GOLDEN[::-1], np.float32)
        return np.float32(0.5) * tab[ref.nibbles32(qs[None]).reshape(-1)]

    assert fails(2, q4_interleaved) and fails(2, q4_offset_7)
    assert fails(6, q5_fifth_from_byte)
    assert fails(20, iq4_reversed_table)


def _iq4_xs_block(d_bits, ls, codes):
    """One raw IQ4_XS superblock with sub-block scales ls[0..7] and element codes codes[0..255]."""
    sh = sum((l >> 4) << (2 * i) for i, l in enumerate(ls))
    sl = bytes((ls[2 * i] & 15) | ((ls[2 * i + 1] & 15) << 4) for i in range(4))
    qs = b"".join(bytes((codes[32 * i + j] & 15) | ((codes[32 * i + j + 16] & 15) << 4)
                        for j in range(16)) for i in range(8))
    return struct.pack("<HH", d_bits, sh) + sl + qs


def test_iq4_xs_scales_closed_form(ref):
    """Each sub-block scale changed through its scales_l nibble alone, then its scales_h
    bit pair alone: every element is d * (ls - 32) * kvalues[code] with d = 1."""
    rng = random.Random(23)
    codes = [rng.randrange(16) for _ in range(256)]
    for i in range(8):
        # the other sub-blocks keep ls = 32 (bit pair 10, nibble 0: scale 0)
        for ls in ([32] * i + [37] + [32] * (7 - i),                # nibble 5, bit pair kept
                   [32] * i + [48] + [32] * (7 - i),                 # bit pair 11, nibble kept
                   [32] * i + [0] + [32] * (7 - i),                  # bit pair 00, nibble 0
                   [32] * i + [63] + [32] * (7 - i)):                # both at their maximum
            raw = _iq4_xs_block(0x3C00, ls, codes)
            want = [(ls[e // 32] - 32) * IQ4NL_GOLDEN[codes[e]] for e in range(256)]
            got = ref.dequant_ggml(23, raw, 256)
            assert np.array_equal(got, np.array(want, np.float32)), (i, ls)
            assert np.array_equal(ref.dequant_ggml_loop(23, raw, 256), got)


def test_iq4_xs_is_eight_iq4_nl_blocks(ref):
    """Where d * (ls - 32) is an f16, an IQ4_XS superblock decodes like eight IQ4_NL
    blocks carrying that scale and the same code bytes."""
    rng = random.Random(5)
    for rep_ in range(10):
        ls = [rng.randrange(64) for _ in range(8)]
        codes = [rng.randrange(16) for _ in range(256)]
        raw = _iq4_xs_block(0x3400, ls, codes)                       # d = 0.25
        nl = b"".join(struct.pack("<e", 0.25 * (ls[i] - 32)) + raw[8 + 16 * i:24 + 16 * i]
                      for i in range(8))
        assert np.array_equal(ref.dequant_ggml(23, raw, 256), ref.dequant_ggml(20, nl, 256))


def test_iq4_xs_quantizer_roundtrip(ref, pkg):
    """The package quantizer's IQ4_XS bytes decode to d * (ls - 32) * table[q] for the
    integers it chose (recomputed here from the weights)."""
    w = pkg.quantize.synthetic_weight(2, 512, seed=77)
    raw = pkg.quantize.quantize(w, 23)
    sb = w.reshape(-1, 8, 32)
    b = sb.reshape(-1, 32)
    s = (b[np.arange(b.shape[0]), np.abs(b).argmax(axis=1)] / np.float32(-127)).reshape(-1, 8)
    d = (np.abs(s).max(axis=1) / np.float32(31)).astype(np.float16).astype(np.float32)[:, None]
    l = np.clip(np.rint(s / d), -32, 31)
    dl = (d * l.astype(np.float32))[:, :, None]
    tab = np.array(IQ4NL_GOLDEN, np.float32)
    q = np.abs((sb / dl)[..., None] - tab).argmin(axis=-1)
    want = (dl * tab[q]).reshape(2, 512).astype(np.float32)
    assert np.array_equal(ref.dequant_rows(23, raw, 2, 512), want)


def test_iq4_xs_mutations_are_caught(ref):
    """Plausible misreadings of the scale bits fail the closed-form pin."""
    rng = random.Random(9)
    ls = [rng.randrange(64) for _ in range(8)]
    codes = [rng.randrange(16) for _ in range(256)]
    raw = _iq4_xs_block(0x3C00, ls, codes)
    good = ref.dequant_ggml(23, raw, 256)
    sh = raw[2] | raw[3] << 8
    tab = np.array(IQ4NL_GOLDEN, np.float32)
    cod = np.array(codes).reshape(8, 32)

    def decode(scale_of):
        return np.concatenate([np.float32(scale_of(i) - 32) * tab[cod[i]] for i in range(8)])

    nib_swapped = decode(lambda i: ((raw[4 + i // 2] >> (4 * (1 - i % 2))) & 15) | (((sh >> 2 * i) & 3) << 4))
    h_one_bit = decode(lambda i: ((raw[4 + i // 2] >> (4 * (i % 2))) & 15) | (((sh >> i) & 3) << 4))
    no_bias = decode(lambda i: ls[i] + 32)
    for bad in (nib_swapped, h_one_bit, no_bias):
        assert not np.array_equal(bad, good)


def test_q2_k_closed_form(ref):
    """Scale byte i = (i % 16) + 16 (i // 8) with d = 1, dmin = 1/2, and code bits chosen so
    that element e holds code (e // 16 + e) % 4: each element's value names its group
    and code, so a shifted group, code plane or byte moves at least one element."""
    sc = bytes((i % 16) | ((i // 8) << 4) for i in range(16))
    qs = bytearray(64)
    for e in range(256):
        h, j, s, l = e // 128, (e // 32) % 4, (e // 16) % 2, e % 16
        qs[32 * h + 16 * s + l] |= ((e // 16 + e) % 4) << (2 * j)
    raw = sc + bytes(qs) + struct.pack("<ee", 1.0, 0.5)
    want = [(e // 16 % 16) * ((e // 16 + e) % 4) - 0.5 * (e // 16 // 8) for e in range(256)]
    got = ref.dequant_ggml(10, raw, 256)
    assert np.array_equal(got, np.array(want, np.float32))
    assert np.array_equal(ref.dequant_ggml_loop(10, raw, 256), got)


def test_q2_k_quantizer_roundtrip(ref, pkg):
    """The package quantizer's Q2_K bytes decode to d sc q - dmin mn for the integers it
    chose (recomputed here from the weights)."""
    w = pkg.quantize.synthetic_weight(2, 512, seed=78)
    raw = pkg.quantize.quantize(w, 10)
    g = w.reshape(-1, 16, 16)
    mn = -np.minimum(g.min(axis=2), 0)
    sc = (g.max(axis=2) + mn) / np.float32(3)
    d = (sc.max(axis=1) / np.float32(15)).astype(np.float16).astype(np.float32)[:, None]
    dm = (mn.max(axis=1) / np.float32(15)).astype(np.float16).astype(np.float32)[:, None]
    isc = np.clip(np.rint(sc / d), 0, 15)
    imn = np.clip(np.rint(mn / dm), 0, 15)
    dl, ml = (d * isc)[:, :, None], (dm * imn)[:, :, None]
    q = np.clip(np.rint((g + ml) / dl), 0, 3)
    want = (dl * q - ml).reshape(2, 512).astype(np.float32)
    assert np.array_equal(ref.dequant_rows(10, raw, 2, 512), want)


def test_q2_k_mutations_are_caught(ref):
    """Misreadings of the Q2_K element order fail the exact-rational pin."""
    raw = _random_blocks(10, 2, seed=101)
    good = np.array(exact_q2_k(raw), np.float32) + np.float32(0)

    def decode(code_of, scale_of):
        out = []
        for b in range(2):
            blk = raw[84 * b:84 * (b + 1)]
            d = np.float32(np.frombuffer(blk[80:82], "<f2")[0])
            dm = np.float32(np.frombuffer(blk[82:84], "<f2")[0])
            for e in range(256):
                sb = blk[scale_of(e)]
                out.append(d * np.float32(sb & 15) * np.float32(code_of(blk, e)) - dm * np.float32(sb >> 4))
        return np.array(out, np.float32) + np.float32(0)

    right_code = lambda blk, e: (blk[16 + 32 * (e // 128) + e % 32] >> (2 * ((e // 32) % 4))) & 3
    right_scale = lambda e: e // 16
    assert np.array_equal(decode(right_code, right_scale), good, equal_nan=True)
    planes_swapped = lambda blk, e: (blk[16 + 32 * (e // 128) + e % 32] >> (2 * (3 - (e // 32) % 4))) & 3
    by_64 = lambda blk, e: (blk[16 + (e % 64)] >> (2 * (e // 64))) & 3      # llama-style misread
    scale_per_32 = lambda e: e // 32
    for bad in (decode(planes_swapped, right_scale), decode(by_64, right_scale),
                decode(right_code, scale_per_32)):
        assert not np.array_equal(bad, good, equal_nan=True)


def test_q3_k_closed_form(ref):
    """Scale i = 32 + (i - 8) (signed -8..7) and code (e // 16 + 3 e) % 8 per element,
    with d = 1: every value names its group and code, and the high bit comes from hmask."""
    sc = [32 + i - 8 for i in range(16)]
    sb = bytearray(12)
    for i in range(8):
        sb[i] = (sc[i] & 15) | ((sc[8 + i] & 15) << 4)
    for i in range(16):
        sb[8 + i % 4] |= ((sc[i] >> 4) & 3) << (2 * (i // 4))
    hm, qs = bytearray(32), bytearray(64)
    code = [(e // 16 + 3 * e) % 8 for e in range(256)]
    for e in range(256):
        h, j, s, l = e // 128, (e // 32) % 4, (e // 16) % 2, e % 16
        qs[32 * h + 16 * s + l] |= (code[e] & 3) << (2 * j)
        hm[16 * s + l] |= (code[e] >> 2) << (4 * h + j)
    raw = bytes(hm) + bytes(qs) + bytes(sb) + struct.pack("<e", 1.0)
    want = [(e // 16 - 8) * (code[e] - 4) for e in range(256)]
    got = ref.dequant_ggml(11, raw, 256)
    assert np.array_equal(got, np.array(want, np.float32))
    assert np.array_equal(ref.dequant_ggml_loop(11, raw, 256), got)


def test_q3_k_quantizer_roundtrip(ref, pkg):
    w = pkg.quantize.synthetic_weight(2, 512, seed=79)
    raw = pkg.quantize.quantize(w, 11)
    g = w.reshape(-1, 16, 16)
    b = g.reshape(-1, 16)
    s = (b[np.arange(b.shape[0]), np.abs(b).argmax(axis=1)] / np.float32(-4)).reshape(-1, 16)
    d = (np.abs(s).max(axis=1) / np.float32(31)).astype(np.float16).astype(np.float32)[:, None]
    l = np.clip(np.rint(s / d), -32, 31)
    dl = (d * l.astype(np.float32))[:, :, None]
    q = np.clip(np.rint(g / dl) + 4, 0, 7)
    want = (dl * (q - 4)).reshape(2, 512).astype(np.float32)
    assert np.array_equal(ref.dequant_rows(11, raw, 2, 512), want)
