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

IN_SCOPE = (8, 12, 13, 14)
BLOCK = {8: (32, 34), 12: (256, 144), 13: (256, 176), 14: (256, 210)}
F16_FIELDS = {8: [0], 12: [0, 2], 13: [0, 2], 14: [208]}


def _samples(golden_samples, types=IN_SCOPE):
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
                                     (14, exact_q6_k)])
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
            struct.pack_into("<H", raw, b * size + o, h if (b // len(SPECIAL_F16)) != 1 or o == 0 else
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
    assert rel < {8: 0.01, 12: 0.12, 13: 0.06, 14: 0.05}[t]


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
