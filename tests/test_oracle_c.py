"""Pins for the compiled CPU restatement (oracle/gguf_ref_c.c) that bench.py's
CPU baseline times — CPU only.

* the reference's gguf-py golden vectors for Q4_K (webgpu/test-fixtures), bit-exact;
* random superblocks, with special d / dmin values (0, subnormal, Inf, NaN),
  bit-exact against the numpy oracle, which tests/test_oracle.py pins;
* the fused dequant-matmul against a float64 product of the oracle's values, within
  f32 accumulation error, and bit-identical for any thread count;
* a planted mistake (the 6-bit scale of sub-blocks 4..7 read without its high
  bits, in a copy of the oracle) fails the bit-exact pin.
"""

import ctypes
import struct

import numpy as np
import pytest

from oracle import build_oracle

SPECIAL_F16 = (0x0000, 0x0001, 0x03FF, 0x7C00, 0xFC00, 0x7E00, 0x3C00, 0xBC00)


@pytest.fixture(scope="module")
def clib():
    lib = build_oracle.load()
    if lib is None:
        build_oracle.build()
        lib = build_oracle.load()
    return lib


def _dequant(clib, raw: np.ndarray, n_rows: int, k: int, threads: int = 2) -> np.ndarray:
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    out = np.empty((n_rows, k), np.float32)
    assert clib.oracle_dequant_rows_q4_k(raw.ctypes.data, n_rows, k, out.ctypes.data, threads) > 0
    return out


def _matmul(clib, raw, n_rows, k, x, threads):
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty((x.shape[0], n_rows), np.float32)
    assert clib.oracle_matmul_q4_k(raw.ctypes.data, n_rows, k, x.ctypes.data, x.shape[0],
                                   y.ctypes.data, threads) > 0
    return y


def test_golden_q4_k_bit_exact(clib, ref, golden_samples):
    samples = [s for s in golden_samples if s["ggml_type"] == 12]
    assert len(samples) == 2
    for s in samples:
        raw = np.frombuffer(bytes.fromhex(s["bytes_hex"]), np.uint8)
        n = s["n_elements"]
        got = _dequant(clib, raw, 1, n).reshape(-1)
        want = np.array(s["expected_f32"], np.float64).astype(np.float32)
        assert ref.same_bits(got, want), s["tensor"]


def test_random_blocks_match_numpy_oracle(clib, ref):
    rng = np.random.default_rng(11)
    n_rows, k = 24, 1024
    raw = rng.integers(0, 256, size=n_rows * (k // 256) * 144, dtype=np.uint8)
    blocks = raw.reshape(-1, 144)
    # finite scales for most blocks, every special value in d and in dmin for some
    for b in range(blocks.shape[0]):
        d = SPECIAL_F16[b % len(SPECIAL_F16)] if b < 2 * len(SPECIAL_F16) else int(rng.integers(0, 0x7800))
        dm = SPECIAL_F16[(b + 3) % len(SPECIAL_F16)] if b < 2 * len(SPECIAL_F16) else int(rng.integers(0, 0x7800))
        blocks[b, 0:2] = np.frombuffer(struct.pack("<H", d), np.uint8)
        blocks[b, 2:4] = np.frombuffer(struct.pack("<H", dm), np.uint8)
    got = _dequant(clib, raw, n_rows, k)
    want = ref.dequant_rows(12, raw, n_rows, k)
    assert ref.same_bits(got.reshape(-1), want.reshape(-1))


def test_matmul_against_float64(clib, ref):
    rng = np.random.default_rng(5)
    n_rows, k = 70, 1024
    for d_hi in (0x2000, 0x1400):  # scales around 2^-7 and 2^-10
        raw = rng.integers(0, 256, size=n_rows * (k // 256) * 144, dtype=np.uint8)
        blocks = raw.reshape(-1, 144)
        blocks[:, 0:2] = np.frombuffer(struct.pack("<H", d_hi), np.uint8)
        blocks[:, 2:4] = np.frombuffer(struct.pack("<H", d_hi - 0x0400), np.uint8)
        w = ref.dequant_rows(12, raw, n_rows, k).astype(np.float64)
        for m in (1, 3):
            x = rng.standard_normal((m, k)).astype(np.float32)
            y1 = _matmul(clib, raw, n_rows, k, x, 1)
            y4 = _matmul(clib, raw, n_rows, k, x, 4)
            assert np.array_equal(y1, y4), "thread count changed the result"
            y64 = x.astype(np.float64) @ w.T
            scale = np.abs(x.astype(np.float64)) @ np.abs(w).T
            assert np.max(np.abs(y1 - y64) / scale) < 2e-6


def test_rejects_bad_shapes(clib):
    raw = np.zeros(144, np.uint8)
    out = np.zeros(256, np.float32)
    assert clib.oracle_dequant_rows_q4_k(raw.ctypes.data, 1, 200, out.ctypes.data, 1) == -1
    x = np.zeros((65, 256), np.float32)
    y = np.zeros((65, 1), np.float32)
    assert clib.oracle_matmul_q4_k(raw.ctypes.data, 1, 256, x.ctypes.data, 65, y.ctypes.data, 1) == -1


def test_planted_mistake_fails(tmp_path, ref):
    """A copy of the C oracle with the high bits of the sub-block 4..7 scales
    dropped is caught by the bit-exact pin against the numpy oracle."""
    import subprocess

    src = open(build_oracle.SRC, encoding="utf-8").read()
    bad = src.replace("*sc = (q[j + 4] & 0x0F) | ((q[j - 4] >> 6) << 4);", "*sc = (q[j + 4] & 0x0F);")
    assert bad != src
    (tmp_path / "bad.c").write_text(bad)
    so = tmp_path / "bad.so"
    subprocess.run(["gcc", "-O2", "-fopenmp", "-shared", "-fPIC", str(tmp_path / "bad.c"), "-o", str(so),
                    "-lm"], check=True)
    lib = ctypes.CDLL(str(so))
    lib.oracle_dequant_rows_q4_k.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64,
                                             ctypes.c_void_p, ctypes.c_int]
    rng = np.random.default_rng(3)
    raw = rng.integers(0, 256, size=4 * 144, dtype=np.uint8)
    raw.reshape(-1, 144)[:, 0:4] = np.frombuffer(struct.pack("<HH", 0x2000, 0x1C00), np.uint8)
    out = np.empty((4, 256), np.float32)
    lib.oracle_dequant_rows_q4_k(raw.ctypes.data, 4, 256, out.ctypes.data, 1)
    assert not ref.same_bits(out.reshape(-1), ref.dequant_rows(12, raw, 4, 256).reshape(-1))
