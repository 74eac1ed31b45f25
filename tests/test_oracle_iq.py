"""Oracle for the grid-codebook IQ types (oracle/gguf_iq.py), pinned against the
reference's IQ parity fixture and the mathematics of the formats."""

import json
import os
import re

import numpy as np
import pytest

from oracle import gguf_iq as iq
from oracle import gguf_ref as ref

HERE = os.path.dirname(os.path.abspath(__file__))
with open(os.path.join(HERE, "golden", "iq_parity_samples.json"), encoding="utf-8") as f:
    SAMPLES = json.load(f)["samples"]


def test_fixture_covers_all_six_types():
    assert sorted(s["ggml_type"] for s in SAMPLES) == sorted(iq.IQ_TYPES)


@pytest.mark.parametrize("s", SAMPLES, ids=lambda s: s["tensor"])
def test_parity_fixture_bit_exact(s):
    """gguf-py's output on the reference's random blocks (iq_parity_fixture.json)."""
    raw = bytes.fromhex(s["bytes_hex"])
    want = np.asarray(s["expected_f32"], np.float32)
    for got in (iq.LOOPS[s["ggml_type"]](raw, s["n_elements"]),
                iq.VECTORISED[s["ggml_type"]](raw, s["n_elements"]),
                ref.dequant_ggml(s["ggml_type"], np.frombuffer(raw, np.uint8), s["n_elements"])):
        assert got.dtype == np.float32 and got.shape == want.shape
        assert ref.same_bits(got, want), s["tensor"]


@pytest.mark.parametrize("t", iq.IQ_TYPES)
def test_loops_match_vectorised_on_random_blocks(t):
    raw = iq.random_blocks(t, 3, seed=t, d=0.0078125)
    n = 3 * 256
    assert ref.same_bits(iq.LOOPS[t](bytes(raw), n), iq.VECTORISED[t](raw, n))


def test_grid_tables():
    """Shapes and value sets of the codebooks; the ksigns parity rule (bit 7
    makes the popcount of each sign byte even)."""
    G = iq.grids()
    assert G["iq2xxs"].shape == (256, 8) and G["iq2xs"].shape == (512, 8)
    assert G["iq2s"].shape == (1024, 8) and G["iq3xxs"].shape == (256, 4)
    assert G["iq3s"].shape == (512, 4) and G["iq1s"].shape == (2048, 8)
    for k in ("iq2xxs", "iq2xs", "iq2s"):
        assert set(np.unique(G[k])) <= {8, 25, 43}
        assert len({tuple(r) for r in G[k]}) == len(G[k])          # distinct entries
    assert set(np.unique(G["iq3xxs"])) <= {4, 12, 20, 28, 36, 44, 52, 62}
    assert len({tuple(r) for r in G["iq3xxs"]}) == 256 and len({tuple(r) for r in G["iq3s"]}) == 512
    assert set(np.unique(G["iq3s"])) <= set(range(1, 16, 2))
    assert set(np.unique(G["iq1s"])) <= {-1, 0, 1}
    for i in range(128):
        b = int(G["ksigns"][i])
        assert b & 127 == i and bin(b).count("1") % 2 == 0
    assert G["delta"] == 0.125


@pytest.mark.parametrize("t", [iq.T_IQ2_XXS, iq.T_IQ3_XXS])
def test_single_grid_entry_blocks(t):
    """All grid indices equal, no signs, scale nibble ls: every element is
    d * factor(ls) * grid[e][j % width]."""
    G = iq.grids()
    d = 0.5
    for entry in (0, 1, 77, 255):
        for ls in (0, 7, 15):
            blk = np.zeros(98 if t == iq.T_IQ3_XXS else 66, np.uint8)
            blk[0:2] = np.array([d], np.float16).view(np.uint8)
            if t == iq.T_IQ2_XXS:
                for ib in range(8):
                    blk[2 + 8 * ib: 6 + 8 * ib] = entry
                    blk[6 + 8 * ib: 10 + 8 * ib] = np.array([ls << 28], "<u4").view(np.uint8)
                want = np.tile(d * (0.5 + ls) * 0.25 * G["iq2xxs"][entry].astype(np.float64), 32)
            else:
                blk[2:66] = entry
                for ib in range(8):
                    blk[66 + 4 * ib: 70 + 4 * ib] = np.array([ls << 28], "<u4").view(np.uint8)
                want = np.tile(d * (0.5 + ls) * 0.5 * G["iq3xxs"][entry].astype(np.float64), 64)
            got = iq.VECTORISED[t](blk, 256)
            assert np.array_equal(got, want.astype(np.float32)), (entry, ls)


def test_sign_index_applies_ksigns():
    """IQ2_XXS with sign index s on group l: element j is negative exactly when
    bit j of ksigns[s] is set."""
    G = iq.grids()
    blk = np.zeros(66, np.uint8)
    blk[0:2] = np.array([1.0], np.float16).view(np.uint8)
    for s in (0, 1, 64, 127):
        aux1 = s << 7                                                 # group l = 1
        blk[6:10] = np.array([aux1], "<u4").view(np.uint8)
        got = iq.VECTORISED[iq.T_IQ2_XXS](blk, 256)[8:16]
        sign = np.where((int(G["ksigns"][s]) >> np.arange(8)) & 1, -1.0, 1.0)
        assert np.array_equal(np.sign(got), sign), s


def test_iq1_m_scale_and_delta():
    """IQ1_M: the f16 scale assembled from the scale words' top nibbles; value
    = d (2 s + 1) (grid + delta), delta = -1/8 when its qh bit is set."""
    G = iq.grids()
    d = 0.25
    blk = np.zeros(56, np.uint8)
    bits = int(np.array([d], np.float16).view(np.uint16)[0])
    words = np.array([((bits >> (4 * k)) & 0xF) << 12 for k in range(4)], np.int64)
    words[0] |= 3 | (5 << 3)                         # ib 0: s 3 (l < 2), 5 (l >= 2)
    blk[48:56] = words.astype("<u2").view(np.uint8)
    blk[0:4] = [10, 20, 30, 40]                      # low 8 index bits of ib 0
    blk[32] = 0x08 | (1 << 4)                        # qh0: delta sign l=0, high bit 0x100 for l=1
    blk[33] = 0x80 | 0x02                            # qh1: high bits 0x200 for l=2, delta sign l=3
    got = iq.VECTORISED[iq.T_IQ1_M](blk, 256)[:32].astype(np.float64)
    idx = [10, 20 | 0x100, 30 | 0x200, 40]
    dlt = [-0.125, 0.125, 0.125, -0.125]
    sc = [3, 3, 5, 5]
    want = np.concatenate([d * (2 * sc[l] + 1) * (G["iq1s"][idx[l]].astype(np.float64) + dlt[l])
                           for l in range(4)])
    assert np.array_equal(got, want)


def test_device_tables_match_the_grids():
    """The product's device tables (csrc/iq_tables.hpp) hold, value for value,
    the grids and ksigns table of the fixture the oracle reads."""
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    hdr = open(os.path.join(root, "artifex-assistantv5_amd", "csrc", "iq_tables.hpp"),
               encoding="utf-8").read()
    with open(os.path.join(root, "tests", "golden", "iq_grids.json"), encoding="utf-8") as f:
        grids = json.load(f)["grids"]
    names = {"iq2xxs_grid": "kIq2xxsGrid", "iq2xs_grid": "kIq2xsGrid", "iq2s_grid": "kIq2sGrid",
             "iq3xxs_grid": "kIq3xxsGrid", "iq3s_grid": "kIq3sGrid", "iq1s_grid": "kIq1sGrid",
             "ksigns_iq2xs": "kKsigns"}
    arrays = dict(re.findall(r"const \w+ (k\w+)\[\d+\] = \{([^}]*)\}", hdr))
    assert sorted(arrays) == sorted(names.values())
    for key, cname in names.items():
        vals = [int(v) for v in arrays[cname].replace("\n", "").split(",") if v.strip()]
        assert vals == list(grids[key]["values"]), key
    # a planted mismatch is caught: one grid value changed
    planted = arrays["kIq2sGrid"].replace("8,", "25,", 1)
    assert [int(v) for v in planted.split(",") if v.strip()] != list(grids["iq2s_grid"]["values"])


def test_tile_model_layout_round_trip():
    """The IQ row-tile layout of the numpy model is a byte permutation of the
    raw rows (d of row r at 2 r, the rest of its block at 32 + r (BS - 2);
    IQ1_M blocks whole at 56 r) and inverts exactly."""
    import tile_model
    for t in (16, 17, 22, 18, 21, 29):
        raw = tile_model.random_blocks(t, 19, 768, seed=t, specials=True)
        tiles = tile_model.to_tiles(t, raw, 19, 768)
        assert tiles.size == tile_model.tiled_bytes(t, 19, 768)
        assert np.array_equal(tile_model.from_tiles(t, tiles, 19, 768), raw)
        bs = tile_model.BLOCK[t][1]
        tu = tiles[:16 * bs]                       # tile 0, superblock 0
        blk = raw.reshape(19, 3, bs)[:, 0]
        for r in (0, 7, 15):
            if t == 29:
                assert np.array_equal(tu[56 * r:56 * r + 56], blk[r])
            else:
                assert np.array_equal(tu[2 * r:2 * r + 2], blk[r, :2])
                assert np.array_equal(tu[32 + r * (bs - 2):32 + (r + 1) * (bs - 2)], blk[r, 2:])
