"""GPU: repack and dequantization, bit-exact to the oracle (gguf-dequant.ts)."""

import numpy as np
import pytest
import torch

import tile_model

pytestmark = pytest.mark.gpu

SHAPES = {8: [(1, 32), (3, 96), (5, 4096), (2, 160)],
          12: [(1, 256), (4, 768), (3, 4096), (2, 14336)],
          13: [(1, 256), (4, 768), (3, 4096), (2, 14336)],
          14: [(1, 256), (4, 768), (3, 4096), (2, 14336)],
          2: [(1, 32), (3, 96), (5, 4096), (2, 160)],
          6: [(1, 32), (3, 96), (5, 4096), (2, 160)],
          20: [(1, 32), (3, 96), (5, 4096), (2, 160)], 23: [(1, 256), (3, 512), (17, 4096)],
          10: [(1, 256), (4, 768), (17, 4096), (2, 14336)],
          11: [(1, 256), (4, 768), (17, 4096)]}
ALL = [2, 6, 8, 10, 11, 12, 13, 14, 20, 23]


def _dev_u8(a):
    return torch.from_numpy(np.ascontiguousarray(a, np.uint8)).cuda()


def test_golden_vectors_on_gpu(pkg, ref, golden_samples):
    for s in golden_samples:
        t = s["ggml_type"]
        if t not in (8, 12, 13, 14):
            continue
        raw = np.frombuffer(bytes.fromhex(s["bytes_hex"]), np.uint8)
        want = np.array(s["expected_f32"], np.float64).astype(np.float32)
        n = s["n_elements"]
        w = pkg.repack_gguf_for_gpu(t, raw, n)          # one row of n elements
        got = w.dequant().cpu().numpy().reshape(-1)
        assert ref.same_bits(got, want), (s["tensor"], "tiles")
        got_raw = pkg.dequant_raw(t, raw, n).cpu().numpy()
        assert ref.same_bits(got_raw, want), (s["tensor"], "raw")


@pytest.mark.parametrize("t", ALL)
@pytest.mark.parametrize("specials", [False, True])
def test_repack_layout_and_dequant_bit_exact(pkg, ref, t, specials):
    for i, (n, k) in enumerate(SHAPES[t]):
        raw = tile_model.random_blocks(t, n, k, seed=31 * t + i, specials=specials)
        w = pkg.repack_gguf_for_gpu(t, raw, n, k)
        tiles = w.data.cpu().numpy()
        assert np.array_equal(tiles, tile_model.to_tiles(t, raw, n, k)), (n, k)
        want = ref.dequant_rows(t, raw, n, k)
        assert ref.same_bits(w.dequant().cpu().numpy(), want), (n, k)
        assert ref.same_bits(pkg.dequant_raw(t, raw, n * k).cpu().numpy(), want.reshape(-1))


@pytest.mark.parametrize("t", ALL)
def test_repack_from_unaligned_raw(pkg, ref, t):
    n, k = 3, 512
    raw = tile_model.random_blocks(t, n, k, seed=77)
    buf = torch.zeros(raw.size + 5, dtype=torch.uint8, device="cuda")
    buf[3:3 + raw.size] = _dev_u8(raw)
    view = buf[3:3 + raw.size]                      # odd device address
    w = pkg.repack_gguf_for_gpu(t, view, n, k)
    assert ref.same_bits(w.dequant().cpu().numpy(), ref.dequant_rows(t, raw, n, k))
    assert ref.same_bits(pkg.dequant_raw(t, view, n * k).cpu().numpy(),
                         ref.dequant_rows(t, raw, n, k).reshape(-1))


@pytest.mark.parametrize("t", ALL)
def test_row_views_and_concat(pkg, ref, t):
    k = 512
    raw = tile_model.random_blocks(t, 40, k, seed=5)
    w = pkg.repack_gguf_for_gpu(t, raw, 40, k)
    want = ref.dequant_rows(t, raw, 40, k)
    assert ref.same_bits(w.rows(16, 37).dequant().cpu().numpy(), want[16:37])
    cat = pkg.concat_rows(w.rows(0, 16), w.rows(16, 40))
    assert ref.same_bits(cat.dequant().cpu().numpy(), want)
    with pytest.raises(ValueError):
        w.rows(3, 7)                                   # views start on a tile boundary
    with pytest.raises(ValueError):
        pkg.concat_rows(w.rows(0, 20), w.rows(32, 40))  # inner parts are whole tiles


@pytest.mark.parametrize("t,n,k", [(12, 14336, 4096), (12, 4096, 14336), (14, 4096, 14336),
                                   (8, 4096, 4096), (14, 151936, 4096), (2, 14336, 4096),
                                   (6, 4096, 14336), (20, 4096, 4096)])
def test_full_size_dequant(pkg, ref, t, n, k):
    """Full configuration sizes: repack+dequant equals raw dequant everywhere (GPU vs
    GPU, size independent) and equals the oracle on a sample of rows."""
    rng = np.random.default_rng(n + k + t)
    block, size = tile_model.BLOCK[t]
    rows_bytes = k // block * size
    raw_dev = torch.randint(0, 256, (n * rows_bytes,), dtype=torch.uint8, device="cuda")
    # stamp finite scales into every block on the device
    blocks = raw_dev.view(-1, size)
    offs = {8: [0], 12: [0, 2], 13: [0, 2], 14: [208], 2: [0], 6: [0], 20: [0], 23: [0], 10: [80, 82], 11: [108]}[t]
    for o in offs:
        vals = torch.empty(blocks.shape[0], device="cuda").uniform_(0.001, 0.01).half()
        blocks[:, o:o + 2] = vals.view(torch.uint8).view(-1, 2)
    w = pkg.repack_gguf_for_gpu(t, raw_dev, n, k)
    deq = w.dequant()
    deq_raw = pkg.dequant_raw(t, raw_dev, n * k).view(n, k)
    assert torch.equal(deq.view(torch.int32), deq_raw.view(torch.int32))
    sample = np.sort(rng.choice(n, size=min(n, 64), replace=False))
    raw_rows = raw_dev.view(n, rows_bytes)[torch.from_numpy(sample).cuda()].cpu().numpy()
    want = ref.dequant_rows(t, raw_rows.reshape(-1), len(sample), k)
    assert ref.same_bits(deq[torch.from_numpy(sample).cuda()].cpu().numpy(), want)
