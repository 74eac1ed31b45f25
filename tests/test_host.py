"""Host-side logic (CPU only): type traits, layout math, quantizer, layout model."""

import importlib

import numpy as np
import pytest

import tile_model


def test_type_traits_mirror_reference(pkg):
    g = pkg.ggml
    # gguf.ts:39-73
    assert g.ggml_type_traits(8)[:2] == (32, 34)
    assert g.ggml_type_traits(12)[:2] == (256, 144)
    assert g.ggml_type_traits(14)[:2] == (256, 210)
    assert g.ggml_type_traits(13)[:2] == (256, 176)
    assert g.ggml_type_traits(30)[:2] == (1, 2)
    with pytest.raises(NotImplementedError, match="Unsupported ggml type 99"):
        g.ggml_type_traits(99)


def test_tensor_bytes(pkg):
    g = pkg.ggml
    # gguf.ts:82-92: rowSize(ne0) x prod(outer)
    assert g.ggml_tensor_bytes(12, [4096, 14336]) == 33_030_144
    assert g.ggml_tensor_bytes(14, [4096, 151936]) == 510_504_960
    assert g.ggml_tensor_bytes(8, [4096, 4096]) == 17_825_792
    with pytest.raises(ValueError, match="not divisible by block size"):
        g.ggml_tensor_bytes(12, [100, 3])


@pytest.mark.parametrize("t", [2, 6, 8, 10, 11, 12, 13, 14, 20, 23])
@pytest.mark.parametrize("k", [256, 512, 768, 1280, 4096, 14336])
def test_tile_row_bytes(pkg, t, k):
    trb = pkg.tile_row_bytes(t, k)
    assert trb == tile_model.tile_row_bytes(t, k) == pkg.raw_row_bytes(t, k)
    for n in (1, 15, 16, 17, 14336):
        assert pkg.tiled_bytes(t, n, k) == tile_model.tiled_bytes(t, n, k)
        assert pkg.tiled_bytes(t, n, k) == -(-n // 16) * 16 * trb
        assert (16 * trb) % 16 == 0                       # every tile starts 16-byte aligned


def test_tile_row_bytes_rejects(pkg):
    with pytest.raises(ValueError):
        pkg.tile_row_bytes(12, 100)
    with pytest.raises(NotImplementedError):
        pkg.tile_row_bytes(3, 256)             # Q4_1: known type, no kernel


def test_layout_model_is_a_permutation_of_each_tile_unit():
    for t in (8, 12, 13, 14):
        block, ub = tile_model.BLOCK[t]
        pos = tile_model._unit_maps(t)          # asserts the map is a bijection
        assert pos.shape == (16, ub)
    # header / d of row r sits at a fixed place (what the kernels read directly)
    assert tile_model._unit_maps(12)[5, 0] == 80
    assert tile_model._unit_maps(14)[3, 208] == 3328 + 6
    assert tile_model._unit_maps(8)[7, 0] == 14


@pytest.mark.parametrize("t,k", [(8, 96), (8, 4096), (12, 512), (13, 1024), (14, 768), (14, 4096),
                                 (2, 96), (6, 160), (20, 4096)])
@pytest.mark.parametrize("n", [5, 16, 37])
def test_layout_model_roundtrip(ref, t, k, n):
    raw = tile_model.random_blocks(t, n, k, seed=t + k)
    tiles = tile_model.to_tiles(t, raw, n, k)
    assert tiles.size == tile_model.tiled_bytes(t, n, k)
    back = tile_model.from_tiles(t, tiles, n, k)
    assert np.array_equal(back, raw)
    # padding rows of the last tile are zero
    pad = tile_model.tiled_rows(n) - n
    full = tile_model.from_tiles(t, tiles, n + pad, k)
    assert not full[raw.size:].any()
    assert ref.same_bits(ref.dequant_rows(t, back, 5, k), ref.dequant_rows(t, raw, 5, k))


@pytest.mark.parametrize("t", [2, 6, 8, 10, 11, 12, 13, 14, 20, 23])
def test_quantize_deterministic_and_sized(pkg, t):
    w = pkg.quantize.synthetic_weight(3, 512, seed=11)
    a = pkg.quantize.quantize(w, t)
    b = pkg.quantize.quantize(w.copy(), t)
    assert np.array_equal(a, b)
    assert a.size == pkg.ggml_tensor_bytes(t, [512, 3])


def test_quantize_rejects(pkg):
    with pytest.raises(ValueError):
        pkg.quantize.quantize(np.zeros((2, 100), np.float32), 12)
    with pytest.raises(NotImplementedError):
        pkg.quantize.quantize(np.zeros((2, 256), np.float32), 3)       # Q4_1


def test_synthetic_inputs_seeded(pkg):
    a = pkg.quantize.synthetic_activations(2, 64, seed=5)
    b = pkg.quantize.synthetic_activations(2, 64, seed=5)
    assert np.array_equal(a, b) and a.dtype == np.float32
    h = pkg.quantize.synthetic_activations(2, 64, seed=5, dtype=np.float16)
    assert h.dtype == np.float16 and np.array_equal(h, a.astype(np.float16))


def test_decoder_weight_bytes_per_token():
    dec = importlib.import_module("artifex-assistantv5_amd.decoder")
    cfg = dec.DecoderConfig()
    # 137.82 MB per layer (Q4_K q/k/v/o and gate/up, Q6_K down) + 510.5 MB Q6_K LM head
    assert cfg.weight_bytes_per_token() == 32 * 137_822_208 + 510_504_960
    assert cfg.qkv_rows == 6144


def test_decoder_rope_tables_and_norm():
    import torch
    dec = importlib.import_module("artifex-assistantv5_amd.decoder")
    cfg = dec.DecoderConfig(head_dim=8, max_seq=4, rope_base=100.0)
    cos, sin = dec.rope_tables(cfg, "cpu")
    # theta(pos, i) = pos / base^(2i/d): position 0 is the identity, pairs i and i + d/2
    x = torch.arange(8, dtype=torch.float32).view(1, 1, 8)
    y = dec.apply_rope(x, cos[:1], sin[:1])
    assert torch.equal(x, y)
    y = dec.apply_rope(x, cos[3:4], sin[3:4])
    th = 3.0 / 100.0 ** (torch.arange(4, dtype=torch.float64) * 2 / 8)
    z = torch.complex(x[0, 0, :4].double(), x[0, 0, 4:].double()) * torch.exp(1j * th)
    assert torch.allclose(y[0, 0].double(), torch.cat([z.real, z.imag]), atol=1e-6)
    v = torch.tensor([[3.0, 4.0]])
    assert torch.allclose(dec.rms_norm(v, torch.ones(2), 0.0), v / (12.5 ** 0.5))


def test_glue_rejects_mismatched_buffers(pkg):
    """Every glue wrapper checks element counts against the launch shape before
    anything reaches the C ABI (CPU tensors: the size check comes first)."""
    import types
    import torch
    from importlib import import_module
    glue = import_module("artifex-assistantv5_amd.glue")
    z = lambda *s: torch.zeros(*s)  # noqa: E731
    cases = [
        (lambda: glue.rmsnorm(z(2, 8), z(7), 1e-5, z(2, 8)), "rmsnorm: w"),
        (lambda: glue.rmsnorm(z(2, 8), z(8), 1e-5, z(8)), "rmsnorm: out"),
        (lambda: glue.add_rmsnorm(z(2, 8), z(8), z(8), 1e-5, z(2, 8)), "add_rmsnorm: res"),
        (lambda: glue.add_rmsnorm(z(2, 8), z(2, 8), z(4), 1e-5, z(2, 8)), "add_rmsnorm: w"),
        (lambda: glue.add_rmsnorm(z(2, 8), z(2, 8), z(8), 1e-5, z(1, 8)), "add_rmsnorm: out"),
        (lambda: glue.swiglu(z(2, 15), z(2, 8)), "swiglu: gate_up"),
        (lambda: glue.swiglu(z(4, 8), z(2, 8)), "swiglu: gate_up rows"),
        (lambda: glue.attention_decode(z(6 * 64), z(1), z(16, 32), z(16, 32), z(2, 16, 32), z(2, 16, 64),
                                       None, 4, 1, 64, z(1)), "k_cache rows"),
        (lambda: glue.attention_decode(z(6 * 64), z(1), z(16, 32), z(16, 32), z(2, 16, 64), z(2, 16, 64),
                                       None, 4, 1, 64, z(1)), "attention_decode: k_cache"),
        (lambda: glue.attention_decode(z(6 * 64), z(1), z(16, 32), z(16, 32), z(1, 16, 64), z(2, 16, 64),
                                       None, 4, 1, 64, z(1)), "attention_decode: v_cache"),
        (lambda: glue.attention_decode(z(5 * 64), z(1), z(16, 32), z(16, 32), z(1, 16, 64), z(1, 16, 64),
                                       None, 4, 1, 64, z(1)), "attention_decode: qkv"),
        (lambda: glue.attention_decode(z(6 * 64), z(1), z(15, 32), z(16, 32), z(1, 16, 64), z(1, 16, 64),
                                       None, 4, 1, 64, z(1)), "attention_decode: cos"),
        (lambda: glue.attention_decode(z(6 * 64), z(1), z(16, 32), z(16, 31), z(1, 16, 64), z(1, 16, 64),
                                       None, 4, 1, 64, z(1)), "attention_decode: sin"),
        (lambda: glue.attention_decode(z(6 * 64), z(1), z(16, 32), z(16, 32), z(1, 16, 64), z(1, 16, 64),
                                       z(255), 4, 1, 64, z(1)), "attention_decode: out"),
        (lambda: glue.attention_decode(z(6 * 64), z(2), z(16, 32), z(16, 32), z(1, 16, 64), z(1, 16, 64),
                                       None, 4, 1, 64, z(1)), "pos must hold one"),
        (lambda: glue.argmax(z(0), z(1), z(1)), "argmax"),
        # prefill attention: 4 / 1 heads of 64, max_seq 16, rows of 384 (qkv) and 256 (out)
        (lambda: glue.attention_prefill(z(3 * 384), z(3), z(16, 32), z(16, 32), z(1, 16, 64),
                                        z(1, 16, 64), z(3, 256), 4, 1, 64), "same M"),
        (lambda: glue.attention_prefill(z(3, 384), z(2), z(16, 32), z(16, 32), z(1, 16, 64),
                                        z(1, 16, 64), z(3, 256), 4, 1, 64), "pos holds 2"),
        (lambda: glue.attention_prefill(z(3, 384), z(3), z(16, 32), z(16, 32), z(1, 16, 32),
                                        z(1, 16, 64), z(3, 256), 4, 1, 64), "k_cache must be"),
        (lambda: glue.attention_prefill(z(3, 384), z(3), z(16, 32), z(16, 32), z(1, 16, 64),
                                        z(2, 16, 64), z(3, 256), 4, 1, 64), "prefill: v_cache"),
        (lambda: glue.attention_prefill(z(3, 384), z(3), z(15, 32), z(16, 32), z(1, 16, 64),
                                        z(1, 16, 64), z(3, 256), 4, 1, 64), "prefill: cos"),
        (lambda: glue.attention_prefill(z(3, 383), z(3), z(16, 32), z(16, 32), z(1, 16, 64),
                                        z(1, 16, 64), z(3, 256), 4, 1, 64), "qkv rows hold 383"),
        (lambda: glue.attention_prefill(z(3, 384), z(3), z(16, 32), z(16, 32), z(1, 16, 64),
                                        z(1, 16, 64), z(3, 250), 4, 1, 64), "out rows 250"),
        (lambda: glue.attention_prefill(z(3, 384), z(3), z(16, 32), z(16, 32), z(1, 16, 64),
                                        z(1, 16, 64), z(3, 256), 4, 1, 64), "float32 device rows"),
    ]
    w = types.SimpleNamespace(k=256, n=64, ggml_type=12)
    cases += [
        (lambda: glue.matmul_fused(z(255), w, z(64)), "matmul_fused: x"),
        (lambda: glue.matmul_fused(z(256), w, z(63)), "matmul_fused: x"),
        (lambda: glue.matmul_fused(z(256), w, z(64), glue.PROLOGUE_RMSNORM, z(255)), "norm_w"),
        (lambda: glue.matmul_fused(z(512), w, z(64), glue.PROLOGUE_SWIGLU, None,
                                   epilogue=glue.EPILOGUE_SWIGLU), "matmul_fused: x"),
        (lambda: glue.matmul_attn_merge(z(1), z(2), w, z(64), 4, 1, 64, 16), "pos must hold one"),
    ]
    for fn, msg in cases:
        with pytest.raises(ValueError, match=msg):
            fn()


def test_matmul_workspace_keying_and_growth():
    """One matmul workspace per (device, stream), a separate one under graph
    capture; sizes grow to the next power of two (at least 1 MiB)."""
    lin = importlib.import_module("artifex-assistantv5_amd.linear")
    k = lin.workspace_key
    assert k(0, 111, False) != k(0, 222, False)      # two streams of one device
    assert k(0, 111, False) != k(1, 111, False)      # two devices
    assert k(0, 111, False) != k(0, 111, True)       # eager vs captured on one stream
    assert k(0, 111, False) == k(0, 111, False)
    size = lin.workspace_size
    assert size(1) == 1 << 20 and size(1 << 20) == 1 << 20
    assert size((1 << 20) + 1) == 1 << 21
    assert size(33_000_000) == 1 << 25 and size(1 << 25) == 1 << 25
    # growth is geometric: a run of slowly growing requests reallocates O(log) times
    sizes = {size(n) for n in range(1 << 20, 1 << 26, 1 << 18)}
    assert sizes == {1 << e for e in range(20, 27)}


def test_missing_library_raises(pkg):
    """No CPU fallback: a missing shared library is an error, not a silent path."""
    from importlib import import_module
    native = import_module("artifex-assistantv5_amd._native")
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        native.load_library("/nonexistent/libgguf_hip.so")


def test_package_never_imports_the_oracle():
    """The oracle is test infrastructure: no module of the package imports or
    reads anything under oracle/ (the product path is the HIP library)."""
    import os
    import re
    root = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))),
                        "artifex-assistantv5_amd")
    bad = []
    for dirpath, _, files in os.walk(root):
        for f in files:
            if f.endswith((".py", ".hip", ".hpp", ".h", ".c")):
                text = open(os.path.join(dirpath, f), encoding="utf-8").read()
                if re.search(r"^\s*(import|from)\s+oracle|gguf_ref|gguf_iq|liboracle", text, re.M):
                    bad.append(f)
    assert not bad, bad
