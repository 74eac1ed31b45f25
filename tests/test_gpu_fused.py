"""Fused decode-step projections (gguf_hip_matmul_fused) against a float64 composition.

The K-quant and 32-element types use the package quantizer's weights; the
grid-codebook IQ types (IQ2_XXS .. IQ1_M) use random valid blocks (every bit
pattern decodes), whose dequantization is pinned to the oracle elsewhere."""
import importlib

import numpy as np
import pytest

import tile_model

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu

GRID = (16, 17, 22, 18, 21, 29)


@pytest.fixture(scope="module")
def mods():
    return (importlib.import_module("artifex-assistantv5_amd"),
            importlib.import_module("artifex-assistantv5_amd.glue"))


def _weight(pkg, t, n, k, seed):
    if t in GRID:
        raw = tile_model.random_blocks(t, n, k, seed=seed)
    else:
        raw = pkg.quantize.quantize(pkg.quantize.synthetic_weight(n, k, seed=seed), t)
    return pkg.repack_gguf_for_gpu(t, raw, n, k, device="cuda")


def _rel(a, b):
    return ((a.double() - b.double()).norm() / b.double().norm()).item()


def _elementwise(y, ref, wd, xd):
    """max_n |y - ref| / sum_k |w[n, k] x[k]|: the per-element criterion of the path,
    insensitive to cancellation in the dot products."""
    scale = wd.abs() @ xd.abs()
    return ((y.double() - ref).abs() / scale).max().item()


@pytest.mark.parametrize("t,n,k", [(12, 6144, 4096), (12, 1000, 4096), (14, 4096, 14336),
                                   (8, 512, 4096), (12, 4096, 14336), (14, 2048, 4096),
                                   (2, 1000, 4096), (6, 512, 14336), (20, 2048, 4096),
                                   (23, 1000, 4096), (23, 4096, 14336), (10, 1000, 4096),
                                   (10, 4096, 14336), (11, 1000, 4096), (11, 4096, 14336),
                                   (16, 1000, 4096), (17, 1000, 4096), (22, 1000, 4096),
                                   (18, 1000, 4096), (21, 1000, 4096), (29, 1000, 4096),
                                   (16, 4096, 14336), (21, 6144, 4096)])
def test_rmsnorm_prologue(mods, t, n, k):
    pkg, glue = mods
    w = _weight(pkg, t, n, k, seed=n + k)
    g = torch.Generator(device="cuda").manual_seed(k)
    x = torch.randn(k, device="cuda", generator=g) * 5
    nw = 1 + 0.1 * torch.randn(k, device="cuda", generator=g)
    y = torch.empty(n, device="cuda")
    glue.matmul_fused(x, w, y, glue.PROLOGUE_RMSNORM, nw, 1e-6)
    xd = x.double()
    h = xd / torch.sqrt((xd * xd).mean() + 1e-6) * nw.double()
    wd = w.dequant().double()
    ref = wd @ h
    assert _rel(y, ref) < 1e-5
    assert _elementwise(y, ref, wd, h) < 1e-6


@pytest.mark.parametrize("t,n,k", [(14, 4096, 14336), (12, 4096, 14336), (8, 256, 2048),
                                   (18, 4096, 14336), (29, 1024, 2048), (17, 512, 4096)])
def test_swiglu_prologue_accumulate(mods, t, n, k):
    pkg, glue = mods
    w = _weight(pkg, t, n, k, seed=7 * n + k)
    g = torch.Generator(device="cuda").manual_seed(n)
    gu = torch.randn(2 * k, device="cuda", generator=g) * 3
    y0 = torch.randn(n, device="cuda", generator=g)
    y = y0.clone()
    glue.matmul_fused(gu, w, y, glue.PROLOGUE_SWIGLU, accumulate=True)
    gd, ud = gu[:k].double(), gu[k:].double()
    a = ud * gd / (1 + torch.exp(-gd))
    wd = w.dequant().double()
    ref = y0.double() + wd @ a
    # f32-grade per element (normwise it is ~1e-5: the products cancel heavily)
    assert _elementwise(y, ref, wd, a) < 1e-6


@pytest.mark.parametrize("t,ffn,k", [(12, 14336, 4096), (12, 512, 2048), (13, 1024, 4096),
                                     (14, 256, 4096), (8, 768, 1024), (23, 1024, 4096),
                                     (10, 1024, 4096), (11, 1024, 4096), (16, 14336, 4096),
                                     (22, 1024, 4096), (21, 512, 2048), (29, 1024, 4096)])
@pytest.mark.parametrize("norm", [False, True])
def test_swiglu_epilogue(mods, t, ffn, k, norm):
    """Interleaved gate / up tiles: y = up * silu(gate) straight from the projection,
    against the float64 composition; the gate / up values themselves equal a plain
    matmul over the interleaved weight, split back by ``split_interleaved``."""
    pkg, glue = mods
    gw, uw = _weight(pkg, t, ffn, k, seed=ffn + k), _weight(pkg, t, ffn, k, seed=ffn + k + 1)
    w = pkg.interleave_tiles(gw, uw)
    g = torch.Generator(device="cuda").manual_seed(ffn)
    x = torch.randn(k, device="cuda", generator=g) * 2
    nw = 1 + 0.1 * torch.randn(k, device="cuda", generator=g)
    y = torch.full((ffn,), float("nan"), device="cuda")
    if norm:
        glue.matmul_fused(x, w, y, glue.PROLOGUE_RMSNORM, nw, 1e-5, epilogue=glue.EPILOGUE_SWIGLU)
        xd = x.double()
        h = xd / torch.sqrt((xd * xd).mean() + 1e-5) * nw.double()
    else:
        glue.matmul_fused(x, w, y, epilogue=glue.EPILOGUE_SWIGLU)
        h = x.double()
    gd, ud = gw.dequant().double(), uw.dequant().double()
    gv, uv = gd @ h, ud @ h
    ref = uv * gv / (1 + torch.exp(-gv))
    # per element, relative to the magnitudes that enter: |d up| silu(g) + |up| |d silu(g)|
    sg, su = gd.abs() @ h.abs(), ud.abs() @ h.abs()
    bound = su * gv.abs() + uv.abs() * sg * 1.1
    assert torch.isfinite(y).all()
    assert ((y.double() - ref).abs() / bound).max().item() < 1e-6
    # the raw rows: the interleaved matmul, split, equals the row-concatenated one
    # (same number of row tiles, hence the same K split and summation order)
    r = torch.empty(1, 2 * ffn, device="cuda")
    pkg.dispatch_matmul_gguf(x.view(1, -1), w, r, 1, 2 * ffn, k)
    c = torch.empty(1, 2 * ffn, device="cuda")
    pkg.dispatch_matmul_gguf(x.view(1, -1), pkg.concat_rows(gw, uw), c, 1, 2 * ffn, k)
    gs, us = pkg.split_interleaved(r)
    assert torch.equal(gs, c[:, :ffn]) and torch.equal(us, c[:, ffn:])


def test_plain_accumulate_matches_matmul(mods):
    pkg, glue = mods
    w = _weight(pkg, 12, 4096, 4096, seed=3)
    x = torch.randn(4096, device="cuda")
    y0 = torch.randn(4096, device="cuda")
    y = y0.clone()
    glue.matmul_fused(x, w, y, accumulate=True)
    z = torch.empty(1, 4096, device="cuda")
    pkg.dispatch_matmul_gguf(x.view(1, -1), w, z, 1, 4096, 4096)
    assert torch.allclose(y, y0 + z[0], rtol=1e-6, atol=1e-6)   # same kernel, plus one add
    z2 = torch.empty(4096, device="cuda")
    glue.matmul_fused(x, w, z2)
    assert torch.equal(z2, z[0])


def _attention_inputs(nh, nkv, hd, max_seq, p):
    g = torch.Generator(device="cuda").manual_seed(p + 3 * nh + hd)
    qkv = torch.randn((nh + 2 * nkv) * hd, device="cuda", generator=g)
    kc = torch.randn(nkv, max_seq, hd, device="cuda", generator=g)
    vc = torch.randn(nkv, max_seq, hd, device="cuda", generator=g)
    half = hd // 2
    inv = 1.0 / (10000.0 ** (torch.arange(half, dtype=torch.float64) * 2 / hd))
    ang = torch.arange(max_seq, dtype=torch.float64)[:, None] * inv[None]
    return qkv, kc, vc, ang.cos().float().cuda(), ang.sin().float().cuda()


# positions: one split, a full split, two splits, the register chunk of eight
# splits exactly, and ranges past it (records merged one at a time)
@pytest.mark.parametrize("t,nh,nkv,hd,max_seq,p", [
    (12, 32, 8, 128, 1200, 0), (12, 32, 8, 128, 1200, 63), (12, 32, 8, 128, 1200, 64),
    (12, 32, 8, 128, 1200, 300), (12, 32, 8, 128, 1200, 511), (12, 32, 8, 128, 1200, 1199),
    (14, 32, 8, 128, 640, 383), (8, 8, 8, 64, 128, 100), (12, 16, 2, 256, 700, 650),
    (13, 64, 8, 128, 256, 200), (23, 32, 8, 128, 300, 130), (10, 32, 8, 128, 300, 77),
    (11, 32, 8, 128, 300, 200), (16, 32, 8, 128, 640, 383), (17, 32, 8, 128, 300, 64),
    (22, 32, 8, 128, 300, 130), (18, 16, 2, 256, 700, 650), (21, 32, 8, 128, 1200, 1199),
    (29, 32, 8, 128, 300, 0)])
def test_attention_merge_projection(mods, t, nh, nkv, hd, max_seq, p):
    """Records-only attention + the merge prologue equal, bit for bit, attention
    with its own merge followed by the plain fused projection (same arithmetic
    in the same order), for STORE and ACCUMULATE."""
    _merge_case(mods, t, nh, nkv, hd, max_seq, p, 1024)


# the 32-element-block types at the decoder's output-projection shape (32 x 128
# heads, N = 4096), whose K split and waves per workgroup differ from N = 1024
@pytest.mark.parametrize("t", [2, 6, 8, 20])
@pytest.mark.parametrize("p", [130, 511])
def test_attention_merge_projection_n4096_small_blocks(mods, t, p):
    _merge_case(mods, t, 32, 8, 128, 600, p, 4096)


def _merge_case(mods, t, nh, nkv, hd, max_seq, p, n):
    pkg, glue = mods
    k = nh * hd
    w = _weight(pkg, t, n, k, seed=k + p)
    qkv, kc, vc, cos, sin = _attention_inputs(nh, nkv, hd, max_seq, p)
    kc2, vc2 = kc.clone(), vc.clone()
    pos = torch.tensor([p], device="cuda")
    work_a = glue.attention_workspace(nh, nkv, hd, max_seq, "cuda")
    work_b = glue.attention_workspace(nh, nkv, hd, max_seq, "cuda")
    work_b.fill_(float("nan"))           # records-only mode reads no counters, writes every record
    a = torch.empty(k, device="cuda")
    glue.attention_decode(qkv, pos, cos, sin, kc, vc, a, nh, nkv, hd, work_a)
    assert glue.attention_decode(qkv, pos, cos, sin, kc2, vc2, None, nh, nkv, hd, work_b) is None
    assert torch.equal(kc, kc2) and torch.equal(vc, vc2)      # both wrote slot p the same way
    y_ref = torch.empty(n, device="cuda")
    glue.matmul_fused(a, w, y_ref)
    y = torch.full((n,), float("nan"), device="cuda")
    glue.matmul_attn_merge(work_b, pos, w, y, nh, nkv, hd, max_seq)
    assert torch.equal(y, y_ref), (y - y_ref).abs().max().item()
    # accumulate into a residual
    r = torch.randn(n, device="cuda")
    y_acc, y_acc_ref = r.clone(), r.clone()
    glue.matmul_fused(a, w, y_acc_ref, accumulate=True)
    glue.matmul_attn_merge(work_b, pos, w, y_acc, nh, nkv, hd, max_seq, accumulate=True)
    assert torch.equal(y_acc, y_acc_ref)
    # and against float64: a from the attention test's reference path is covered
    # there; here the projection of the merged output
    wd = w.dequant().double()
    ref = wd @ a.double()
    assert _rel(y, ref) < 1e-4
    assert _elementwise(y, ref, wd, a.double()) < 1e-6


def test_attention_merge_bad_position(mods):
    """A position outside the cache leaves the records unwritten; the merged
    projection then yields NaN instead of a stale result."""
    pkg, glue = mods
    nh, nkv, hd, max_seq = 32, 8, 128, 256
    w = _weight(pkg, 12, 256, nh * hd, seed=5)
    work = glue.attention_workspace(nh, nkv, hd, max_seq, "cuda")
    y = torch.zeros(256, device="cuda")
    for p in (max_seq, -1):
        glue.matmul_attn_merge(work, torch.tensor([p], device="cuda"), w, y, nh, nkv, hd, max_seq)
        assert torch.isnan(y).all()


def test_fused_lm_head_full_vocab(mods):
    """The decode step's LM head: RMSNorm prologue over a Q6_K weight of 151936 x 4096."""
    pkg, glue = mods
    dec = importlib.import_module("artifex-assistantv5_amd.decoder")
    n, k = 151936, 4096
    w = dec._tiled_rows(14, 2048, n, k, seed=11, device="cuda")
    g = torch.Generator(device="cuda").manual_seed(5)
    x = torch.randn(k, device="cuda", generator=g) * 3
    nw = 1 + 0.02 * torch.randn(k, device="cuda", generator=g)
    y = torch.empty(n, device="cuda")
    glue.matmul_fused(x, w, y, glue.PROLOGUE_RMSNORM, nw, 1e-6)
    xd = x.double()
    h = xd / torch.sqrt((xd * xd).mean() + 1e-6) * nw.double()
    wd = w.dequant().double()
    ref = wd @ h
    assert torch.isfinite(y).all()
    assert _rel(y, ref) < 1e-5
    assert _elementwise(y, ref, wd, h) < 1e-6
    del wd
    torch.cuda.empty_cache()
