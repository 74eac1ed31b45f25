"""GPU: the matmul paths have no activation range limit beyond f32's own.

The reference's GEMVs take f32 activations and are scale-invariant
(webgpu/src/shaders/matmul_gguf.wgsl:3191-3245).  Here activations enter f16
matrix cores, so every path scales them by powers of two first: the decode
kernels per 256- or 32-element unit of each row (then an exact f16 hi + lo
split), the GEMM per row (then fp16 rounding).  These tests draw the usual
N(0, 1) activations times 2^-60 .. 2^60, rows that mix 1e-6 and 1e4
magnitudes, and units whose largest element is far from the rest, and hold
every result to the same gates as at unit scale, against the oracle's f64
product (the gates are scale-invariant):

  decode   per element |y - y_ref| <= 2e-5 * sum_k |x_k w_nk|, normwise <= 1e-3
  GEMM     per element and normwise <= 1e-3
  fused    the float64 composition, with the thresholds of test_gpu_fused.py
"""

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

TYPES = [2, 6, 8, 10, 11, 12, 13, 14, 20, 23]
SCALES = [2.0 ** -60, 2.0 ** -24, 2.0 ** -16, 2.0 ** -8, 2.0 ** 8, 2.0 ** 15, 2.0 ** 60]
DECODE, GEMM, AUTO = 1, 2, 0
DECODE_TOL = 2e-5


def _case(pkg, t, n, k, seed):
    w = pkg.quantize.synthetic_weight(n, k, seed=seed)
    raw = pkg.quantize.quantize(w, t)
    return raw, pkg.repack_gguf_for_gpu(t, raw, n, k)


def _mixed_rows(m, k, seed):
    """N(0, 1) times 1e-6 or 1e4 per element, at random: every unit mixes both."""
    rng = np.random.default_rng(seed)
    mag = np.where(rng.random((m, k)) < 0.5, 1e-6, 1e4)
    return (rng.standard_normal((m, k)) * mag).astype(np.float32)


def _spiky_rows(m, k, seed):
    """N(0, 1) rows with one element per 32 raised to 1e5: each unit's scale is
    set by its spike, the rest sits 2^17 lower."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((m, k)).astype(np.float32)
    x[:, rng.integers(0, 32)::32] *= 1e5
    return x


def _metrics(ref, y, x, wdeq):
    x64 = np.asarray(x, np.float64)
    return ref.parity_metrics(y, ref.matmul_bt(x64, wdeq), ref.matmul_bt_abs(x64, wdeq))


@pytest.mark.parametrize("t", TYPES)
@pytest.mark.parametrize("m", [1, 8, 32])
def test_decode_any_scale(pkg, ref, t, m):
    n, k = 80, 1024
    raw, w = _case(pkg, t, n, k, seed=31 * t + m)
    wdeq = ref.dequant_rows(t, raw, n, k)
    base = pkg.quantize.synthetic_activations(m, k, seed=100 + m)
    cases = [("scale", s, (base * np.float32(s)).astype(np.float32)) for s in SCALES]
    cases += [("mixed", 0, _mixed_rows(m, k, 7 + m)), ("spiky", 0, _spiky_rows(m, k, 9 + m))]
    for name, s, x in cases:
        assert np.isfinite(x).all()
        y = pkg.qlinear(torch.from_numpy(x).cuda(), w, variant=DECODE).cpu().numpy()
        met = _metrics(ref, y, x, wdeq)
        assert met["finite"] and met["elemwise"] <= DECODE_TOL and met["normwise"] <= 1e-3, (
            t, m, name, s, met)


@pytest.mark.parametrize("t", TYPES)
def test_decode_any_scale_f16(pkg, ref, t):
    """f16 activations at the edges of the f16 range (subnormal to 65504)."""
    n, k = 48, 512
    raw, w = _case(pkg, t, n, k, seed=7 * t)
    wdeq = ref.dequant_rows(t, raw, n, k)
    base = pkg.quantize.synthetic_activations(8, k, seed=5)
    for s in (2.0 ** -20, 2.0 ** -12, 2.0 ** 13):
        x = np.clip(base * s, -65504, 65504).astype(np.float16)
        for m in (1, 8):
            y = pkg.qlinear(torch.from_numpy(x[:m]).cuda(), w, variant=DECODE).cpu().numpy()
            met = _metrics(ref, y, x[:m].astype(np.float32), wdeq)
            assert met["finite"] and met["elemwise"] <= DECODE_TOL, (t, m, s, met)


@pytest.mark.parametrize("t", [12, 14, 8, 2, 10, 23])
@pytest.mark.parametrize("m", [40, 64, 300, 600])
def test_gemm_f32_rows_any_scale(pkg, ref, t, m):
    """f32 activations through the GEMM (explicit variant) with rows scaled to
    1e4, 1e-5, 2^15 and 2^-24 side by side, plus a mixed row; AUTO keeps f32
    batches below 512 rows on the f32-grade decode path."""
    n, k = 96, 1024
    raw, w = _case(pkg, t, n, k, seed=m + t)
    wdeq = ref.dequant_rows(t, raw, n, k)
    x = pkg.quantize.synthetic_activations(m, k, seed=m)
    row_scale = np.array([1e4, 1e-5, 2.0 ** 15, 2.0 ** -24, 1.0], np.float64)[np.arange(m) % 5]
    x = (x * row_scale[:, None]).astype(np.float32)
    x[m // 2] = _mixed_rows(1, k, m)[0]
    xt = torch.from_numpy(x).cuda()
    y = pkg.qlinear(xt, w, variant=GEMM).cpu().numpy()
    met = _metrics(ref, y, x, wdeq)
    assert met["ok"], (t, m, "gemm", met)
    y = pkg.qlinear(xt, w, variant=AUTO).cpu().numpy()
    met = _metrics(ref, y, x, wdeq)
    if m < 512:
        assert met["finite"] and met["elemwise"] <= DECODE_TOL, (t, m, "auto", met)
    else:
        assert met["ok"], (t, m, "auto", met)


def _elementwise(y, refv, wd, xd):
    return ((y.double() - refv).abs() / (wd.abs() @ xd.abs())).max().item()


@pytest.mark.parametrize("t", [12, 14, 8, 23, 10])
@pytest.mark.parametrize("scale", [2.0 ** -24, 2.0 ** -8, 2.0 ** 8, 2.0 ** 15, 2.0 ** 40])
def test_rmsnorm_prologue_any_scale(pkg, t, scale):
    """The RMSNorm prologue stages the unnormalised x * w: a residual stream at
    any magnitude."""
    glue = __import__("importlib").import_module("artifex-assistantv5_amd.glue")
    n, k = 1000, 4096
    w = pkg.repack_gguf_for_gpu(t, pkg.quantize.quantize(
        pkg.quantize.synthetic_weight(n, k, seed=t), t), n, k)
    g = torch.Generator(device="cuda").manual_seed(t)
    x = torch.randn(k, device="cuda", generator=g) * scale
    nw = 1 + 0.1 * torch.randn(k, device="cuda", generator=g)
    y = torch.empty(n, device="cuda")
    glue.matmul_fused(x, w, y, glue.PROLOGUE_RMSNORM, nw, 1e-6)
    xd = x.double()
    h = xd / torch.sqrt((xd * xd).mean() + 1e-6) * nw.double()
    wd = w.dequant().double()
    refv = wd @ h
    assert torch.isfinite(y).all()
    assert _elementwise(y, refv, wd, h) < 1e-6, (t, scale)


@pytest.mark.parametrize("t", [14, 12])
@pytest.mark.parametrize("scale", [2.0 ** -12, 2.0 ** 12])
def test_swiglu_prologue_any_scale(pkg, t, scale):
    glue = __import__("importlib").import_module("artifex-assistantv5_amd.glue")
    n, k = 1024, 4096
    w = pkg.repack_gguf_for_gpu(t, pkg.quantize.quantize(
        pkg.quantize.synthetic_weight(n, k, seed=t + 1), t), n, k)
    g = torch.Generator(device="cuda").manual_seed(n)
    gu = torch.randn(2 * k, device="cuda", generator=g) * scale
    y = torch.empty(n, device="cuda")
    glue.matmul_fused(gu, w, y, glue.PROLOGUE_SWIGLU)
    gd, ud = gu[:k].double(), gu[k:].double()
    a = ud * gd / (1 + torch.exp(-gd))
    wd = w.dequant().double()
    assert torch.isfinite(y).all()
    assert _elementwise(y, wd @ a, wd, a) < 1e-6, (t, scale)


@pytest.mark.parametrize("scale", [2.0 ** -24, 2.0 ** 15])
def test_attention_merge_prologue_any_scale(pkg, scale):
    """Attention outputs (V) at any magnitude through the merge prologue."""
    glue = __import__("importlib").import_module("artifex-assistantv5_amd.glue")
    nh, nkv, hd, max_seq, p = 32, 8, 128, 256, 200
    k, n = nh * hd, 512
    w = pkg.repack_gguf_for_gpu(12, pkg.quantize.quantize(
        pkg.quantize.synthetic_weight(n, k, seed=3), 12), n, k)
    g = torch.Generator(device="cuda").manual_seed(p)
    qkv = torch.randn((nh + 2 * nkv) * hd, device="cuda", generator=g)
    qkv[(nh + nkv) * hd:] *= scale
    kc = torch.randn(nkv, max_seq, hd, device="cuda", generator=g)
    vc = torch.randn(nkv, max_seq, hd, device="cuda", generator=g) * scale
    half = hd // 2
    inv = 1.0 / (10000.0 ** (torch.arange(half, dtype=torch.float64) * 2 / hd))
    ang = torch.arange(max_seq, dtype=torch.float64)[:, None] * inv[None]
    cos, sin = ang.cos().float().cuda(), ang.sin().float().cuda()
    pos = torch.tensor([p], device="cuda")
    work = glue.attention_workspace(nh, nkv, hd, max_seq, "cuda")
    a = torch.empty(k, device="cuda")
    glue.attention_decode(qkv, pos, cos, sin, kc.clone(), vc.clone(), a, nh, nkv, hd, work)
    glue.attention_decode(qkv, pos, cos, sin, kc, vc, None, nh, nkv, hd, work)
    y = torch.empty(n, device="cuda")
    glue.matmul_attn_merge(work, pos, w, y, nh, nkv, hd, max_seq)
    y_ref = torch.empty(n, device="cuda")
    glue.matmul_fused(a, w, y_ref)
    assert torch.equal(y, y_ref)
    wd = w.dequant().double()
    assert torch.isfinite(y).all()
    assert _elementwise(y, wd @ a.double(), wd, a.double()) < 1e-6
