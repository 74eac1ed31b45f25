"""GPU: the grid-codebook IQ types (IQ2_XXS, IQ2_XS, IQ2_S, IQ3_XXS, IQ3_S, IQ1_M).

* repack into the row-tile layout (byte-exact against the numpy tile model),
  tile dequant, raw dequant and the row gather: bit-exact to the oracle, whose
  dequant is pinned to the reference's IQ parity fixture
  (webgpu/tests/fixtures/iq_parity_fixture.json, tests/test_oracle_iq.py);
* the decode matmul for M = 1 .. 40 (two passes of at most 32 rows above 32),
  f32 and f16 activations: per element |y - y_ref| <= 2e-5 sum_k |x_k w_nk|
  against the f64 product of the oracle's dequantized weights (the same
  f32-grade gate as the other types' decode path);
* the GEMM (M > 32): the gate of the other types' fp16 GEMM;
* the API contract: no workspace needed up to K = 16384 (the one-shot kernel,
  once per row without one), a workspace required beyond it.
"""

import ctypes

import numpy as np
import pytest
import torch

import tile_model

pytestmark = pytest.mark.gpu

GRID = (16, 17, 22, 18, 21, 29)
NAMES = {16: "IQ2_XXS", 17: "IQ2_XS", 22: "IQ2_S", 18: "IQ3_XXS", 21: "IQ3_S", 29: "IQ1_M"}
DECODE_TOL = 2e-5
DECODE, GEMM, AUTO = 1, 2, 0


@pytest.fixture(scope="module")
def native(pkg):
    from importlib import import_module
    return import_module("artifex-assistantv5_amd._native")


def _weight(pkg, t, n, k, seed):
    raw = tile_model.random_blocks(t, n, k, seed=seed)
    return raw, pkg.repack_gguf_for_gpu(t, raw, n, k)


@pytest.mark.parametrize("t", GRID)
@pytest.mark.parametrize("specials", [False, True])
def test_repack_layout_and_dequant_bit_exact(pkg, ref, t, specials):
    for i, (n, k) in enumerate([(1, 256), (3, 512), (17, 4096), (2, 14336)]):
        raw = tile_model.random_blocks(t, n, k, seed=41 * t + i, specials=specials)
        w = pkg.repack_gguf_for_gpu(t, raw, n, k)
        assert np.array_equal(w.data.cpu().numpy(), tile_model.to_tiles(t, raw, n, k)), (n, k)
        want = ref.dequant_rows(t, raw, n, k)
        assert ref.same_bits(w.dequant().cpu().numpy(), want), (NAMES[t], n, k, "tiles")
        got = pkg.dequant_raw(t, raw, n * k).cpu().numpy()
        assert ref.same_bits(got, want.reshape(-1)), (NAMES[t], n, k, "raw")


@pytest.mark.parametrize("t", GRID)
def test_get_rows_bit_exact(pkg, ref, t):
    n, k = 37, 512
    raw = tile_model.random_blocks(t, n, k, seed=7 * t)
    table = pkg.QuantEmbedding(torch.from_numpy(raw).cuda(), t, n, k)
    ids = torch.tensor([0, 36, 5, 5, 17], dtype=torch.int64, device="cuda")
    got = table.gather(ids).cpu().numpy()
    want = ref.dequant_rows(t, raw, n, k)[[0, 36, 5, 5, 17]]
    assert ref.same_bits(got, want)


@pytest.mark.parametrize("t", GRID)
@pytest.mark.parametrize("xdt", ["f32", "f16"])
def test_decode_matmul_f32_grade(pkg, ref, t, xdt):
    shapes = [(1, 1, 256), (1, 300, 1024), (4, 37, 512), (8, 64, 768), (17, 40, 512),
              (32, 130, 1280), (40, 33, 512), (1, 48, 14336), (32, 16, 14336)]
    for i, (m, n, k) in enumerate(shapes):
        raw, w = _weight(pkg, t, n, k, seed=300 * t + i)
        wdeq = ref.dequant_rows(t, raw, n, k)
        x = pkg.quantize.synthetic_activations(m, k, seed=800 + i,
                                               dtype=np.float32 if xdt == "f32" else np.float16)
        y = pkg.qlinear(torch.from_numpy(x).cuda(), w, variant=DECODE).cpu().numpy()
        x64 = x.astype(np.float64)
        met = ref.parity_metrics(y, ref.matmul_bt(x64, wdeq), ref.matmul_bt_abs(x64, wdeq))
        assert met["finite"] and met["elemwise"] <= DECODE_TOL, ((NAMES[t], xdt, m, n, k), met)


@pytest.mark.parametrize("t", GRID)
@pytest.mark.parametrize("m,xdt", [(8, torch.float32), (16, torch.float16), (3, torch.float32)])
def test_decode_full_width(pkg, t, m, xdt):
    """Batched decode at the FFN width (N = 14336, K = 4096; the K ranges'
    sums added by the second launch) against the f64 product of the
    GPU-dequantized weights (pinned to the oracle by the dequant tests), and
    deterministic."""
    n, k = 14336, 4096
    raw, w = _weight(pkg, t, n, k, seed=31 * t + m)
    g = torch.Generator(device="cuda").manual_seed(t * 100 + m)
    x = torch.randn(m, k, device="cuda", generator=g).to(xdt)
    y = pkg.qlinear(x, w, variant=DECODE)
    x64, w64 = x.double(), w.dequant().view(n, k).double()
    err = (y.double() - x64 @ w64.T).abs()
    elem = (err / (x64.abs() @ w64.abs().T)).max().item()
    assert torch.isfinite(y).all() and elem <= DECODE_TOL, (NAMES[t], m, xdt, elem)
    assert torch.equal(pkg.qlinear(x, w, variant=DECODE), y)


@pytest.mark.parametrize("t", GRID)
def test_decode_matmul_wide_range_activations(pkg, ref, t):
    """Activations spanning 2^-60 .. 2^60 across units and rows: every unit is
    scaled by its own power of two before it enters the matrix cores."""
    m, n, k = 5, 48, 1024
    raw, w = _weight(pkg, t, n, k, seed=11 * t)
    rng = np.random.default_rng(t)
    x = rng.standard_normal((m, k)).astype(np.float32)
    x *= np.exp2(rng.integers(-60, 61, size=(m, k // 256, 1))).repeat(256, axis=2).reshape(m, k)
    y = pkg.qlinear(torch.from_numpy(x).cuda(), w).cpu().numpy()
    wdeq = ref.dequant_rows(t, raw, n, k)
    x64 = x.astype(np.float64)
    met = ref.parity_metrics(y, ref.matmul_bt(x64, wdeq), ref.matmul_bt_abs(x64, wdeq))
    assert met["finite"] and met["elemwise"] <= DECODE_TOL, (NAMES[t], met)


def test_api_contract(pkg, native):
    lib = native.load_library()
    t, m, n, k = 16, 3, 32, 512
    raw, w = _weight(pkg, t, n, k, seed=5)
    x = torch.from_numpy(pkg.quantize.synthetic_activations(m, k, seed=6)).cuda()
    y = torch.zeros(m, n, device="cuda")
    # the GEMM variant needs no workspace
    rc = lib.gguf_hip_matmul_variant(x.data_ptr(), 0, k, w.ptr(), t, n, k, y.data_ptr(), n, m,
                                     GEMM, None)
    assert rc == 0, native.last_error(lib)
    # M = 1 needs no workspace; M >= 2 asks for one (the batched kernel) but
    # runs without it too, and a workspace one byte short is taken as none
    assert lib.gguf_hip_matmul_workspace(t, 0, n, k, 1) == 0
    need = lib.gguf_hip_matmul_workspace(t, 0, n, k, m)
    assert need > 0
    ws = torch.zeros(need, dtype=torch.uint8, device="cuda")  # zero-filled
    outs = []
    for work, nb in ((None, 0), (ws.data_ptr(), need - 1), (ws.data_ptr(), need)):
        y.zero_()
        rc = lib.gguf_hip_matmul_ws(x.data_ptr(), 0, k, w.ptr(), t, n, k, y.data_ptr(), n, m,
                                    AUTO, work, nb, None)
        assert rc == 0, native.last_error(lib)
        outs.append(y.cpu().numpy().copy())
    assert np.array_equal(outs[0], outs[1])
    assert np.count_nonzero(ws.cpu().numpy()[:65536]) == 0  # the reserved prefix is never written
    # beyond K = 16384 only the batched kernel serves the grid types: a workspace is required
    kb = 16640
    assert lib.gguf_hip_matmul_workspace(t, 0, n, kb, 1) > 0
    rc = lib.gguf_hip_matmul(x.data_ptr(), 0, kb, w.ptr(), t, n, kb, y.data_ptr(), n, 1, None)
    assert rc == native.ERR_SHAPE and "workspace" in native.last_error(lib)
    torch.cuda.synchronize()
    # the fused decode-step kernel without prologue or epilogue is the plain M = 1 kernel
    rc = lib.gguf_hip_matmul_fused(x.data_ptr(), w.ptr(), t, n, k, y.data_ptr(), 0, None,
                                   ctypes.c_float(0.0), 0, None)
    assert rc == 0, native.last_error(lib)
    z = torch.empty(1, n, device="cuda")
    assert lib.gguf_hip_matmul(x.data_ptr(), 0, k, w.ptr(), t, n, k, z.data_ptr(), n, 1,
                               None) == 0
    torch.cuda.synchronize()
    assert torch.equal(y.view(-1)[:n], z[0])


@pytest.mark.parametrize("t", GRID)
def test_plain_matmul_entry_without_workspace(pkg, ref, native, t):
    """gguf_hip_matmul (dispatchMatmulGGUF's counterpart, forward-pass.ts:1496-1544)
    serves the grid types with no workspace: M = 1, 8 and 32 with f32 activations
    (the decode path: per element within 2e-5 sum_k |x_k w_nk|) and M = 64 with
    f16 activations (AUTO takes the GEMM: its 1e-3 gates), against the oracle."""
    lib = native.load_library()
    n, k = 80, 1024
    raw, w = _weight(pkg, t, n, k, seed=61 * t)
    wdeq = ref.dequant_rows(t, raw, n, k)
    for m, xdt, tol in ((1, np.float32, DECODE_TOL), (8, np.float32, DECODE_TOL),
                        (32, np.float32, DECODE_TOL), (64, np.float16, None)):
        x = pkg.quantize.synthetic_activations(m, k, seed=m + t, dtype=xdt)
        xd = torch.from_numpy(x).cuda()
        y = torch.full((m, n), float("nan"), device="cuda")
        rc = lib.gguf_hip_matmul(xd.data_ptr(), 0 if xdt == np.float32 else 1, k, w.ptr(), t, n,
                                 k, y.data_ptr(), n, m, None)
        assert rc == 0, (NAMES[t], m, native.last_error(lib))
        x64 = x.astype(np.float64)
        met = ref.parity_metrics(y.cpu().numpy(), ref.matmul_bt(x64, wdeq),
                                 ref.matmul_bt_abs(x64, wdeq))
        ok = met["ok"] if tol is None else met["finite"] and met["elemwise"] <= tol
        assert ok, (NAMES[t], m, met)


GEMM_TOL = 1e-3


@pytest.mark.parametrize("t", GRID)
@pytest.mark.parametrize("xdt", ["f16", "f32"])
def test_gemm_matches_oracle(pkg, ref, t, xdt):
    """The MFMA GEMM with fp16 operands (weights rounded once from the exact f32
    dequant value): normwise and elementwise within 1e-3 of the f64 product, as
    for the other types (tests/test_gpu_matmul.py)."""
    for i, (m, n, k) in enumerate([(40, 70, 512), (130, 200, 768), (300, 64, 1024),
                                   (64, 33, 4096)]):
        raw, w = _weight(pkg, t, n, k, seed=900 * t + i)
        wdeq = ref.dequant_rows(t, raw, n, k)
        x = pkg.quantize.synthetic_activations(m, k, seed=40 + i,
                                               dtype=np.float32 if xdt == "f32" else np.float16)
        y = pkg.qlinear(torch.from_numpy(x).cuda(), w, variant=GEMM).cpu().numpy()
        x64 = x.astype(np.float64)
        met = ref.parity_metrics(y, ref.matmul_bt(x64, wdeq), ref.matmul_bt_abs(x64, wdeq))
        assert met["ok"], ((NAMES[t], xdt, m, n, k), met)


@pytest.mark.parametrize("t", GRID)
def test_auto_takes_the_gemm_for_prefill(pkg, ref, t):
    """f16 activations above 32 rows take the GEMM under AUTO, no workspace needed."""
    m, n, k = 96, 48, 512
    raw, w = _weight(pkg, t, n, k, seed=77 * t)
    x = pkg.quantize.synthetic_activations(m, k, seed=3, dtype=np.float16)
    y = pkg.qlinear(torch.from_numpy(x).cuda(), w).cpu().numpy()
    wdeq = ref.dequant_rows(t, raw, n, k)
    x64 = x.astype(np.float64)
    met = ref.parity_metrics(y, ref.matmul_bt(x64, wdeq), ref.matmul_bt_abs(x64, wdeq))
    assert met["ok"], (NAMES[t], met)
