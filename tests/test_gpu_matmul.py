"""GPU: dequant-matmul parity against the oracle.

Gate (both must hold; written here and in oracle.gguf_ref.parity_metrics):
    normwise  ||y - y_ref||_2 / ||y_ref||_2            <= 1e-3
    elemwise  max |y - y_ref| / sum_k |x_k * w_nk|      <= 1e-3
y_ref is the f64 product of the oracle's dequantized weights (bit-exact to
gguf-dequant.ts) with the same activations.
"""

import importlib

import numpy as np
import pytest
import torch

import tile_model

pytestmark = pytest.mark.gpu

TOL = 1e-3
DECODE, GEMM, AUTO = 1, 2, 0


def _check(ref, y, x, wdeq, label, normwise=True):
    """Both gates; ``normwise=False`` keeps only the per-element gate (used for
    the fp16-weight GEMM on outputs of fewer than 64 elements, where the
    normwise error of a few cancelling dot products is ill-posed)."""
    x64 = np.asarray(x, np.float64)
    y_ref = ref.matmul_bt(x64, wdeq)
    met = ref.parity_metrics(y, y_ref, ref.matmul_bt_abs(x64, wdeq))
    if normwise:
        assert met["ok"], (label, met)
    else:
        assert met["finite"] and met["elemwise"] <= TOL, (label, met)
    return met


def _case(pkg, t, n, k, seed):
    w = pkg.quantize.synthetic_weight(n, k, seed=seed)
    raw = pkg.quantize.quantize(w, t)
    return raw, pkg.repack_gguf_for_gpu(t, raw, n, k)


SMALL = [(1, 1, 256), (1, 70, 512), (3, 70, 512), (1, 257, 1280), (7, 9, 768), (17, 130, 512),
         (32, 64, 1024), (33, 129, 512), (130, 200, 768)]


@pytest.mark.parametrize("t", [2, 6, 8, 10, 11, 12, 13, 14, 20, 23])
@pytest.mark.parametrize("variant", [DECODE, GEMM, AUTO])
@pytest.mark.parametrize("xdt", ["f32", "f16"])
def test_small_shapes(pkg, ref, t, variant, xdt):
    for i, (m, n, k) in enumerate(SMALL):
        raw, w = _case(pkg, t, n, k, seed=10 * t + i)
        wdeq = ref.dequant_rows(t, raw, n, k)
        x = pkg.quantize.synthetic_activations(m, k, seed=500 + i,
                                               dtype=np.float32 if xdt == "f32" else np.float16)
        xt = torch.from_numpy(x).cuda()
        y = pkg.qlinear(xt, w, variant=variant).cpu().numpy()
        gemm = variant == GEMM or (variant == AUTO and m > 32)
        _check(ref, y, x.astype(np.float32), wdeq, (t, variant, xdt, m, n, k),
               normwise=not gemm or m * n >= 64)


@pytest.mark.parametrize("t", [8, 2, 6, 20])
def test_q8_0_k_not_multiple_of_64(pkg, ref, t):
    for variant in (DECODE, GEMM):
        for m, n, k in [(1, 33, 96), (5, 40, 160), (40, 17, 32)]:
            raw, w = _case(pkg, t, n, k, seed=n + k)
            x = pkg.quantize.synthetic_activations(m, k, seed=k)
            y = pkg.qlinear(torch.from_numpy(x).cuda(), w, variant=variant).cpu().numpy()
            _check(ref, y, x, ref.dequant_rows(t, raw, n, k), (variant, m, n, k))


DECODE_TOL = 2e-5


@pytest.mark.parametrize("t", [2, 6, 8, 10, 11, 12, 13, 14, 20, 23])
def test_decode_is_f32_grade(pkg, ref, t):
    """The decode path feeds exact quant codes and hi/lo-split f32 activations to
    the matrix cores: per element |y - y_ref| <= 2e-5 * sum_k |x_k w_nk| (a
    50x margin inside the 1e-3 gate), for every M it serves, and including a
    single output (N = 1), where cancellation makes normwise error ill-posed."""
    for i, (m, n, k) in enumerate([(1, 1, 256), (1, 300, 1024), (4, 37, 512), (16, 64, 768),
                                   (17, 40, 512), (32, 130, 1280)]):
        raw, w = _case(pkg, t, n, k, seed=900 + i)
        wdeq = ref.dequant_rows(t, raw, n, k)
        x = pkg.quantize.synthetic_activations(m, k, seed=700 + i)
        y = pkg.qlinear(torch.from_numpy(x).cuda(), w, variant=DECODE).cpu().numpy()
        x64 = x.astype(np.float64)
        met = ref.parity_metrics(y, ref.matmul_bt(x64, wdeq), ref.matmul_bt_abs(x64, wdeq))
        assert met["finite"] and met["elemwise"] <= DECODE_TOL, ((t, m, n, k), met)


@pytest.mark.parametrize("t", [14, 8, 12])
@pytest.mark.parametrize("xdt", [np.float32, np.float16])
def test_batched_decode_random_blocks(pkg, ref, t, xdt):
    """The batched decode (M = 2 .. 32) on random blocks: every code and every
    scale value (Q6_K's int8 group scales include -128 and the negative high
    nibbles that the kernel splits off; Q8_0 blocks of one unit carry unrelated
    scales, each block its own activation exponent), with and without a
    workspace, per element within 2e-5 sum_k |x_k w_nk| of the oracle's f64
    product.  K = 4128 (Q8_0: not a multiple of 256) takes the other batched
    kernel."""
    lib = pkg.load_library()
    s = torch.cuda.current_stream().cuda_stream
    x_type = 0 if xdt == np.float32 else 1
    shapes = [(2, 48, 512), (8, 100, 1024), (16, 64, 768), (17, 33, 1280), (32, 130, 2048)]
    if t == 8:
        shapes.append((9, 40, 4128))
    for i, (m, n, k) in enumerate(shapes):
        raw = tile_model.random_blocks(t, n, k, seed=70 * t + i, specials=False)
        rng = np.random.default_rng(i)
        x = rng.standard_normal((m, k)).astype(np.float32)
        if t == 8 and xdt == np.float32:
            # one block per 256 elements holds activations 2^30 larger but all-zero
            # codes: the other blocks carry the whole result, at full precision
            # only if each block has its own exponent
            b0 = i % 8
            raw.reshape(n, k // 32, 34)[:, b0::8, 2:] = 0
            xb = x.reshape(m, k // 32, 32)
            xb[:, b0::8, :] *= 2.0 ** 30
        w = pkg.repack_gguf_for_gpu(t, raw, n, k)
        wdeq = ref.dequant_rows(t, raw, n, k)
        x = x.astype(xdt)
        xd = torch.from_numpy(x).cuda()
        need = lib.gguf_hip_matmul_workspace(t, x_type, n, k, m)
        outs = []
        for use_ws in (True, False):
            work = torch.zeros(max(need, 16), dtype=torch.uint8, device="cuda") if use_ws else None
            y = torch.full((m, n), float("nan"), device="cuda")
            rc = lib.gguf_hip_matmul_ws(xd.data_ptr(), x_type, k, w.ptr(), t, n, k, y.data_ptr(), n,
                                        m, DECODE, work.data_ptr() if use_ws else None,
                                        need if use_ws else 0, s)
            assert rc == 0, lib.gguf_hip_last_error()
            x64 = x.astype(np.float64)
            met = ref.parity_metrics(y.cpu().numpy(), ref.matmul_bt(x64, wdeq),
                                     ref.matmul_bt_abs(x64, wdeq))
            assert met["finite"] and met["elemwise"] <= DECODE_TOL, ((t, xdt, m, n, k, use_ws), met)
            if use_ws:
                assert int(torch.count_nonzero(work[:65536])) == 0
            outs.append(y)


def test_reference_kernel_test_shapes(pkg, ref):
    """kernel-tests.ts:910-927: M=3, N=70, K=512 per type, and N > 65535 (Q8_0, M=1, K=64)."""
    for t in (2, 6, 8, 10, 11, 12, 13, 14, 20, 23):
        raw = tile_model.random_blocks(t, 70, 512, seed=t)
        w = pkg.repack_gguf_for_gpu(t, raw, 70, 512)
        a = (np.random.default_rng(t).random((3, 512), dtype=np.float32) * 0.5 - 0.25)
        y = pkg.qlinear(torch.from_numpy(a).cuda(), w).cpu().numpy()
        _check(ref, y, a, ref.dequant_rows(t, raw, 70, 512), t)
    raw = tile_model.random_blocks(8, 65600, 64, seed=1)
    w = pkg.repack_gguf_for_gpu(8, raw, 65600, 64)
    a = np.random.default_rng(2).random((1, 64), dtype=np.float32) - 0.5
    y = pkg.qlinear(torch.from_numpy(a).cuda(), w).cpu().numpy()
    _check(ref, y, a, ref.dequant_rows(8, raw, 65600, 64), "wide")


def test_no_writes_outside_output(pkg, ref):
    t, m, n, k = 12, 5, 70, 512
    raw, w = _case(pkg, t, n, k, seed=3)
    x = torch.from_numpy(pkg.quantize.synthetic_activations(m, k, seed=4)).cuda()
    for variant in (DECODE, GEMM):
        big = torch.full((m + 2, n + 9), float("nan"), device="cuda")
        out = big[1:1 + m, 3:3 + n]                      # strided window, ldy = n + 9
        pkg.dispatch_matmul_gguf(x, w, out, m, n, k, "win", variant=variant)
        b = big.cpu().numpy()
        assert np.isnan(b[0]).all() and np.isnan(b[-1]).all()
        assert np.isnan(b[:, :3]).all() and np.isnan(b[:, 3 + n:]).all()
        assert np.isfinite(b[1:1 + m, 3:3 + n]).all()


def test_io_offsets_window(pkg, ref):
    t, m, n, k = 14, 2, 33, 512
    raw, w = _case(pkg, t, n, k, seed=9)
    x = pkg.quantize.synthetic_activations(m, k, seed=10)
    a = torch.zeros(64 + m * k, device="cuda")
    a[64:] = torch.from_numpy(x.reshape(-1)).cuda()
    c = torch.zeros(16 + m * n, device="cuda")
    pkg.dispatch_matmul_gguf(a, w, c, m, n, k, "io", io={"aOffset": 256, "cOffset": 64})
    y = c[16:].view(m, n).cpu().numpy()
    _check(ref, y, x, ref.dequant_rows(t, raw, n, k), "io")


def test_projection_and_gate_up_fusion(pkg, ref):
    t, k, ffn = 12, 512, 256
    rg, wg = _case(pkg, t, ffn, k, seed=21)
    ru, wu = _case(pkg, t, ffn, k, seed=22)
    x = torch.from_numpy(pkg.quantize.synthetic_activations(1, k, seed=23)).cuda()
    lw = pkg.LayerWeights(gate_gg=wg, up_gg=wu, gateUp_gg=pkg.concat_rows(wg, wu))
    g = torch.empty(ffn, device="cuda")
    u = torch.empty(ffn, device="cuda")
    gu = torch.empty(2 * ffn, device="cuda")
    pkg.dispatch_projection(x, lw, "gate", g, 1, ffn, k, "gate")
    pkg.dispatch_projection(x, lw, "up", u, 1, ffn, k, "up")
    pkg.dispatch_projection(x, lw, "gateUp", gu, 1, 2 * ffn, k, "gateUp")
    # rows are reduced independently of their neighbours: the fused GEMV is byte-identical
    assert torch.equal(gu, torch.cat([g, u]))
    with pytest.raises(ValueError):
        pkg.dispatch_projection(x, lw, "down", g, 1, ffn, k, "down")


def test_errors_raise_like_reference(pkg):
    raw, w = _case(pkg, 12, 8, 256, seed=1)
    x = torch.zeros(1, 512, device="cuda")
    with pytest.raises(ValueError):
        pkg.qlinear(x, w)
    with pytest.raises(ValueError):
        pkg.dispatch_matmul_gguf(torch.zeros(256, device="cuda"), w, torch.zeros(8, device="cuda"),
                                 1, 8, 512, "bad-k")
    with pytest.raises(ValueError, match="byteLength"):
        pkg.repack_gguf_for_gpu(12, raw[:-1], 8, 256)
    with pytest.raises(NotImplementedError):
        pkg.repack_gguf_for_gpu(3, raw, 8, 256)


def test_deterministic(pkg):
    raw, w = _case(pkg, 12, 4096, 4096, seed=2)
    for m in (1, 8, 100):
        x = torch.from_numpy(pkg.quantize.synthetic_activations(m, 4096, seed=m)).cuda()
        assert torch.equal(pkg.qlinear(x, w), pkg.qlinear(x, w))


@pytest.mark.parametrize("t", [12, 14, 8])
def test_gemm_deterministic(pkg, t):
    """The prefill GEMM gives bit-identical results call after call: f16
    activations at M = 2048 (AUTO: the GEMM), f32 at M = 600 with the GEMM
    variant forced, and a split-K shape (M = 128, N = 512: few output tiles,
    partial sums added by the reduction in split order).  Each is run five
    times, with other launches in between."""
    w14 = _case(pkg, t, 14336, 4096, seed=5)[1]
    w5 = _case(pkg, t, 512, 4096, seed=6)[1]
    cases = [(w14, 2048, np.float16, AUTO), (w14, 600, np.float32, GEMM),
             (w5, 128, np.float16, AUTO)]
    for w, m, xdt, variant in cases:
        x = torch.from_numpy(pkg.quantize.synthetic_activations(m, 4096, seed=m, dtype=xdt)).cuda()
        first = pkg.qlinear(x, w, variant=variant)
        for _ in range(4):
            pkg.qlinear(x[:1].float(), w14)  # another shape in between (decode path)
            assert torch.equal(pkg.qlinear(x, w, variant=variant), first), (t, m, xdt)
        assert torch.isfinite(first).all()


# ---------------------------------------------------------------------------
# full-size configurations (reference product in f64 on the GPU from the
# GPU-dequantized weights, which test_gpu_dequant pins bit-exact to the oracle)
# ---------------------------------------------------------------------------

def _gpu_check(y, x, wdeq, label):
    x64 = x.double()
    w64 = wdeq.double()
    y_ref = x64 @ w64.T
    sa = x64.abs() @ w64.abs().T
    err = (y.double() - y_ref).abs()
    normwise = (torch.linalg.norm(y.double() - y_ref) / torch.linalg.norm(y_ref)).item()
    elem = (err / sa).max().item()
    assert torch.isfinite(y).all()
    assert normwise <= TOL and elem <= TOL, (label, normwise, elem)


FULL = [  # (type, M, N, K, x dtype)
    (8, 1, 4096, 4096, torch.float32),
    (12, 1, 14336, 4096, torch.float32), (12, 8, 14336, 4096, torch.float32),
    (12, 32, 14336, 4096, torch.float32),
    # the batched decode at the FFN width: Q6_K, Q8_0, 16 f16 rows, a ragged N
    (14, 8, 14336, 4096, torch.float32), (8, 8, 14336, 4096, torch.float32),
    (12, 16, 14336, 4096, torch.float16), (12, 5, 14400, 3072, torch.float32),
    (12, 1, 4096, 14336, torch.float32), (12, 8, 4096, 14336, torch.float32),
    (12, 32, 4096, 14336, torch.float32),
    (14, 1, 151936, 4096, torch.float32),
    # the prefill GEMM at every (M, N) of the Q4_K prefill configuration
    (12, 512, 4096, 4096, torch.float16), (12, 512, 14336, 4096, torch.float16),
    (12, 2048, 4096, 4096, torch.float16), (12, 2048, 14336, 4096, torch.float16),
    (12, 8192, 4096, 4096, torch.float16), (12, 8192, 14336, 4096, torch.float16),
    # f32 activations: below 512 rows the decode path, from 512 on the row-scaled GEMM
    (12, 100, 4096, 4096, torch.float32), (12, 512, 4096, 4096, torch.float32),
    (13, 1, 4096, 14336, torch.float32), (13, 8, 1024, 4096, torch.float32),
    (13, 512, 4096, 4096, torch.float16),
    (2, 1, 14336, 4096, torch.float32), (2, 8, 4096, 14336, torch.float32),
    (2, 512, 4096, 4096, torch.float16), (6, 1, 4096, 14336, torch.float32),
    (6, 32, 4096, 4096, torch.float32), (20, 1, 4096, 4096, torch.float32),
    (20, 2048, 4096, 4096, torch.float16),
    (23, 1, 14336, 4096, torch.float32), (23, 8, 4096, 14336, torch.float32),
    (23, 2048, 4096, 4096, torch.float16),
    (10, 1, 14336, 4096, torch.float32), (10, 8, 4096, 14336, torch.float32),
    (10, 32, 4096, 4096, torch.float32), (10, 2048, 4096, 4096, torch.float16),
    (11, 1, 14336, 4096, torch.float32), (11, 8, 4096, 14336, torch.float32),
    (11, 2048, 4096, 4096, torch.float16),
]


@pytest.mark.parametrize("t,m,n,k,xdt", FULL)
def test_full_size_configs(pkg, t, m, n, k, xdt):
    g = torch.Generator(device="cuda").manual_seed(n + k + m)
    if n * k <= 64 << 20:
        wf = torch.randn(n, k, device="cuda", generator=g) * 0.02
        raw = pkg.quantize.quantize(wf.cpu().numpy(), t)
        w = pkg.repack_gguf_for_gpu(t, raw, n, k)
    else:  # LM head: random blocks with finite scales, drawn on the device
        block, size = tile_model.BLOCK[t]
        rawd = torch.randint(0, 256, (n * k // block * size,), dtype=torch.uint8, device="cuda",
                             generator=g)
        blocks = rawd.view(-1, size)
        for o in {8: [0], 12: [0, 2], 13: [0, 2], 14: [208], 2: [0], 6: [0], 20: [0], 23: [0], 10: [80, 82], 11: [108]}[t]:
            v = (torch.rand(blocks.shape[0], device="cuda", generator=g) * 0.003 + 0.0005).half()
            blocks[:, o:o + 2] = v.view(torch.uint8).view(-1, 2)
        w = pkg.repack_gguf_for_gpu(t, rawd, n, k)
    x = torch.randn(m, k, device="cuda", generator=g).to(xdt)
    y = pkg.qlinear(x, w)
    _gpu_check(y, x.float(), w.dequant().view(n, k), (t, m, n, k))


@pytest.mark.parametrize("t,m,n,k", [(12, 1000, 14000, 4096), (12, 777, 29000, 1536),
                                     (12, 2100, 8200, 4096), (8, 1000, 14000, 4096),
                                     (8, 777, 29000, 1536), (8, 2100, 8200, 4096),
                                     (14, 2100, 14000, 1536), (14, 1500, 29000, 1536),
                                     (13, 2100, 14000, 1536), (11, 2100, 14000, 1536),
                                     (10, 1000, 14000, 4096), (23, 1000, 14000, 1536),
                                     (2, 1000, 14000, 4096), (6, 777, 29000, 1536),
                                     (20, 1000, 14000, 1536), (12, 2048, 14000, 1024),
                                     (8, 2000, 14000, 1024)])
def test_wide_gemm_ragged(pkg, t, m, n, k):
    """Every type but the grid-codebook IQ types: prefill with fp16 activations
    on grids large enough for the wide-tile GEMM (192 tiles of 128 x 512; Q6_K,
    Q5_K and Q3_K 512 of 128 x 384):
    rows past M in the last row tile, a last workgroup with fewer weight row
    tiles than the others, N not a multiple of 16 and a K of 6 superblocks,
    against the f64 product of the dequantized weights; a second call gives
    the same bits."""
    g = torch.Generator(device="cuda").manual_seed(m + n + k + t)
    wf = torch.randn(n, k, device="cuda", generator=g) * 0.02
    raw = pkg.quantize.quantize(wf.cpu().numpy(), t)
    w = pkg.repack_gguf_for_gpu(t, raw, n, k)
    x = torch.randn(m, k, device="cuda", generator=g).half()
    y = pkg.qlinear(x, w)
    _gpu_check(y, x.float(), w.dequant().view(n, k), (t, m, n, k))
    assert torch.equal(pkg.qlinear(x, w), y)


@pytest.mark.parametrize("t,m,k", [(12, 1280, 4096), (8, 1280, 4096), (8, 1280, 1568),
                                   (12, 2048, 4096), (8, 2048, 4096), (12, 4096, 1024),
                                   (10, 2048, 4096), (23, 2048, 4096), (2, 2048, 4096),
                                   (6, 2048, 4096), (20, 2048, 4096), (16, 2048, 4096),
                                   (17, 2048, 4096),
                                   (14, 2048, 4096), (13, 2048, 4096), (11, 2048, 4096),
                                   (10, 1280, 4096), (23, 1280, 4096), (2, 1280, 4096),
                                   (6, 1280, 4096), (20, 1280, 4096), (16, 1280, 4096),
                                   (17, 1280, 4096), (21, 2048, 4096), (22, 2048, 4096),
                                   (29, 2048, 4096), (29, 2048, 1536)])
def test_wide_gemm_equals_gemm_kernel_rows(pkg, t, m, k):
    """The wide-tile GEMM (1280 rows: 280 tiles of 128 x 512; Q6_K 2048 rows:
    608 tiles of 128 x 384) and gemm_kernel (a slice of 128 rows: 56 tiles of
    128 x 256, no workspace, so no K split) run each output element's MFMAs in
    the same k order: the same bits, and a second call the same bits again.  A
    Q8_0 K that is not a multiple of 256 keeps gemm_kernel for the whole call.
    Q4_K and Q8_0 at 2048 rows run the wide tile over 8192 columns and its
    three-tile form over the rest (the other four-tile types the wide tile over
    every column); Q4_K at 4096 rows the wide tile over 12288 and gemm_kernel
    over the rest."""
    n = 14336
    if t in (16, 17, 18, 21, 22, 29):  # random valid blocks: every bit pattern decodes
        raw = tile_model.random_blocks(t, n, k, seed=t + k)
        w = pkg.repack_gguf_for_gpu(t, raw, n, k)
    else:
        raw, w = _case(pkg, t, n, k, seed=t + k)
    g = torch.Generator(device="cuda").manual_seed(k)
    x = torch.randn(m, k, device="cuda", generator=g).half()
    lib = pkg.load_library()
    s = torch.cuda.current_stream().cuda_stream

    def gemm(xs):
        y = torch.full((xs.shape[0], n), float("nan"), device="cuda")
        rc = lib.gguf_hip_matmul_variant(xs.data_ptr(), 1, k, w.ptr(), t, n, k, y.data_ptr(), n,
                                         xs.shape[0], GEMM, s)
        assert rc == 0, lib.gguf_hip_last_error()
        return y
    y = gemm(x)
    assert torch.equal(gemm(x), y), "a second call gave other bits"
    for m0 in (0, 640, m - 128):
        assert torch.equal(gemm(x[m0:m0 + 128].contiguous()), y[m0:m0 + 128]), m0


@pytest.mark.parametrize("t,m,n,k", [(12, 1300, 14336, 1024), (14, 2000, 14000, 768),
                                     (8, 1500, 14336, 512), (29, 2000, 14336, 512),
                                     (10, 1100, 14336, 1024), (2, 1100, 14000, 512)])
def test_f32_wide_gemm_stages_rows_exactly(pkg, t, m, n, k):
    """f32 activations with a workspace on a wide-tile grid: a first launch
    writes each row times 2^e (e puts the row's largest magnitude in
    [2^14, 2^15), clamped to [-126, 126]) as an fp16 image, the wide tile
    multiplies it and scales its sums by 2^-e.  The result equals bit for bit
    (a) the fp16 GEMM of that image, computed here from the rows' maxima, times
    2^-e and (b) the call without a workspace (gemm_kernel, which stages the
    same fp16 values in LDS).  Rows of zeros and of magnitudes 1e-30 .. 1e30,
    a row with one large entry, ragged M, ldx > K, and a workspace filled with
    NaN (the padding of the row scales is read, never used)."""
    if t in (16, 17, 18, 21, 22, 29):
        w = pkg.repack_gguf_for_gpu(t, tile_model.random_blocks(t, n, k, seed=t + m), n, k)
    else:
        _, w = _case(pkg, t, n, k, seed=t + m)
    g = torch.Generator(device="cuda").manual_seed(m + k)
    xs = torch.empty(m, k + 64, device="cuda")
    x = xs[:, :k]
    x.copy_(torch.randn(m, k, device="cuda", generator=g))
    x *= 10.0 ** (torch.rand(m, 1, device="cuda", generator=g) * 60 - 30)
    x[3] = 0
    x[5] = 1.0
    x[5, 7] = 3e4
    lib = pkg.load_library()
    s = torch.cuda.current_stream().cuda_stream
    need = lib.gguf_hip_matmul_workspace(t, 0, n, k, m)
    assert need >= 65536 + 4 * (m * k // 2 + m), need
    work = torch.full((need,), 255, dtype=torch.uint8, device="cuda")

    def call(xp, x_type, ldx, ws):
        y = torch.full((m, n), float("nan"), device="cuda")
        rc = lib.gguf_hip_matmul_ws(xp, x_type, ldx, w.ptr(), t, n, k, y.data_ptr(), n, m, GEMM,
                                    ws.data_ptr() if ws is not None else None,
                                    need if ws is not None else 0, s)
        assert rc == 0, lib.gguf_hip_last_error()
        return y

    y = call(xs.data_ptr(), 0, k + 64, work)
    mx = x.abs().amax(1)
    e = (141 - ((mx.view(torch.int32) >> 23) & 0xFF)).clamp(-126, 126)
    up = ((e + 127) << 23).to(torch.int32).view(torch.float32)
    down = ((127 - e) << 23).to(torch.int32).view(torch.float32)
    img = (x * up[:, None]).half().contiguous()
    y16 = call(img.data_ptr(), 1, k, None)
    assert torch.equal(y, y16 * down[:, None])
    assert torch.equal(y, call(xs.data_ptr(), 0, k + 64, None))
    assert torch.isfinite(y).all() and (y[3] == 0).all()


@pytest.mark.parametrize("k", [2048, 4096, 4352, 8192, 12288, 16384, 32768, 33024])
def test_f32_staging_every_row_length(pkg, k):
    """The row-staging launch holds a row of up to 2048 / 4096 / 8192 (256
    threads) or 16384 / 32768 (1024 threads) values in registers and reads
    longer rows twice: at and past each bound, 70 f32 rows through a small
    GEMM grid (gemm_kernel on the image, K split over the workspace after it)
    give the same bits as without a workspace, up to the split's order of
    addition, and as the fp16 GEMM of the image times 2^-e bit for bit."""
    t, m, n = 12, 70, 256
    w = pkg.repack_gguf_for_gpu(t, tile_model.random_blocks(t, n, k, seed=k), n, k)
    g = torch.Generator(device="cuda").manual_seed(k)
    x = torch.randn(m, k, device="cuda", generator=g)
    x *= 10.0 ** (torch.rand(m, 1, device="cuda", generator=g) * 20 - 10)
    lib = pkg.load_library()
    s = torch.cuda.current_stream().cuda_stream
    need = lib.gguf_hip_matmul_workspace(t, 0, n, k, m)
    need16 = lib.gguf_hip_matmul_workspace(t, 1, n, k, m)
    assert need >= 65536 + 4 * (128 + m * k // 2), need
    work = torch.full((need,), 255, dtype=torch.uint8, device="cuda")

    def call(xt, x_type, nbytes):
        y = torch.full((m, n), float("nan"), device="cuda")
        rc = lib.gguf_hip_matmul_ws(xt.data_ptr(), x_type, k, w.ptr(), t, n, k, y.data_ptr(), n, m,
                                    GEMM, work.data_ptr() if nbytes else None, nbytes, s)
        assert rc == 0, lib.gguf_hip_last_error()
        return y

    y = call(x, 0, need)
    mx = x.abs().amax(1)
    e = (141 - ((mx.view(torch.int32) >> 23) & 0xFF)).clamp(-126, 126)
    up = ((e + 127) << 23).to(torch.int32).view(torch.float32)
    down = ((127 - e) << 23).to(torch.int32).view(torch.float32)
    img = (x * up[:, None]).half()
    assert torch.equal(y, call(img, 1, need16) * down[:, None])
    y0 = call(x, 0, 0)
    assert torch.allclose(y, y0, rtol=1e-5, atol=1e-6 * float(y0.abs().max()))


@pytest.mark.parametrize("t,m,n,k", [(12, 8, 14336, 4096), (12, 32, 4096, 14336), (14, 17, 4096, 14336),
                                     (2, 32, 4096, 4096), (8, 5, 1000, 2048), (10, 32, 512, 8192),
                                     (13, 2, 300, 4096)])
def test_batched_split_k_and_whole_k_agree(pkg, ref, t, m, n, k):
    """The batched decode with a workspace (K split over the grid, slices added in
    a fixed order by a second kernel) and without (each workgroup walks all of K)
    both meet the decode gate against the oracle, and each is deterministic."""
    raw, w = _case(pkg, t, n, k, seed=m + n)
    wdeq = ref.dequant_rows(t, raw, n, k)
    x = pkg.quantize.synthetic_activations(m, k, seed=k + m)
    xt = torch.from_numpy(x).cuda()
    lib = pkg.load_library()
    need = lib.gguf_hip_matmul_workspace(t, 0, n, k, m)
    assert need >= 0
    s = torch.cuda.current_stream().cuda_stream
    outs = []
    for use_ws in (True, False):
        y = torch.full((m, n), float("nan"), device="cuda")
        work = torch.zeros(max(need, 16), dtype=torch.uint8, device="cuda") if use_ws else None
        rc = lib.gguf_hip_matmul_ws(xt.data_ptr(), 0, k, w.ptr(), t, n, k, y.data_ptr(), n, m, DECODE,
                                    work.data_ptr() if use_ws else None, need if use_ws else 0, s)
        assert rc == 0, lib.gguf_hip_last_error()
        y2 = torch.empty_like(y)
        lib.gguf_hip_matmul_ws(xt.data_ptr(), 0, k, w.ptr(), t, n, k, y2.data_ptr(), n, m, DECODE,
                               work.data_ptr() if use_ws else None, need if use_ws else 0, s)
        assert torch.equal(y, y2)
        met = _metrics_decode(ref, y.cpu().numpy(), x, wdeq)
        assert met["finite"] and met["elemwise"] <= DECODE_TOL, ((t, m, n, k, use_ws), met)
        outs.append(y)


def _metrics_decode(ref, y, x, wdeq):
    x64 = x.astype(np.float64)
    return ref.parity_metrics(y, ref.matmul_bt(x64, wdeq), ref.matmul_bt_abs(x64, wdeq))


@pytest.mark.parametrize("t,m,n,k", [(12, 200, 300, 4096), (14, 64, 256, 2048), (23, 130, 256, 4096),
                                     (10, 100, 512, 4096), (13, 40, 200, 4096), (11, 96, 64, 8192),
                                     (12, 512, 4096, 4096), (13, 40, 202, 4096)])
@pytest.mark.parametrize("xdt", [np.float16, np.float32])
def test_gemm_split_k(pkg, ref, t, m, n, k, xdt):
    """Grids of fewer than 192 workgroups split K when given the workspace
    (gguf_hip_matmul_workspace), adding the splits' partial sums in split order
    (four outputs per thread when N is a multiple of 4, N = 202 one per thread):
    within the GEMM gate of the oracle, and within f32 rounding of the same
    GEMM without a workspace (one K range)."""
    lib = pkg.load_library()
    raw, w = _case(pkg, t, n, k, seed=t * 7 + m)
    wdeq = ref.dequant_rows(t, raw, n, k)
    x = pkg.quantize.synthetic_activations(m, k, seed=m + k, dtype=xdt)
    xt = torch.from_numpy(x).cuda()
    x_type = 0 if xdt == np.float32 else 1
    need = lib.gguf_hip_matmul_workspace(t, x_type, n, k, m)
    assert need > 0, "this shape should split K"
    work = torch.zeros(need, dtype=torch.uint8, device="cuda")
    y = torch.full((m, n), float("nan"), device="cuda")
    y1 = torch.full((m, n), float("nan"), device="cuda")
    assert lib.gguf_hip_matmul_ws(xt.data_ptr(), x_type, k, w.ptr(), t, n, k, y.data_ptr(), n, m,
                                  GEMM, work.data_ptr(), need, None) == 0
    assert lib.gguf_hip_matmul_variant(xt.data_ptr(), x_type, k, w.ptr(), t, n, k, y1.data_ptr(), n,
                                       m, GEMM, None) == 0
    torch.cuda.synchronize()
    ys, y1s = y.cpu().numpy(), y1.cpu().numpy()
    _check(ref, ys, x.astype(np.float32), wdeq, (t, m, n, k, "split"))
    assert np.abs(ys - y1s).max() <= 1e-5 * np.abs(y1s).max(), (t, m, n, k)


@pytest.mark.parametrize("t,m,n,k,xdt", [(12, 1300, 14336, 1024, torch.float32),
                                         (14, 64, 4096, 14336, torch.float16),
                                         (12, 200, 302, 4096, torch.float32),
                                         (8, 600, 4096, 4096, torch.float32)])
def test_gemm_paths_replay_in_graphs(pkg, t, m, n, k, xdt):
    """The GEMM's launch sequences captured in a HIP graph (the staged f32 rows
    on the wide tile; a K split with the four-wide and the scalar reduction;
    the staged rows with gemm_kernel): three replays, each after eager calls
    of other shapes on the same stream and an output poisoned with NaN, give
    the eager result bit for bit."""
    if t == 14:
        w = pkg.repack_gguf_for_gpu(t, tile_model.random_blocks(t, n, k, seed=5), n, k)
    else:
        _, w = _case(pkg, t, n, k, seed=5)
    g = torch.Generator(device="cuda").manual_seed(m)
    x = torch.randn(m, k, device="cuda", generator=g).to(xdt)
    y_eager = pkg.qlinear(x, w, variant=GEMM)
    out = torch.empty(m, n, device="cuda")
    pkg.qlinear(x, w, out=out, variant=GEMM)  # warm-up outside the capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        pkg.qlinear(x, w, out=out, variant=GEMM)
    other = torch.randn(70, k, device="cuda", generator=g)
    for rep in range(3):
        pkg.qlinear(other, w)  # eager work between the replays
        pkg.qlinear(x[: m // 2 + 1], w)
        out.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, y_eager), rep


@pytest.mark.parametrize("m,k", [(64, 14336), (128, 14336), (100, 4864)])
def test_gemm_split_k_with_uneven_ranges(pkg, m, k):
    """K = 14336 is 56 superblocks: 16 splits round to 14 ranges of 4, and the
    workspace gguf_hip_matmul_workspace sizes for 14 must be enough for the
    launch to split (it once compared it with 16 and ran one K range on 16
    workgroups, 4x slower).  The partial sums land in the workspace past its
    reserved prefix; the result is within f32 rounding of the unsplit call."""
    t, n = 14, 4096
    lib = pkg.load_library()
    w = pkg.repack_gguf_for_gpu(t, tile_model.random_blocks(t, n, k, seed=m), n, k)
    x = torch.randn(m, k, device="cuda").half()
    need = lib.gguf_hip_matmul_workspace(t, 1, n, k, m)
    work = torch.full((need,), 255, dtype=torch.uint8, device="cuda")
    y = torch.full((m, n), float("nan"), device="cuda")
    y1 = torch.full((m, n), float("nan"), device="cuda")
    assert lib.gguf_hip_matmul_ws(x.data_ptr(), 1, k, w.ptr(), t, n, k, y.data_ptr(), n, m, GEMM,
                                  work.data_ptr(), need, None) == 0
    assert lib.gguf_hip_matmul_variant(x.data_ptr(), 1, k, w.ptr(), t, n, k, y1.data_ptr(), n, m,
                                       GEMM, None) == 0
    torch.cuda.synchronize()
    assert bool((work[:65536] == 255).all())
    assert int((work[65536:65536 + 4 * m * n] != 255).sum()) > 0, "the call did not split K"
    assert torch.isfinite(y).all()
    assert float((y - y1).abs().max()) <= 1e-5 * float(y1.abs().max())


@pytest.mark.gpu
def test_shared_workspace_prefix_stays_zero(pkg, ref):
    """One workspace serves, in turn, the batched decode with K split over the
    grid (the K ranges' partial sums added in range order by a second
    launch), the split-K GEMM and the other types' split decode; up to 16 f32
    rows the batched decode converts the activations in every workgroup, 32
    f32 rows go through the prep launch.  The reserved 64 KB prefix reads zero
    after every call, and each call repeats its first result exactly."""
    lib = pkg.load_library()
    cases = [(12, 8, 4096, 4096, 0, DECODE), (12, 3, 1024, 2048, 1, DECODE),
             (12, 512, 4096, 4096, 1, GEMM), (14, 8, 512, 4096, 0, DECODE),
             (12, 16, 2048, 14336, 0, DECODE), (12, 32, 4096, 4096, 1, DECODE),
             (12, 32, 1024, 4096, 0, DECODE)]
    need = max(lib.gguf_hip_matmul_workspace(t, xt_, n, k, m) for t, m, n, k, xt_, _ in cases)
    work = torch.zeros(need, dtype=torch.uint8, device="cuda")
    s = torch.cuda.current_stream().cuda_stream
    runs = []
    for t, m, n, k, x_type, var in cases:
        raw, w = _case(pkg, t, n, k, seed=t + m)
        x = pkg.quantize.synthetic_activations(m, k, seed=m + n,
                                               dtype=np.float16 if x_type else np.float32)
        runs.append((t, m, n, k, x_type, var, w, torch.from_numpy(x).cuda(), raw, x))
    first = []
    for rep in range(2):
        for i, (t, m, n, k, x_type, var, w, xt, raw, x) in enumerate(runs):
            y = torch.full((m, n), float("nan"), device="cuda")
            rc = lib.gguf_hip_matmul_ws(xt.data_ptr(), x_type, k, w.ptr(), t, n, k, y.data_ptr(), n,
                                        m, var, work.data_ptr(), need, s)
            assert rc == 0, lib.gguf_hip_last_error()
            torch.cuda.synchronize()
            assert int(work[:65536].count_nonzero()) == 0, ("reserved prefix", t, m, n, k)
            if rep == 0:
                first.append(y)
                if var == DECODE and x_type == 0:
                    wdeq = ref.dequant_rows(t, raw, n, k)
                    met = _metrics_decode(ref, y.cpu().numpy(), x, wdeq)
                    assert met["finite"] and met["elemwise"] <= DECODE_TOL, ((t, m, n, k), met)
            else:
                assert torch.equal(y, first[i]), ("repeat", t, m, n, k)


def test_workspace_per_stream(pkg):
    """Batched decode (Q4_K, M = 8, K = 14336: split K, the K ranges' partial
    sums in the workspace) alternating between two streams of one device:
    each stream gets its own workspace and the results equal the
    single-stream ones bit for bit."""
    lin = importlib.import_module("artifex-assistantv5_amd.linear")
    raw, w = _case(pkg, 12, 4096, 14336, seed=9)
    xs = [torch.from_numpy(pkg.quantize.synthetic_activations(8, 14336, seed=s)).cuda()
          for s in range(4)]
    want = [pkg.qlinear(x, w) for x in xs]
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    outs = []
    for rep in range(3):
        for i, x in enumerate(xs):
            s = streams[i % 2]
            s.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(s):
                outs.append((i, pkg.qlinear(x, w)))
    torch.cuda.synchronize()
    for i, y in outs:
        assert torch.equal(y, want[i]), i
    keys = [lin.workspace_key(torch.cuda.current_device(), s.cuda_stream, False) for s in streams]
    wss = [lin._WORKSPACES[k] for k in keys]
    assert wss[0].data_ptr() != wss[1].data_ptr()
    for ws in wss:
        assert int(torch.count_nonzero(ws[:65536])) == 0
