"""Decode glue kernels (libgguf_hip) against torch float32 / float64 references."""
import ctypes
import importlib
import math

import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def lib():
    return importlib.import_module("artifex-assistantv5_amd._native").load_library()


def _s():
    return torch.cuda.current_stream().cuda_stream


def _ok(lib, rc):
    assert rc == 0, importlib.import_module("artifex-assistantv5_amd._native").last_error(lib)


@pytest.mark.parametrize("rows,n", [(1, 4096), (3, 256), (2, 14336)])
def test_rmsnorm_and_add_rmsnorm(lib, rows, n):
    g = torch.Generator(device="cuda").manual_seed(n + rows)
    x = torch.randn(rows, n, device="cuda", generator=g) * 3
    r = torch.randn(rows, n, device="cuda", generator=g)
    w = 1 + 0.1 * torch.randn(n, device="cuda", generator=g)
    y = torch.empty_like(x)
    _ok(lib, lib.gguf_hip_rmsnorm(x.data_ptr(), w.data_ptr(), 1e-6, y.data_ptr(), rows, n, _s()))
    xd = x.double()
    ref = xd / torch.sqrt((xd * xd).mean(-1, keepdim=True) + 1e-6) * w.double()
    assert torch.allclose(y.double(), ref, rtol=2e-6, atol=1e-6)
    x2 = x.clone()
    _ok(lib, lib.gguf_hip_add_rmsnorm(x2.data_ptr(), r.data_ptr(), w.data_ptr(), 1e-6, y.data_ptr(),
                                      rows, n, _s()))
    assert torch.equal(x2, x + r)                    # the residual add is one f32 add
    s = (x + r).double()
    ref = s / torch.sqrt((s * s).mean(-1, keepdim=True) + 1e-6) * w.double()
    assert torch.allclose(y.double(), ref, rtol=2e-6, atol=1e-6)


def test_swiglu(lib):
    ffn = 14336
    gu = torch.randn(2, 2 * ffn, device="cuda") * 4
    out = torch.empty(2, ffn, device="cuda")
    _ok(lib, lib.gguf_hip_swiglu(gu.data_ptr(), out.data_ptr(), 2, ffn, _s()))
    g, u = gu[:, :ffn].double(), gu[:, ffn:].double()
    assert torch.allclose(out.double(), u * g / (1 + torch.exp(-g)), rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("nh,nkv,hd,max_seq,p", [(32, 8, 128, 512, 0), (32, 8, 128, 512, 137),
                                                  (32, 8, 128, 512, 511), (4, 2, 64, 64, 63),
                                                  (8, 8, 64, 128, 64), (16, 2, 256, 200, 130)])
def test_attention_decode(lib, nh, nkv, hd, max_seq, p):
    g = torch.Generator(device="cuda").manual_seed(p + nh)
    qkv = torch.randn((nh + 2 * nkv) * hd, device="cuda", generator=g)
    kc = torch.randn(nkv, max_seq, hd, device="cuda", generator=g)
    vc = torch.randn(nkv, max_seq, hd, device="cuda", generator=g)
    kc0, vc0 = kc.clone(), vc.clone()
    half = hd // 2
    inv = 1.0 / (10000.0 ** (torch.arange(half, dtype=torch.float64) * 2 / hd))
    ang = torch.arange(max_seq, dtype=torch.float64)[:, None] * inv[None]
    cos, sin = ang.cos().float().cuda(), ang.sin().float().cuda()
    pos = torch.tensor([p], device="cuda")
    out = torch.empty(nh * hd, device="cuda")
    nbytes = lib.gguf_hip_attention_workspace(nh, nkv, hd, max_seq)
    work = torch.full(((nbytes + 3) // 4,), float("nan"), device="cuda")  # stale records
    ctr = (nkv * 4 + 15) // 16 * 4           # counter words at the end, zero before first use
    work.view(torch.int32)[-ctr:] = 0

    def run(out_):
        _ok(lib, lib.gguf_hip_attention_decode(qkv.data_ptr(), pos.data_ptr(), cos.data_ptr(),
                                               sin.data_ptr(), kc.data_ptr(), vc.data_ptr(),
                                               out_.data_ptr(), nh, nkv, hd, max_seq,
                                               work.data_ptr(), _s()))
    run(out)
    assert not work.view(torch.int32)[-ctr:].any()        # every call leaves them at zero
    # float64 reference: complex-rotation RoPE, explicit softmax
    th = torch.tensor(float(p), dtype=torch.float64) * inv
    rot = lambda v: torch.view_as_real(  # noqa: E731
        torch.complex(v[..., :half], v[..., half:]) * torch.exp(1j * th.cuda())).transpose(-1, -2).reshape(v.shape)
    q = rot(qkv[:nh * hd].double().view(nh, hd))
    k = rot(qkv[nh * hd:(nh + nkv) * hd].double().view(nkv, hd))
    v = qkv[(nh + nkv) * hd:].double().view(nkv, hd)
    K, V = kc0.double().clone(), vc0.double().clone()
    K[:, p], V[:, p] = k, v
    assert torch.allclose(kc[:, p].double(), k, rtol=1e-5, atol=1e-6)   # cache slot p written
    assert torch.equal(vc[:, p], qkv[(nh + nkv) * hd:].view(nkv, hd))
    others = [t for t in range(max_seq) if t != p]
    assert torch.equal(kc[:, others], kc0[:, others]) and torch.equal(vc[:, others], vc0[:, others])
    ref = torch.empty(nh, hd, dtype=torch.float64, device="cuda")
    for h in range(nh):
        kv = h // (nh // nkv)
        s = K[kv, :p + 1] @ q[h] / math.sqrt(hd)
        e = torch.exp(s - s.max())
        ref[h] = (e / e.sum()) @ V[kv, :p + 1]
    assert torch.allclose(out.double().view(nh, hd), ref, rtol=1e-4, atol=2e-5)
    # a second call on the same workspace (slot p rewritten with the same k / v) is identical
    out2 = torch.empty_like(out)
    run(out2)
    assert torch.equal(out, out2) and not work.view(torch.int32)[-ctr:].any()


def test_argmax_first_index_and_ties(lib):
    out = torch.empty(1, dtype=torch.long, device="cuda")
    work = torch.empty(lib.gguf_hip_argmax_workspace() // 8, dtype=torch.long, device="cuda")
    x = torch.randn(151936, device="cuda")
    _ok(lib, lib.gguf_hip_argmax(x.data_ptr(), x.numel(), out.data_ptr(), work.data_ptr(), _s()))
    assert out.item() == torch.argmax(x).item()
    x[[7, 90000, 151935]] = 100.0                    # ties: the first index wins
    _ok(lib, lib.gguf_hip_argmax(x.data_ptr(), x.numel(), out.data_ptr(), work.data_ptr(), _s()))
    assert out.item() == 7
    y = torch.full((5,), float("-inf"), device="cuda")
    _ok(lib, lib.gguf_hip_argmax(y.data_ptr(), 5, out.data_ptr(), work.data_ptr(), _s()))
    assert out.item() == 0
    z = torch.tensor([1.0, float("nan"), 3.0, 2.0], device="cuda")
    _ok(lib, lib.gguf_hip_argmax(z.data_ptr(), 4, out.data_ptr(), work.data_ptr(), _s()))
    assert out.item() == 2                           # NaN never wins
    x[151935] = 1000.0                               # maximum in the last workgroup's chunk
    _ok(lib, lib.gguf_hip_argmax(x.data_ptr(), x.numel(), out.data_ptr(), work.data_ptr(), _s()))
    assert out.item() == 151935


def _rope_inv(hd, max_seq):
    half = hd // 2
    inv = 1.0 / (10000.0 ** (torch.arange(half, dtype=torch.float64) * 2 / hd))
    ang = torch.arange(max_seq, dtype=torch.float64)[:, None] * inv[None]
    return inv.cuda(), ang.cos().float().cuda(), ang.sin().float().cuda()


@pytest.mark.parametrize("nh,nkv,hd,max_seq,m,pos0,order", [
    (32, 8, 128, 512, 128, 0, "seq"),     # the decoder's 128-token prompt
    (32, 8, 128, 512, 248, 128, "seq"),   # a second prefill over 128 cached slots
    (4, 2, 64, 64, 17, 0, "seq"),         # a ragged block of rows
    (8, 8, 64, 128, 1, 100, "seq"),       # one row, one query head per KV head
    (12, 4, 128, 96, 40, 20, "perm"),     # groups of 3 (an idle wave), rows out of order
    (16, 2, 256, 200, 70, 130, "seq"),    # head_dim 256, groups of 8 (two passes), last slot
    (32, 8, 128, 300, 50, 7, "bad"),      # rows at positions -1 and max_seq
])
def test_attention_prefill(lib, nh, nkv, hd, max_seq, m, pos0, order):
    """RoPE, KV append and causal GQA attention of m rows against float64:
    RoPE as a complex rotation, attention as an explicit masked softmax over the
    whole cache (slots below the call's rows hold earlier keys)."""
    g = torch.Generator(device="cuda").manual_seed(m + pos0 + hd)
    row, orow, grp, half = (nh + 2 * nkv) * hd, nh * hd, nh // nkv, hd // 2
    qkv = torch.randn(m, row + 8, device="cuda", generator=g)[:, :row]   # row stride > row
    kc = torch.randn(nkv, max_seq, hd, device="cuda", generator=g)
    vc = torch.randn(nkv, max_seq, hd, device="cuda", generator=g)
    kc0, vc0 = kc.clone(), vc.clone()
    inv, cos, sin = _rope_inv(hd, max_seq)
    p = torch.arange(pos0, pos0 + m)
    if order == "perm":
        p = p[torch.randperm(m, generator=torch.Generator().manual_seed(1))]
    if order == "bad":
        p[3], p[m - 2] = -1, max_seq
    pos = p.cuda()
    obuf = torch.full((m, orow + 4), float("nan"), device="cuda")
    out = obuf[:, :orow]

    def run(o):
        _ok(lib, lib.gguf_hip_attention_prefill(qkv.data_ptr(), qkv.stride(0), pos.data_ptr(), m,
                                                cos.data_ptr(), sin.data_ptr(), kc.data_ptr(),
                                                vc.data_ptr(), o.data_ptr(), o.stride(0), nh, nkv,
                                                hd, max_seq, _s()))
    run(out)
    valid = (p >= 0) & (p < max_seq)
    vr = valid.nonzero().flatten().tolist()
    pv = p[valid].tolist()
    th = p.clamp(0, max_seq - 1).cuda().double()[:, None, None] * inv   # [m, 1, half]

    def rot(x):
        z = torch.complex(x[..., :half], x[..., half:]) * torch.exp(1j * th)
        return torch.cat([z.real, z.imag], dim=-1)
    q = rot(qkv[:, :orow].double().view(m, nh, hd))
    k = rot(qkv[:, orow:orow + nkv * hd].double().view(m, nkv, hd))
    v = qkv[:, orow + nkv * hd:].double().view(m, nkv, hd)
    K, V = kc0.double().clone(), vc0.double().clone()
    K[:, pv], V[:, pv] = k[vr].transpose(0, 1), v[vr].transpose(0, 1)
    # the caches: the valid rows' slots written (v copied as is), every other slot untouched
    assert torch.allclose(kc[:, pv].double(), K[:, pv], rtol=1e-5, atol=1e-6)
    assert torch.equal(vc[:, pv], qkv[vr, orow + nkv * hd:].view(-1, nkv, hd).transpose(0, 1))
    others = [t for t in range(max_seq) if t not in set(pv)]
    assert torch.equal(kc[:, others], kc0[:, others]) and torch.equal(vc[:, others], vc0[:, others])
    # attention of the valid rows
    T = torch.arange(max_seq, device="cuda")
    masked = T[None, :] > p.cuda()[:, None]                               # [m, max_seq]
    ref = torch.empty(m, nh, hd, dtype=torch.float64, device="cuda")
    for h in range(nh):
        s = (q[:, h] @ K[h // grp].T) / math.sqrt(hd)
        s = s.masked_fill(masked, float("-inf"))
        e = torch.exp(s - s.max(dim=1, keepdim=True).values)
        ref[:, h] = (e / e.sum(dim=1, keepdim=True)) @ V[h // grp]
    got = out.double().view(m, nh, hd)
    assert torch.allclose(got[vr], ref[vr], rtol=1e-4, atol=2e-5)
    bad = [r for r in range(m) if r not in set(vr)]
    assert torch.isnan(out[bad]).all()                 # rows without a slot are not written
    assert torch.isnan(obuf[:, orow:]).all()           # nothing past a row
    # a second call (the same slots rewritten with the same k / v) is bit-identical
    out2 = torch.full_like(out, float("nan"))
    run(out2)
    assert torch.equal(out[vr], out2[vr])
