"""GPU: gguf_hip_attention_decode_noalloc (workspace in the library's own device
array) against gguf_hip_attention_decode with a caller workspace, through the C ABI.

Two calls in a row, the second with a smaller shape (fewer heads, a shorter
cache, another head dim): the outputs and the appended K / V cache slots must be
bit-identical to the workspace entry point's (same kernels, same arithmetic).
"""
import ctypes
import importlib

import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def lib():
    return importlib.import_module("artifex-assistantv5_amd").load_library()


def _inputs(nh, nkv, hd, max_seq, p, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    qkv = torch.randn((nh + 2 * nkv) * hd, device="cuda", generator=g)
    kc = torch.randn(nkv, max_seq, hd, device="cuda", generator=g)
    vc = torch.randn(nkv, max_seq, hd, device="cuda", generator=g)
    half = hd // 2
    inv = 1.0 / (10000.0 ** (torch.arange(half, dtype=torch.float64) * 2 / hd))
    ang = torch.arange(max_seq, dtype=torch.float64)[:, None] * inv[None]
    return qkv, kc, vc, ang.cos().float().cuda(), ang.sin().float().cuda(), torch.tensor([p], device="cuda")


def _run(lib, noalloc, nh, nkv, hd, max_seq, p, seed):
    qkv, kc, vc, cos, sin, pos = _inputs(nh, nkv, hd, max_seq, p, seed)
    out = torch.full((nh * hd,), float("nan"), device="cuda")
    s = torch.cuda.current_stream().cuda_stream
    if noalloc:
        rc = lib.gguf_hip_attention_decode_noalloc(
            qkv.data_ptr(), pos.data_ptr(), cos.data_ptr(), sin.data_ptr(), kc.data_ptr(),
            vc.data_ptr(), out.data_ptr(), nh, nkv, hd, max_seq, s)
    else:
        nbytes = lib.gguf_hip_attention_workspace(nh, nkv, hd, max_seq)
        work = torch.zeros((nbytes + 15) // 16 * 4, device="cuda")
        rc = lib.gguf_hip_attention_decode(
            qkv.data_ptr(), pos.data_ptr(), cos.data_ptr(), sin.data_ptr(), kc.data_ptr(),
            vc.data_ptr(), out.data_ptr(), nh, nkv, hd, max_seq, work.data_ptr(), s)
    assert rc == 0, lib.gguf_hip_last_error()
    torch.cuda.synchronize()
    return out, kc, vc


@pytest.mark.parametrize("shapes", [
    [(32, 8, 128, 1200, 700), (8, 2, 64, 300, 100)],
    [(32, 8, 128, 640, 63), (16, 2, 256, 200, 130)],
])
def test_noalloc_matches_workspace_entry(lib, shapes):
    for i, (nh, nkv, hd, max_seq, p) in enumerate(shapes):
        a = _run(lib, True, nh, nkv, hd, max_seq, p, seed=7 + i)
        b = _run(lib, False, nh, nkv, hd, max_seq, p, seed=7 + i)
        assert torch.isfinite(a[0]).all()
        for x, y in zip(a, b):
            assert torch.equal(x, y), (i, nh, nkv, hd, max_seq, p)


def test_noalloc_rejects_oversized_workspace(lib):
    # 8 KV heads x 8 queries each x 65536 slots of 132-float records: beyond the library's array
    rc = lib.gguf_hip_attention_decode_noalloc(
        ctypes.c_void_p(16), ctypes.c_void_p(16), ctypes.c_void_p(16), ctypes.c_void_p(16),
        ctypes.c_void_p(16), ctypes.c_void_p(16), ctypes.c_void_p(16), 64, 8, 128, 65536, None)
    assert rc == -2 and b"noalloc" in lib.gguf_hip_last_error()
