"""Decode-step glue kernels of libgguf_hip (f32 torch tensors on the current HIP stream).

Each function is one launch.  Every buffer's element count is checked against
the launch shape here, before the dtype / device checks and before the C ABI
(which cannot see tensor sizes): a mismatch raises ValueError instead of
reading or writing past a buffer on the device.
Reference shaders: rmsnorm.wgsl:1-9,58-67, rope.wgsl:1-10,
elementwise.wgsl:96-102 (gate_silu), argmax.wgsl; layer loop
webgpu/src/engine/forward-pass.ts:2925-3297.
"""

from __future__ import annotations

import torch

from . import _native


def _s(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _f32(*ts: torch.Tensor) -> None:
    for t in ts:
        if t.dtype != torch.float32 or not t.is_cuda or not t.is_contiguous():
            raise ValueError("glue kernels take contiguous float32 device tensors")


def _numel(what: str, t: torch.Tensor, want: int) -> None:
    if t.numel() != want:
        raise ValueError(f"{what} has {t.numel()} elements, the launch needs {want}")


def rmsnorm(x: torch.Tensor, w: torch.Tensor, eps: float, out: torch.Tensor) -> torch.Tensor:
    """out = x / sqrt(mean(x^2) + eps) * w over the last dimension."""
    n = x.shape[-1]
    _numel("rmsnorm: w", w, n)
    _numel("rmsnorm: out", out, x.numel())
    _f32(x, w, out)
    lib = _native.load_library()
    _native.check(lib.gguf_hip_rmsnorm(x.data_ptr(), w.data_ptr(), eps, out.data_ptr(),
                                       x.numel() // n, n, _s(x)), lib)
    return out


def add_rmsnorm(x: torch.Tensor, res: torch.Tensor, w: torch.Tensor, eps: float,
                out: torch.Tensor) -> torch.Tensor:
    """x += res (in place), then out = rmsnorm(x) * w."""
    n = x.shape[-1]
    _numel("add_rmsnorm: res", res, x.numel())
    _numel("add_rmsnorm: w", w, n)
    _numel("add_rmsnorm: out", out, x.numel())
    _f32(x, res, w, out)
    lib = _native.load_library()
    _native.check(lib.gguf_hip_add_rmsnorm(x.data_ptr(), res.data_ptr(), w.data_ptr(), eps,
                                           out.data_ptr(), x.numel() // n, n, _s(x)), lib)
    return out


def swiglu(gate_up: torch.Tensor, out: torch.Tensor) -> torch.Tensor:
    """out = up * silu(gate) for rows [gate | up]."""
    ffn = out.shape[-1]
    _numel("swiglu: gate_up", gate_up, 2 * out.numel())
    if gate_up.dim() > 1 and gate_up.shape[-1] != 2 * ffn:
        raise ValueError(f"swiglu: gate_up rows hold {gate_up.shape[-1]} values, need {2 * ffn}")
    _f32(gate_up, out)
    lib = _native.load_library()
    _native.check(lib.gguf_hip_swiglu(gate_up.data_ptr(), out.data_ptr(), out.numel() // ffn, ffn,
                                      _s(out)), lib)
    return out


def attention_workspace(n_heads: int, n_kv_heads: int, head_dim: int, max_seq: int,
                        device) -> torch.Tensor:
    """Device workspace for ``attention_decode`` (allocate once, reuse every step).
    Zero-filled: its per-KV-head counters must start at zero (each call leaves
    them at zero)."""
    lib = _native.load_library()
    nbytes = _native.check(lib.gguf_hip_attention_workspace(n_heads, n_kv_heads, head_dim,
                                                            max_seq), lib)
    return torch.zeros((nbytes + 15) // 16 * 4, dtype=torch.float32, device=device)


def _check_attention_work(lib, work: torch.Tensor, n_heads: int, n_kv_heads: int,
                          head_dim: int, max_seq: int) -> None:
    need = _native.check(lib.gguf_hip_attention_workspace(n_heads, n_kv_heads, head_dim,
                                                          max_seq), lib)
    if work.numel() * work.element_size() < need:
        raise ValueError(f"attention workspace holds {work.numel() * work.element_size()} bytes, "
                         f"needs {need}")


def attention_decode(qkv: torch.Tensor, pos: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
                     k_cache: torch.Tensor, v_cache: torch.Tensor, out: torch.Tensor | None,
                     n_heads: int, n_kv_heads: int, head_dim: int,
                     work: torch.Tensor) -> torch.Tensor | None:
    """RoPE + KV append at slot ``pos`` (device int64 [1]) + causal GQA attention.
    ``out=None`` writes only the partial-softmax records into ``work``, for
    ``matmul_attn_merge`` to merge inside the output projection.  Caches are
    ``[n_kv_heads, max_seq, head_dim]``, cos / sin ``[max_seq, head_dim / 2]``."""
    if k_cache.dim() < 2:
        raise ValueError("attention_decode: k_cache must be [n_kv_heads, max_seq, head_dim]")
    max_seq = k_cache.shape[-2]
    if k_cache.shape[-1] != head_dim:
        raise ValueError(f"attention_decode: k_cache rows hold {k_cache.shape[-1]} values, "
                         f"head_dim is {head_dim}")
    _numel("attention_decode: k_cache", k_cache, n_kv_heads * max_seq * head_dim)
    _numel("attention_decode: v_cache", v_cache, n_kv_heads * max_seq * head_dim)
    _numel("attention_decode: qkv", qkv, (n_heads + 2 * n_kv_heads) * head_dim)
    _numel("attention_decode: cos", cos, max_seq * (head_dim // 2))
    _numel("attention_decode: sin", sin, max_seq * (head_dim // 2))
    if out is not None:
        _numel("attention_decode: out", out, n_heads * head_dim)
    if pos.numel() != 1:
        raise ValueError("attention_decode: pos must hold one position")
    _f32(qkv, cos, sin, k_cache, v_cache, *(() if out is None else (out,)))
    if pos.dtype != torch.int64 or not pos.is_cuda:
        raise ValueError("pos must be an int64 device tensor")
    lib = _native.load_library()
    _check_attention_work(lib, work, n_heads, n_kv_heads, head_dim, k_cache.shape[-2])
    _native.check(lib.gguf_hip_attention_decode(
        qkv.data_ptr(), pos.data_ptr(), cos.data_ptr(), sin.data_ptr(), k_cache.data_ptr(),
        v_cache.data_ptr(), None if out is None else out.data_ptr(), n_heads, n_kv_heads,
        head_dim, k_cache.shape[-2], work.data_ptr(), _s(qkv)), lib)
    return out


def attention_prefill(qkv: torch.Tensor, pos: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
                      k_cache: torch.Tensor, v_cache: torch.Tensor, out: torch.Tensor,
                      n_heads: int, n_kv_heads: int, head_dim: int) -> torch.Tensor:
    """RoPE + KV append + causal GQA attention of M rows at once (prefill).
    ``qkv`` [M, >= (n_heads + 2 n_kv_heads) head_dim] and ``out`` [M, >= n_heads
    head_dim] may have a row stride (unit column stride); ``pos`` device int64
    [M] holds distinct positions.  Row r attends over cache slots 0..pos[r]:
    the slots this call does not write must already hold keys.  Two launches."""
    if qkv.dim() != 2 or out.dim() != 2 or qkv.shape[0] != out.shape[0]:
        raise ValueError("attention_prefill: qkv and out must be [M, ...] with the same M")
    m = qkv.shape[0]
    if pos.numel() != m:
        raise ValueError(f"attention_prefill: pos holds {pos.numel()} positions, M = {m}")
    if k_cache.dim() < 2 or k_cache.shape[-1] != head_dim:
        raise ValueError("attention_prefill: k_cache must be [n_kv_heads, max_seq, head_dim]")
    max_seq = k_cache.shape[-2]
    _numel("attention_prefill: k_cache", k_cache, n_kv_heads * max_seq * head_dim)
    _numel("attention_prefill: v_cache", v_cache, n_kv_heads * max_seq * head_dim)
    _numel("attention_prefill: cos", cos, max_seq * (head_dim // 2))
    _numel("attention_prefill: sin", sin, max_seq * (head_dim // 2))
    row, orow = (n_heads + 2 * n_kv_heads) * head_dim, n_heads * head_dim
    if qkv.shape[1] < row or out.shape[1] < orow:
        raise ValueError(f"attention_prefill: qkv rows hold {qkv.shape[1]} values (need {row}), "
                         f"out rows {out.shape[1]} (need {orow})")
    for name, t in (("qkv", qkv), ("out", out)):
        if t.dtype != torch.float32 or not t.is_cuda or (m > 1 and t.stride(1) != 1) \
                or t.stride(0) < t.shape[1]:
            raise ValueError(f"attention_prefill: {name} must be float32 device rows "
                             "with unit column stride")
    _f32(cos, sin, k_cache, v_cache)
    if pos.dtype != torch.int64 or not pos.is_cuda:
        raise ValueError("pos must be an int64 device tensor")
    lib = _native.load_library()
    _native.check(lib.gguf_hip_attention_prefill(
        qkv.data_ptr(), qkv.stride(0), pos.data_ptr(), m, cos.data_ptr(), sin.data_ptr(),
        k_cache.data_ptr(), v_cache.data_ptr(), out.data_ptr(), out.stride(0), n_heads,
        n_kv_heads, head_dim, max_seq, _s(qkv)), lib)
    return out


def matmul_attn_merge(work: torch.Tensor, pos: torch.Tensor, w, y: torch.Tensor, n_heads: int,
                      n_kv_heads: int, head_dim: int, max_seq: int,
                      accumulate: bool = False) -> torch.Tensor:
    """The attention output projection with the merge fused in: ``y = a @ dequant(w)^T``
    (``y +=`` with ``accumulate``), a = the attention output merged from the
    records that ``attention_decode(..., out=None, work=work)`` wrote for ``pos``.
    ``w`` is a GGUFWeight with k = n_heads * head_dim."""
    if pos.numel() != 1:
        raise ValueError("matmul_attn_merge: pos must hold one position")
    _f32(y)
    if pos.dtype != torch.int64 or not pos.is_cuda:
        raise ValueError("pos must be an int64 device tensor")
    if w.k != n_heads * head_dim or y.numel() != w.n:
        raise ValueError(f"matmul_attn_merge: weight {w.n}x{w.k} for {n_heads}x{head_dim} heads, "
                         f"y has {y.numel()} elements")
    lib = _native.load_library()
    _check_attention_work(lib, work, n_heads, n_kv_heads, head_dim, max_seq)
    _native.check(lib.gguf_hip_matmul_attn_merge(
        work.data_ptr(), pos.data_ptr(), n_heads, n_kv_heads, head_dim, max_seq, w.ptr(),
        w.ggml_type, w.n, y.data_ptr(), EPILOGUE_ACCUMULATE if accumulate else EPILOGUE_STORE,
        _s(y)), lib)
    return y


def argmax_workspace(device) -> torch.Tensor:
    lib = _native.load_library()
    return torch.empty(lib.gguf_hip_argmax_workspace() // 8, dtype=torch.int64, device=device)


def argmax(x: torch.Tensor, out: torch.Tensor, work: torch.Tensor) -> torch.Tensor:
    """out[0] = first index of max(x) (int64 device tensor)."""
    if x.numel() == 0 or out.numel() < 1:
        raise ValueError("argmax: x must be non-empty and out must hold one index")
    _f32(x)
    if out.dtype != torch.int64 or not out.is_cuda:
        raise ValueError("argmax output must be an int64 device tensor")
    lib = _native.load_library()
    if work.numel() * work.element_size() < lib.gguf_hip_argmax_workspace():
        raise ValueError("argmax workspace too small")
    _native.check(lib.gguf_hip_argmax(x.data_ptr(), x.numel(), out.data_ptr(), work.data_ptr(),
                                      _s(x)), lib)
    return out


PROLOGUE_NONE, PROLOGUE_RMSNORM, PROLOGUE_SWIGLU = (_native.PROLOGUE_NONE, _native.PROLOGUE_RMSNORM,
                                                    _native.PROLOGUE_SWIGLU)
EPILOGUE_STORE, EPILOGUE_ACCUMULATE, EPILOGUE_SWIGLU = (
    _native.EPILOGUE_STORE, _native.EPILOGUE_ACCUMULATE, _native.EPILOGUE_SWIGLU)


def matmul_fused(x: torch.Tensor, w, y: torch.Tensor, prologue: int = PROLOGUE_NONE,
                 norm_w: torch.Tensor | None = None, eps: float = 0.0,
                 accumulate: bool = False, epilogue: int | None = None) -> torch.Tensor:
    """One activation row through a quantized weight with fused neighbours:
    ``r = x' @ dequant(w)^T`` where x' is x, ``rmsnorm(x) * norm_w`` or, for
    x = [gate | up], ``up * silu(gate)``; then ``y = r``, ``y += r``
    (``accumulate`` / EPILOGUE_ACCUMULATE) or, for a weight of interleaved
    gate / up tiles (``interleave_tiles``), ``y = up * silu(gate)``
    (EPILOGUE_SWIGLU, ``w.n / 2`` outputs).  ``w`` is a GGUFWeight."""
    k = w.k
    epi = epilogue if epilogue is not None else (EPILOGUE_ACCUMULATE if accumulate
                                                 else EPILOGUE_STORE)
    want = 2 * k if prologue == PROLOGUE_SWIGLU else k
    n_out = w.n // 2 if epi == EPILOGUE_SWIGLU else w.n
    if x.numel() != want or y.numel() != n_out:
        raise ValueError(f"matmul_fused: x has {x.numel()} elements (needs {want}), "
                         f"y has {y.numel()} (needs {n_out})")
    if prologue == PROLOGUE_RMSNORM:
        if norm_w is None:
            raise ValueError("matmul_fused: RMSNORM prologue needs norm_w")
        _numel("matmul_fused: norm_w", norm_w, k)
    _f32(x, y, *((norm_w,) if prologue == PROLOGUE_RMSNORM else ()))
    lib = _native.load_library()
    _native.check(lib.gguf_hip_matmul_fused(
        x.data_ptr(), w.ptr(), w.ggml_type, w.n, k, y.data_ptr(), prologue,
        norm_w.data_ptr() if norm_w is not None else None, float(eps), int(epi), _s(y)), lib)
    return y
