"""Llama-style decoder whose every projection is a quantized GGUF matmul.

This is the caller of the dequant-matmul path in the reference's engine: the
per-layer loop of webgpu/src/engine/forward-pass.ts:2925-3297 (input RMSNorm,
Q/K/V projections, rotate_half RoPE, GQA causal attention over a KV cache,
output projection and residual, FFN RMSNorm, gate+up projection, gate_silu,
down projection and residual), the final norm and LM head
(forward-pass.ts:3642-3644), and greedy argmax sampling.

Glue semantics follow the reference's shaders:
* RMSNorm  ``x * 1/sqrt(mean(x^2) + eps) * w``           rmsnorm.wgsl:1-9,58-67
* RoPE     rotate_half pairing of ``i`` with ``i + d/2``,
           ``theta = pos / base^(2i/d)``                  rope.wgsl:1-10
* SwiGLU   ``up * silu(gate)``                            elementwise.wgsl:96-102 (gate_silu)
* tok/s    generated tokens / decode wall time, prefill excluded (generate.ts:1155-1160)

Every projection goes through ``dispatch_matmul_gguf`` (libgguf_hip): Q/K/V are
one row-concatenated weight and gate/up another (the reference's gate+up
fusion, forward-pass.ts:740-791, applied to Q/K/V too; byte-identical to
separate dispatches).  A decode step runs the glue as libgguf_hip kernels
(``glue.py``: the input norms and SwiGLU run as prologues of the projections
that consume them, the residual adds as accumulate epilogues of the output
and down projections, RoPE + KV append + GQA attention as one launch whose
records the output projection merges, argmax) over preallocated buffers: five
launches per layer.  Prefill (many positions at once) runs the glue as
libgguf_hip kernels too: RMSNorm rows, each residual add fused with the
RMSNorm after it, RoPE + KV append + causal GQA attention of all rows
(``glue.attention_prefill``, the reference's attention.wgsl with
new_seq_len > 1), SwiGLU rows.  ``hip_glue=False`` runs the prefill glue as
torch f32 ops instead, and ``fused=False`` does the same for decode steps.
A decode step keeps
the token and position in device tensors, so it can be captured once in a HIP
graph and replayed for every generated token without host synchronization.
"""

from __future__ import annotations

import dataclasses
import math
import time
from typing import Optional, Union

import numpy as np
import torch

from . import glue, quantize
from .ggml import FUSED_TYPES, Q4_K, Q6_K, raw_row_bytes
from .linear import (GGUFWeight, LayerWeights, QuantEmbedding, concat_rows, dispatch_matmul_gguf,
                     interleave_tiles, repack_gguf_for_gpu, split_interleaved)


@dataclasses.dataclass
class DecoderConfig:
    n_layers: int = 32
    d_model: int = 4096
    n_heads: int = 32
    n_kv_heads: int = 8
    head_dim: int = 128
    ffn: int = 14336
    vocab: int = 151936
    rope_base: float = 1_000_000.0
    eps: float = 1e-6
    max_seq: int = 512
    attn_type: int = Q4_K      # q, k, v, o
    gate_up_type: int = Q4_K
    down_type: int = Q6_K
    lm_head_type: int = Q6_K
    rope_freq_factors: Optional[tuple] = None   # per-pair divisors of theta (llama rope_freqs)

    @property
    def qkv_rows(self) -> int:
        return (self.n_heads + 2 * self.n_kv_heads) * self.head_dim

    def weight_bytes_per_token(self) -> int:
        """Quantized weight bytes one decode step streams from HBM."""
        d, f = self.d_model, self.ffn
        per_layer = (self.qkv_rows * raw_row_bytes(self.attn_type, d)
                     + d * raw_row_bytes(self.attn_type, self.n_heads * self.head_dim)
                     + 2 * f * raw_row_bytes(self.gate_up_type, d)
                     + d * raw_row_bytes(self.down_type, f))
        return self.n_layers * per_layer + self.vocab * raw_row_bytes(self.lm_head_type, d)


@dataclasses.dataclass
class DecoderWeights:
    """Per-layer ``LayerWeights`` slots: ``qkv_gg`` (Q, K, V rows concatenated) or,
    when the three have different GGUF types, ``qkv_parts = [q, k, v]``; the FFN
    input as ``gateUpI_gg`` (gate and up tiles interleaved, ``interleave_tiles``:
    the decode step then applies SwiGLU in the projection's epilogue),
    ``gateUp_gg`` (rows concatenated) or ``gateUp_parts = [gate, up]``; ``o_gg``,
    ``down_gg`` and the f32 norms ``attn_norm`` / ``ffn_norm``.  ``embed`` is a
    dense ``[vocab, d_model]`` table or a ``QuantEmbedding`` of raw GGUF rows."""
    layers: list
    final_norm: torch.Tensor
    lm_head_gg: GGUFWeight
    embed: Union[torch.Tensor, QuantEmbedding]

    def weight_bytes_per_token(self) -> int:
        """Quantized bytes one decode step streams (projections and LM head)."""
        def nb(w):
            return w.n * raw_row_bytes(w.ggml_type, w.k)
        total = nb(self.lm_head_gg)
        for lw in self.layers:
            for slot in ("qkv", "gateUp"):
                total += sum(nb(w) for w in parts(lw, slot))
            total += nb(lw.o_gg) + nb(lw.down_gg)
        return total


def all_weights(w: DecoderWeights) -> list:
    """Every quantized projection of the model, the LM head included."""
    out = [w.lm_head_gg]
    for lw in w.layers:
        for slot in ("qkv", "gateUp"):
            out += parts(lw, slot)
        out += [lw.o_gg, lw.down_gg]
    return out


def parts(lw: LayerWeights, slot: str) -> list:
    """The weights of a slot: ``[<slot>_gg]``, ``[<slot>I_gg]`` (tile-interleaved)
    or ``<slot>_parts``."""
    for name in (f"{slot}_gg", f"{slot}I_gg"):
        w = lw.get(name)
        if w is not None:
            return [w]
    return list(lw.get(f"{slot}_parts"))


def _quantized(ggml_type: int, n: int, k: int, seed: int, device) -> GGUFWeight:
    w = quantize.synthetic_weight(n, k, seed=seed)
    return repack_gguf_for_gpu(ggml_type, quantize.quantize(w, ggml_type), n, k, device=device)


def _tiled_rows(ggml_type: int, unique_rows: int, n: int, k: int, seed: int, device) -> GGUFWeight:
    """An ``[n, k]`` weight whose rows repeat a block of ``unique_rows`` quantized rows
    (``unique_rows`` a multiple of 16); every row still has its own bytes in HBM."""
    base = _quantized(ggml_type, unique_rows, k, seed, device)
    reps = -(-n // unique_rows)
    data = base.data[:base.nbytes].repeat(reps)
    full = GGUFWeight(data, ggml_type, reps * unique_rows, k)
    return full.rows(0, n) if full.n != n else full


def synthetic_weights(cfg: DecoderConfig, seed: int = 0, device="cuda",
                      distinct_layers: bool = False,
                      lm_head_unique_rows: Optional[int] = None) -> DecoderWeights:
    """Seeded N(0, 0.02) weights quantized in the configured GGUF types.

    Quantizing 32 layers on the host is slow, so unless ``distinct_layers`` the
    layers share one quantized set of values held in separate device buffers
    (each decode step still streams every layer's own bytes from HBM).  The LM
    head likewise repeats ``lm_head_unique_rows`` quantized rows when given."""
    d, hd = cfg.d_model, cfg.head_dim
    g = torch.Generator(device=device).manual_seed(seed)

    def layer_set(s):
        q = _quantized(cfg.attn_type, cfg.n_heads * hd, d, s + 1, device)
        k = _quantized(cfg.attn_type, cfg.n_kv_heads * hd, d, s + 2, device)
        v = _quantized(cfg.attn_type, cfg.n_kv_heads * hd, d, s + 3, device)
        o = _quantized(cfg.attn_type, d, cfg.n_heads * hd, s + 4, device)
        gate = _quantized(cfg.gate_up_type, cfg.ffn, d, s + 5, device)
        up = _quantized(cfg.gate_up_type, cfg.ffn, d, s + 6, device)
        down = _quantized(cfg.down_type, d, cfg.ffn, s + 7, device)
        return concat_rows(q, k, v), o, interleave_tiles(gate, up), down

    layers = []
    shared = None if distinct_layers else layer_set(seed * 1000)
    for l in range(cfg.n_layers):
        qkv, o, gu, down = layer_set(seed * 1000 + 10 * l) if distinct_layers else shared
        if not distinct_layers:
            qkv, o, gu, down = (GGUFWeight(w.data[w.byte_offset:w.byte_offset + w.nbytes].clone(),
                                           w.ggml_type, w.n, w.k) for w in shared)
        layers.append(LayerWeights(
            qkv_gg=qkv, o_gg=o, gateUpI_gg=gu, down_gg=down,
            attn_norm=1.0 + 0.02 * torch.randn(d, device=device, generator=g),
            ffn_norm=1.0 + 0.02 * torch.randn(d, device=device, generator=g)))
    if lm_head_unique_rows:
        lm = _tiled_rows(cfg.lm_head_type, lm_head_unique_rows, cfg.vocab, d, seed + 99, device)
    else:
        lm = _quantized(cfg.lm_head_type, cfg.vocab, d, seed + 99, device)
    embed = (torch.randn(cfg.vocab, d, device=device, generator=g)).half()
    final_norm = 1.0 + 0.02 * torch.randn(d, device=device, generator=g)
    return DecoderWeights(layers, final_norm, lm, embed)


def rms_norm(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    """rmsnorm.wgsl:58-67 with a direct weight (use_residual_weight = 0)."""
    return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps) * w


def rope_tables(cfg: DecoderConfig, device) -> tuple[torch.Tensor, torch.Tensor]:
    half = cfg.head_dim // 2
    inv = 1.0 / (cfg.rope_base ** (torch.arange(half, dtype=torch.float64) * 2.0 / cfg.head_dim))
    if cfg.rope_freq_factors is not None:
        f = torch.tensor(cfg.rope_freq_factors, dtype=torch.float64)
        if f.numel() != half:
            raise ValueError(f"rope_freq_factors has {f.numel()} entries, head_dim/2 = {half}")
        inv = inv / f
    ang = torch.arange(cfg.max_seq, dtype=torch.float64)[:, None] * inv[None, :]
    return ang.cos().float().to(device), ang.sin().float().to(device)


def apply_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """rotate_half RoPE (rope.wgsl:1-10): x [M, H, D], cos/sin [M, D/2]."""
    half = x.shape[-1] // 2
    x1, x2 = x[..., :half], x[..., half:]
    c, s = cos[:, None, :], sin[:, None, :]
    return torch.cat([x1 * c - x2 * s, x2 * c + x1 * s], dim=-1)


def glue_shapes(cfg: DecoderConfig) -> bool:
    """Whether the glue kernels take the configuration: head_dim 64, 128 or 256,
    at most 8 query heads per KV head, rows of a multiple of 4 values."""
    return (cfg.head_dim in (64, 128, 256) and cfg.n_heads % cfg.n_kv_heads == 0
            and cfg.n_heads // cfg.n_kv_heads <= 8 and cfg.d_model % 4 == 0
            and cfg.ffn % 4 == 0)


class QuantDecoder:
    """Greedy decoder over ``DecoderWeights`` with an f32 KV cache in HBM."""

    def __init__(self, cfg: DecoderConfig, weights: DecoderWeights, device="cuda",
                 fused: bool = True, hip_glue: bool = True):
        # a weight of a type without fused decode-step kernels runs the step unfused
        grid = any(w.ggml_type not in FUSED_TYPES for w in all_weights(weights))
        self.cfg, self.w, self.device = cfg, weights, torch.device(device)
        self.fused = fused and not grid
        self.hip_glue = hip_glue and glue_shapes(cfg)
        L, kv, T, hd = cfg.n_layers, cfg.n_kv_heads, cfg.max_seq, cfg.head_dim
        self.k_cache = torch.zeros(L, kv, T, hd, device=self.device)
        self.v_cache = torch.zeros(L, kv, T, hd, device=self.device)
        self.cos, self.sin = rope_tables(cfg, self.device)
        self.t_idx = torch.arange(T, device=self.device)
        self._graph = None
        # static buffers of the fused decode step
        e = lambda n: torch.empty(1, n, device=self.device)  # noqa: E731
        d = cfg.d_model
        self.b_x, self.b_h, self.b_qkv = e(d), e(d), e(cfg.qkv_rows)
        self.b_att, self.b_o = e(cfg.n_heads * hd), e(d)
        self.b_gu, self.b_a, self.b_d = e(2 * cfg.ffn), e(cfg.ffn), e(d)
        self.b_logits = e(cfg.vocab)
        self.w_att = glue.attention_workspace(cfg.n_heads, cfg.n_kv_heads, hd, T, self.device)
        self.w_arg = glue.argmax_workspace(self.device)

    # -- one pass of all layers over M tokens at positions ``pos`` (device [M]) --
    def _proj(self, x: torch.Tensor, w: GGUFWeight, label: str) -> torch.Tensor:
        M = x.shape[0]
        y = torch.empty(M, w.n, device=self.device)
        dispatch_matmul_gguf(x, w, y, M, w.n, w.k, label)
        return y

    def _proj_slot(self, x: torch.Tensor, lw: LayerWeights, slot: str, label: str) -> torch.Tensor:
        ws = parts(lw, slot)
        if len(ws) == 1:
            return self._proj(x, ws[0], label)
        return torch.cat([self._proj(x, w, f"{label}{i}") for i, w in enumerate(ws)], dim=1)

    def _gate_up(self, h: torch.Tensor, lw: LayerWeights, label: str):
        """(gate, up) projections of the FFN input ``h``."""
        w = lw.get("gateUpI_gg")
        if w is not None:
            return split_interleaved(self._proj(h, w, label))
        gu = self._proj_slot(h, lw, "gateUp", label)
        return gu[:, :self.cfg.ffn], gu[:, self.cfg.ffn:]

    def _embed(self, tok: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
        e = self.w.embed
        if isinstance(e, QuantEmbedding):
            return e.gather(tok, out)
        x = e.index_select(0, tok).float()
        if out is None:
            return x
        out.copy_(x)
        return out

    def _layers(self, x: torch.Tensor, pos: torch.Tensor) -> torch.Tensor:
        cfg = self.cfg
        M, nh, nkv, hd = x.shape[0], cfg.n_heads, cfg.n_kv_heads, cfg.head_dim
        grp = nh // nkv
        cos, sin = self.cos.index_select(0, pos), self.sin.index_select(0, pos)
        # causal mask over cache slots: query at position p sees slots t <= p
        mask = torch.where(self.t_idx[None, :] <= pos[:, None], 0.0, float("-inf"))  # [M, T]
        mask = mask.repeat_interleave(grp, dim=0)[None]                            # [1, M*grp, T]
        scale = 1.0 / math.sqrt(hd)
        for l, lw in enumerate(self.w.layers):
            h = rms_norm(x, lw.attn_norm, cfg.eps)
            qkv = self._proj_slot(h, lw, "qkv", f"L{l}-qkv")
            q = qkv[:, :nh * hd].view(M, nh, hd)
            k = qkv[:, nh * hd:(nh + nkv) * hd].view(M, nkv, hd)
            v = qkv[:, (nh + nkv) * hd:].view(M, nkv, hd)
            q, k = apply_rope(q, cos, sin), apply_rope(k, cos, sin)
            self.k_cache[l].index_copy_(1, pos, k.transpose(0, 1))
            self.v_cache[l].index_copy_(1, pos, v.transpose(0, 1))
            # GQA: query head h reads KV head h // grp
            qg = q.view(M, nkv, grp, hd).permute(1, 0, 2, 3).reshape(nkv, M * grp, hd)
            s = torch.matmul(qg, self.k_cache[l].transpose(1, 2)) * scale + mask
            o = torch.matmul(torch.softmax(s, dim=-1), self.v_cache[l])           # [nkv, M*grp, hd]
            o = o.view(nkv, M, grp, hd).permute(1, 0, 2, 3).reshape(M, nh * hd)
            x = x + self._proj(o, lw.o_gg, f"L{l}-o")
            h = rms_norm(x, lw.ffn_norm, cfg.eps)
            gate, up = self._gate_up(h, lw, f"L{l}-gateUp")
            a = up * torch.nn.functional.silu(gate)
            x = x + self._proj(a, lw.down_gg, f"L{l}-down")
        return x

    def _layers_glue(self, x: torch.Tensor, pos: torch.Tensor) -> torch.Tensor:
        """All layers over the M rows of ``x`` (updated in place) with the glue as
        libgguf_hip kernels; returns the rows after the final RMSNorm."""
        cfg, layers = self.cfg, self.w.layers
        M = x.shape[0]
        h = torch.empty_like(x)
        att = torch.empty(M, cfg.n_heads * cfg.head_dim, device=self.device)
        a = torch.empty(M, cfg.ffn, device=self.device)
        glue.rmsnorm(x, layers[0].attn_norm, cfg.eps, h)
        for l, lw in enumerate(layers):
            qkv = self._proj_slot(h, lw, "qkv", f"L{l}-qkv")
            glue.attention_prefill(qkv, pos, self.cos, self.sin, self.k_cache[l],
                                   self.v_cache[l], att, cfg.n_heads, cfg.n_kv_heads,
                                   cfg.head_dim)
            glue.add_rmsnorm(x, self._proj(att, lw.o_gg, f"L{l}-o"), lw.ffn_norm, cfg.eps, h)
            w = lw.get("gateUpI_gg")
            if w is not None:  # tile-interleaved gate / up columns -> [gate | up] rows
                gu = torch.cat(split_interleaved(self._proj(h, w, f"L{l}-gateUp")), dim=1)
            else:
                gu = self._proj_slot(h, lw, "gateUp", f"L{l}-gateUp")
            glue.swiglu(gu, a)
            nxt = layers[l + 1].attn_norm if l + 1 < len(layers) else self.w.final_norm
            glue.add_rmsnorm(x, self._proj(a, lw.down_gg, f"L{l}-down"), nxt, cfg.eps, h)
        return h

    def _logits(self, x_last: torch.Tensor) -> torch.Tensor:
        h = rms_norm(x_last, self.w.final_norm, self.cfg.eps)
        return self._proj(h, self.w.lm_head_gg, "lm_head")

    @torch.no_grad()
    def prefill(self, tokens: torch.Tensor, pos0: int = 0) -> torch.Tensor:
        """Run ``tokens`` (device int64 [M]) at positions pos0.. and return the
        last position's logits [1, vocab]."""
        M = tokens.numel()
        if pos0 + M > self.cfg.max_seq:
            raise ValueError(f"sequence of {pos0 + M} exceeds max_seq {self.cfg.max_seq}")
        pos = torch.arange(pos0, pos0 + M, device=self.device)
        x = self._embed(tokens)
        if self.hip_glue:
            h = self._layers_glue(x, pos)
            return self._proj(h[-1:], self.w.lm_head_gg, "lm_head")
        x = self._layers(x, pos)
        return self._logits(x[-1:])

    def _proj_into(self, x: torch.Tensor, w: GGUFWeight, y: torch.Tensor, label: str) -> None:
        dispatch_matmul_gguf(x, w, y, 1, w.n, w.k, label)

    def _step_fused(self, tok: torch.Tensor, pos: torch.Tensor) -> torch.Tensor:
        """Five launches per layer: Q/K/V projection with the input RMSNorm as its
        prologue, attention (partial-softmax records only), output projection
        that merges the records as its prologue and accumulates into the
        residual, gate/up projection with the FFN RMSNorm prologue and the
        SwiGLU epilogue (interleaved gate / up tiles), down projection
        accumulated into the residual.  With concatenated or split gate / up
        weights, SwiGLU runs as the down projection's prologue instead; with
        n_heads * head_dim above 8192 the attention merges its own records."""
        cfg, W = self.cfg, self.w
        x = self.b_x
        merge = cfg.n_heads * cfg.head_dim <= 8192
        self._embed(tok, x)
        for l, lw in enumerate(W.layers):
            self._fused_slot(x, lw, "qkv", self.b_qkv, lw.attn_norm)
            glue.attention_decode(self.b_qkv, pos, self.cos, self.sin, self.k_cache[l],
                                  self.v_cache[l], None if merge else self.b_att, cfg.n_heads,
                                  cfg.n_kv_heads, cfg.head_dim, self.w_att)
            if merge:
                glue.matmul_attn_merge(self.w_att, pos, lw.o_gg, x, cfg.n_heads, cfg.n_kv_heads,
                                       cfg.head_dim, cfg.max_seq, accumulate=True)
            else:
                glue.matmul_fused(self.b_att, lw.o_gg, x, accumulate=True)
            gui = lw.get("gateUpI_gg")
            if gui is not None:
                glue.matmul_fused(x, gui, self.b_a, glue.PROLOGUE_RMSNORM, lw.ffn_norm, cfg.eps,
                                  epilogue=glue.EPILOGUE_SWIGLU)
                glue.matmul_fused(self.b_a, lw.down_gg, x, accumulate=True)
            else:
                self._fused_slot(x, lw, "gateUp", self.b_gu, lw.ffn_norm)
                glue.matmul_fused(self.b_gu, lw.down_gg, x, glue.PROLOGUE_SWIGLU,
                                  accumulate=True)
        glue.matmul_fused(x, W.lm_head_gg, self.b_logits, glue.PROLOGUE_RMSNORM, W.final_norm,
                          cfg.eps)
        glue.argmax(self.b_logits, tok, self.w_arg)
        pos.add_(1)
        return self.b_logits

    def _fused_slot(self, x, lw, slot, y, norm_w) -> None:
        """RMSNorm-prologue projection of a concatenated slot into ``y`` (one launch
        per part; the parts write consecutive column ranges of ``y``)."""
        c = 0
        for w in parts(lw, slot):
            glue.matmul_fused(x, w, y[:, c:c + w.n], glue.PROLOGUE_RMSNORM, norm_w, self.cfg.eps)
            c += w.n

    @torch.no_grad()
    def step(self, tok: torch.Tensor, pos: torch.Tensor) -> torch.Tensor:
        """One greedy decode step in place: reads token ``tok`` [1] at position
        ``pos`` [1], writes the next token into ``tok`` and advances ``pos``.
        Touches no host state, so it can be captured in a graph."""
        if self.fused:
            return self._step_fused(tok, pos)
        x = self._embed(tok)
        x = self._layers(x, pos)
        logits = self._logits(x)
        tok.copy_(torch.argmax(logits, dim=-1))
        pos.add_(1)
        return logits

    @torch.no_grad()
    def capture(self, tok: torch.Tensor, pos: torch.Tensor) -> None:
        """Capture ``step(tok, pos)`` in a HIP graph (tok / pos are the static inputs).
        The capture run itself executes one step, so it is made on a copy."""
        s = torch.cuda.Stream(device=self.device)
        s.wait_stream(torch.cuda.current_stream(self.device))
        t0, p0 = tok.clone(), pos.clone()
        kc, vc = self.k_cache.clone(), self.v_cache.clone()
        with torch.cuda.stream(s):
            self.step(tok, pos)                    # warm-up outside the graph
        torch.cuda.current_stream(self.device).wait_stream(s)
        tok.copy_(t0)
        pos.copy_(p0)
        self.k_cache.copy_(kc)
        self.v_cache.copy_(vc)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            self._graph_logits = self.step(tok, pos)
        tok.copy_(t0)
        pos.copy_(p0)
        self.k_cache.copy_(kc)
        self.v_cache.copy_(vc)
        del kc, vc
        self._graph = g

    @torch.no_grad()
    def generate(self, prompt: torch.Tensor, n_new: int, graph: bool = True) -> dict:
        """Greedy generation: returns the new token ids and prefill / decode timings.
        tok/s = n_new / decode wall time (prefill excluded, generate.ts:1155-1160)."""
        dev = self.device
        if prompt.numel() + n_new > self.cfg.max_seq:
            raise ValueError(f"prompt {prompt.numel()} + {n_new} new tokens exceed max_seq "
                             f"{self.cfg.max_seq}")
        self.k_cache.zero_()
        self.v_cache.zero_()
        torch.cuda.synchronize(dev)
        t0 = time.perf_counter()
        logits = self.prefill(prompt, 0)
        tok = torch.argmax(logits, dim=-1).view(1)
        torch.cuda.synchronize(dev)
        t_prefill = time.perf_counter() - t0
        pos = torch.full((1,), prompt.numel(), dtype=torch.long, device=dev)
        out = torch.empty(n_new, dtype=torch.long, device=dev)
        out[0] = tok[0]
        if graph:
            self.capture(tok, pos)
        torch.cuda.synchronize(dev)
        t1 = time.perf_counter()
        for i in range(1, n_new):
            if graph:
                self._graph.replay()
            else:
                self.step(tok, pos)
            out[i] = tok[0]
        torch.cuda.synchronize(dev)
        t_decode = time.perf_counter() - t1
        steps = max(n_new - 1, 1)
        return {"tokens": out, "prefill_s": t_prefill, "decode_s": t_decode,
                "decode_steps": steps, "tok_s": steps / t_decode,
                "prefill_tok_s": prompt.numel() / t_prefill}
