"""Build a ``QuantDecoder`` from a GGUF model file.

The reference maps GGUF tensor names onto its layer slots when it loads a
model (``webgpu/src/model/gguf-loader.ts``, slots of
``webgpu/src/engine/forward-pass.ts:154-171,236-239``).  This module does the
same for the Llama-style decoder of this library (``decoder.py``), which
covers the ``llama`` architecture: per block ``attn_norm``, ``attn_q/k/v``,
``attn_output``, ``ffn_norm``, ``ffn_gate/up/down``; then ``output_norm``,
``output`` (or the tied ``token_embd``) and the ``token_embd`` row table.

llama.cpp's converter stores the Q and K rows of a ``llama`` model permuted
for its interleaved-pair RoPE (within a head, row ``2 j + p`` holds the
original row ``p * head_dim / 2 + j``).  The decoder here rotates the halves
of a head (rotate_half, ``webgpu/src/shaders/rope.wgsl:1-10``), so the loader
un-permutes those rows on the device before the repack; quantization is per
row, so the result is byte-identical to quantizing the original rows.
``rope_freqs.weight`` (Llama 3.x frequency factors) divides the RoPE angles.

Any other architecture, or a block tensor outside that list (biases, Q/K
norms, MoE experts), raises ``NotImplementedError`` before anything is loaded.
"""

from __future__ import annotations

import re
from typing import Optional, Tuple

import numpy as np
import torch

from .decoder import DecoderConfig, DecoderWeights, QuantDecoder
from .ggml import GGML_TYPE_NAMES
from .gguf_file import GGUFFile, GGUFTensorInfo, arch_kv, gguf_architecture, parse_gguf_path
from .gguf_loader import LoadedGGUFModel, load_gguf_model
from .linear import GGUFWeight, LayerWeights, QuantEmbedding, concat_rows, interleave_tiles

SUPPORTED_ARCHS = ("llama",)
BLOCK_TENSORS = ("attn_norm", "attn_q", "attn_k", "attn_v", "attn_output", "ffn_norm",
                 "ffn_gate", "ffn_up", "ffn_down")
GLOBAL_TENSORS = ("token_embd.weight", "output_norm.weight", "output.weight", "rope_freqs.weight")
_BLK = re.compile(r"^blk\.(\d+)\.(.+)\.weight$")


def config_from_gguf(file: GGUFFile, max_seq: int = 2048) -> DecoderConfig:
    """Decoder shape from the ``<arch>.*`` metadata of a llama-architecture file."""
    arch = gguf_architecture(file)
    if arch not in SUPPORTED_ARCHS:
        raise NotImplementedError(f"[gguf-hip] architecture {arch!r}: the decoder supports "
                                  f"{', '.join(SUPPORTED_ARCHS)}")
    d = int(arch_kv(file, "embedding_length"))
    nh = int(arch_kv(file, "attention.head_count"))
    nkv = int(arch_kv(file, "attention.head_count_kv", nh))
    hd = int(arch_kv(file, "attention.key_length", d // nh))
    emb = file.tensors.get("token_embd.weight")
    if emb is None:
        raise ValueError("[GGUF] Missing token_embd.weight")
    return DecoderConfig(
        n_layers=int(arch_kv(file, "block_count")), d_model=d, n_heads=nh, n_kv_heads=nkv,
        head_dim=hd, ffn=int(arch_kv(file, "feed_forward_length")), vocab=int(emb.ne[1]),
        rope_base=float(arch_kv(file, "rope.freq_base", 10000.0)),
        eps=float(arch_kv(file, "attention.layer_norm_rms_epsilon", 1e-5)), max_seq=max_seq)


def _check_tensors(file: GGUFFile, cfg: DecoderConfig) -> None:
    extra = []
    for name in file.tensors:
        m = _BLK.match(name)
        if m:
            if int(m.group(1)) >= cfg.n_layers or m.group(2) not in BLOCK_TENSORS:
                extra.append(name)
        elif name not in GLOBAL_TENSORS:
            extra.append(name)
    if extra:
        shown = ", ".join(extra[:6]) + (" ..." if len(extra) > 6 else "")
        raise NotImplementedError(f"[gguf-hip] the llama decoder has no slot for {len(extra)} "
                                  f"tensor(s): {shown}")


def unpermute_rows(n_heads: int, head_dim: int) -> np.ndarray:
    """Row order that undoes the converter's Q/K permutation: original row
    ``h*hd + p*hd/2 + j`` is stored at ``h*hd + 2*j + p``."""
    half = head_dim // 2
    h, p, j = np.meshgrid(np.arange(n_heads), np.arange(2), np.arange(half), indexing="ij")
    return (h * head_dim + 2 * j + p).reshape(-1)


def load_decoder(path: str, device="cuda", max_seq: int = 2048, fused: bool = True,
                 on_progress=None) -> Tuple[QuantDecoder, LoadedGGUFModel]:
    """Load a llama-architecture GGUF file into a ``QuantDecoder`` on ``device``."""
    file = parse_gguf_path(path)
    cfg = config_from_gguf(file, max_seq)
    _check_tensors(file, cfg)
    dev = torch.device(device)
    perms = {}
    for l in range(cfg.n_layers):
        perms[f"blk.{l}.attn_q.weight"] = unpermute_rows(cfg.n_heads, cfg.head_dim)
        perms[f"blk.{l}.attn_k.weight"] = unpermute_rows(cfg.n_kv_heads, cfg.head_dim)

    def transform(t: GGUFTensorInfo, rows: torch.Tensor) -> torch.Tensor:
        idx = perms.get(t.name)
        if idx is None:
            return rows
        if idx.size != rows.shape[0]:
            raise ValueError(f"[GGUF] {t.name}: {rows.shape[0]} rows, expected {idx.size}")
        return rows.index_select(0, torch.from_numpy(idx).to(rows.device))

    loaded = load_gguf_model(path, dev, on_progress=on_progress, raw_transform=transform)
    rope = loaded.host_tensors.get("rope_freqs.weight")
    if rope is not None:
        info = file.tensors["rope_freqs.weight"]
        if GGML_TYPE_NAMES[info.ggml_type] != "F32":
            raise NotImplementedError("[gguf-hip] rope_freqs.weight must be F32")
        cfg.rope_freq_factors = tuple(float(v) for v in rope.view(np.float32))

    T = loaded.tensors

    def quant(name: str, n: int, k: int) -> GGUFWeight:
        t = T.get(name)
        if t is None:
            raise ValueError(f"[GGUF] Missing {name}")
        if not t.is_quantized:
            raise NotImplementedError(f"[gguf-hip] {name} is {t.dtype}: the decoder's "
                                      "projections need a quantized GGUF type")
        w = t.data
        if (w.n, w.k) != (n, k):
            raise ValueError(f"[GGUF] {name} is [{w.n}, {w.k}], expected [{n}, {k}]")
        return w

    def vec(name: str, n: int) -> torch.Tensor:
        t = T.get(name)
        if t is None or t.is_quantized or t.data.numel() != n:
            raise ValueError(f"[GGUF] {name}: expected an f32/f16/bf16 vector of {n}")
        return t.data.reshape(n).contiguous()

    def fuse(ws):
        if len({w.ggml_type for w in ws}) == 1 and all(w.n % 16 == 0 for w in ws[:-1]):
            return {"gg": concat_rows(*ws)}
        return {"parts": list(ws)}

    def fuse_ffn(gate, up):
        if gate.ggml_type == up.ggml_type and gate.n % 16 == 0:
            return {"I_gg": interleave_tiles(gate, up)}
        return {"_parts": [gate, up]}

    d, hd, nh, nkv, f = cfg.d_model, cfg.head_dim, cfg.n_heads, cfg.n_kv_heads, cfg.ffn
    layers = []
    for l in range(cfg.n_layers):
        b = f"blk.{l}."
        qkv = fuse([quant(b + "attn_q.weight", nh * hd, d), quant(b + "attn_k.weight", nkv * hd, d),
                    quant(b + "attn_v.weight", nkv * hd, d)])
        gu = fuse_ffn(quant(b + "ffn_gate.weight", f, d), quant(b + "ffn_up.weight", f, d))
        slots = dict(o_gg=quant(b + "attn_output.weight", d, nh * hd),
                     down_gg=quant(b + "ffn_down.weight", d, f),
                     attn_norm=vec(b + "attn_norm.weight", d),
                     ffn_norm=vec(b + "ffn_norm.weight", d))
        slots.update({f"qkv_{k}": v for k, v in qkv.items()})
        slots.update({f"gateUp{k}": v for k, v in gu.items()})
        layers.append(LayerWeights(**slots))
        for name in ("attn_q", "attn_k", "attn_v", "ffn_gate", "ffn_up"):
            if (qkv if name.startswith("attn") else gu).keys() & {"gg", "I_gg"}:
                T.pop(b + name + ".weight", None)   # the concatenated copy replaces them
    lm_name = "output.weight" if "output.weight" in T else "token_embd.weight"
    lm = quant(lm_name, cfg.vocab, d)
    embed = loaded.row_tables["token_embd.weight"]
    if isinstance(embed, torch.Tensor) and embed.shape != (cfg.vocab, d):
        raise ValueError(f"[GGUF] token_embd.weight is {tuple(embed.shape)}, expected "
                         f"[{cfg.vocab}, {d}]")
    if isinstance(embed, QuantEmbedding) and (embed.n, embed.k) != (cfg.vocab, d):
        raise ValueError(f"[GGUF] token_embd.weight is [{embed.n}, {embed.k}], expected "
                         f"[{cfg.vocab}, {d}]")
    weights = DecoderWeights(layers, vec("output_norm.weight", d), lm, embed)
    return QuantDecoder(cfg, weights, device=dev, fused=fused), loaded
