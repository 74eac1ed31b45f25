"""Synthetic llama-architecture GGUF files for the loader tests.

Weights are drawn in the usual [out, in] order, quantized row by row with the
package quantizer (the grid-codebook IQ types, which it does not produce: random
valid blocks), and written the way llama.cpp's converter lays a llama
model out: Q and K rows permuted for interleaved-pair RoPE (stored row
``h*hd + 2j + p`` holds original row ``h*hd + p*hd/2 + j``), tensor names
``blk.N.attn_q.weight`` ..., ``ne = [in, out]``.  ``direct_weights`` builds the
same model straight from the unpermuted quantized rows, so a decoder loaded
from the file must match it bit for bit.
"""
from __future__ import annotations

import importlib

import numpy as np

pkg = importlib.import_module("artifex-assistantv5_amd")
gf = importlib.import_module("artifex-assistantv5_amd.gguf_file")

Q8_0, Q4_K, Q5_K, Q6_K, F32, F16, BF16 = 8, 12, 13, 14, 0, 1, 30
GRID = (16, 17, 18, 21, 22, 29)  # IQ2_XXS, IQ2_XS, IQ3_XXS, IQ3_S, IQ2_S, IQ1_M

TINY = dict(n_layers=2, d_model=256, n_heads=4, n_kv_heads=2, head_dim=64, ffn=512, vocab=384)


def permute_rows(n_heads, head_dim):
    """Stored row order of the converter: stored[i] = original[perm[i]]."""
    half = head_dim // 2
    h, j, p = np.meshgrid(np.arange(n_heads), np.arange(half), np.arange(2), indexing="ij")
    return (h * head_dim + p * half + j).reshape(-1)


def make_model(seed=0, types=None, rope_freqs=False, tied=False, cfg=TINY):
    """Quantized rows of every tensor in original order: dict name -> (type, n, k, raw)."""
    t = dict(q=Q4_K, k=Q4_K, v=Q5_K, o=Q4_K, gate=Q4_K, up=Q4_K, down=Q6_K, embd=Q8_0,
             out=Q6_K, norm=F32)
    t.update(types or {})
    rng = np.random.default_rng(seed)
    d, nh, nkv, hd, f, V = (cfg["d_model"], cfg["n_heads"], cfg["n_kv_heads"], cfg["head_dim"],
                            cfg["ffn"], cfg["vocab"])
    tensors = {}

    def quant(name, typ, n, k, scale=0.02):
        if typ in GRID:  # no quantizer for the grid-codebook types: random valid blocks
            from oracle import gguf_iq
            raw = gguf_iq.random_blocks(typ, n * k // 256, seed=int(rng.integers(1 << 30)),
                                        d=2.0 ** -10 if scale < 0.5 else 2.0 ** -5)
            tensors[name] = (typ, n, k, raw)
            return
        w = (rng.standard_normal((n, k)) * scale).astype(np.float32)
        tensors[name] = (typ, n, k, pkg.quantize.quantize(w, typ))

    def vec(name, n):
        v = (1.0 + 0.05 * rng.standard_normal(n)).astype(np.float32)
        tensors[name] = (t["norm"], 1, n, v)

    quant("token_embd.weight", t["embd"], V, d, scale=1.0)
    for l in range(cfg["n_layers"]):
        b = f"blk.{l}."
        vec(b + "attn_norm.weight", d)
        quant(b + "attn_q.weight", t["q"], nh * hd, d)
        quant(b + "attn_k.weight", t["k"], nkv * hd, d)
        quant(b + "attn_v.weight", t["v"], nkv * hd, d)
        quant(b + "attn_output.weight", t["o"], d, nh * hd)
        vec(b + "ffn_norm.weight", d)
        quant(b + "ffn_gate.weight", t["gate"], f, d)
        quant(b + "ffn_up.weight", t["up"], f, d)
        quant(b + "ffn_down.weight", t["down"], d, f)
    vec("output_norm.weight", d)
    if not tied:
        quant("output.weight", t["out"], V, d)
    if rope_freqs:
        tensors["rope_freqs.weight"] = (F32, 1, hd // 2,
                                        np.linspace(1.0, 8.0, hd // 2).astype(np.float32))
    return tensors


def _stored(name, typ, n, k, raw, cfg):
    if typ in (F32, F16, BF16):
        v = raw.astype(np.float32)
        if typ == F16:
            return v.astype(np.float16).view(np.uint8)
        if typ == BF16:
            return (v.view(np.uint32) >> 16).astype(np.uint16).view(np.uint8)
        return v.view(np.uint8)
    rows = raw.reshape(n, -1)
    if name.endswith("attn_q.weight"):
        rows = rows[permute_rows(cfg["n_heads"], cfg["head_dim"])]
    elif name.endswith("attn_k.weight"):
        rows = rows[permute_rows(cfg["n_kv_heads"], cfg["head_dim"])]
    return np.ascontiguousarray(rows).reshape(-1)


def write_model(path, tensors, cfg=TINY, extra_kv=None, extra_tensors=()):
    kv = {"general.architecture": "llama", "general.name": "synthetic",
          "llama.block_count": cfg["n_layers"], "llama.embedding_length": cfg["d_model"],
          "llama.feed_forward_length": cfg["ffn"], "llama.attention.head_count": cfg["n_heads"],
          "llama.attention.head_count_kv": cfg["n_kv_heads"], "llama.rope.freq_base": 10000.0,
          "llama.attention.layer_norm_rms_epsilon": 1e-5, "llama.context_length": 4096}
    kv.update(extra_kv or {})
    out = []
    for name, (typ, n, k, raw) in tensors.items():
        ne = [k] if n == 1 and typ in (F32, F16, BF16) else [k, n]
        out.append((name, ne, typ, _stored(name, typ, n, k, raw, cfg)))
    out.extend(extra_tensors)
    gf.write_gguf(path, kv, out)


def direct_weights(tensors, cfg, device="cuda"):
    """DecoderWeights from the original-order rows (no file involved)."""
    import torch
    from oracle import gguf_ref

    dec = importlib.import_module("artifex-assistantv5_amd.decoder")

    def q(name):
        typ, n, k, raw = tensors[name]
        return pkg.repack_gguf_for_gpu(typ, raw, n, k, device=device)

    def v(name):
        return torch.from_numpy(tensors[name][3].astype(np.float32)).to(device)

    def fuse(ws):
        if len({w.ggml_type for w in ws}) == 1:
            return {"gg": pkg.concat_rows(*ws)}
        return {"parts": ws}

    layers = []
    for l in range(cfg["n_layers"]):
        b = f"blk.{l}."
        slots = dict(o_gg=q(b + "attn_output.weight"), down_gg=q(b + "ffn_down.weight"),
                     attn_norm=v(b + "attn_norm.weight"), ffn_norm=v(b + "ffn_norm.weight"))
        for k_, w_ in fuse([q(b + "attn_q.weight"), q(b + "attn_k.weight"),
                            q(b + "attn_v.weight")]).items():
            slots[f"qkv_{k_}"] = w_
        for k_, w_ in fuse([q(b + "ffn_gate.weight"), q(b + "ffn_up.weight")]).items():
            slots[f"gateUp_{k_}"] = w_
        layers.append(pkg.LayerWeights(**slots))
    typ, n, k, raw = tensors["token_embd.weight"]
    embed = torch.from_numpy(gguf_ref.dequant_rows(typ, raw, n, k)).to(device)
    lm = q("output.weight" if "output.weight" in tensors else "token_embd.weight")
    return dec.DecoderWeights(layers, v("output_norm.weight"), lm, embed)
