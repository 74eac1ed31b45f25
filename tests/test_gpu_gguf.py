"""GGUF loader, row-gather kernel and file-loaded decoder on the GPU.

* ``gguf_hip_get_rows`` is bit-exact to the oracle's dequant of the named rows
  (the reference's CPU embedding row-gather, forward-pass.ts:2171-2186).
* The loader places each tensor kind as ``gguf-loader.ts`` does: quantized
  matrices repacked, F32/F16/BF16 as f32, ``token_embd`` as a gather table,
  experts / vision / ``rope_freqs`` kept off the device.
* A decoder loaded from a synthetic llama GGUF file (Q/K rows permuted as
  llama.cpp's converter writes them, Q/K/V of mixed types, a Q8_0 token table)
  matches a decoder built directly from the same quantized rows bit for bit,
  and the float64 reference decoder of test_gpu_decoder.py with RoPE
  frequency factors.
"""
import importlib

import numpy as np
import pytest

torch = pytest.importorskip("torch")

import gguf_models as gm  # noqa: E402
from test_gpu_decoder import Reference, _rel  # noqa: E402

pytestmark = pytest.mark.gpu

pkg = importlib.import_module("artifex-assistantv5_amd")
loader = importlib.import_module("artifex-assistantv5_amd.gguf_loader")
gmodel = importlib.import_module("artifex-assistantv5_amd.gguf_model")
dec = importlib.import_module("artifex-assistantv5_amd.decoder")


@pytest.mark.parametrize("t", [2, 6, 8, 10, 11, 12, 13, 14, 20, 23])
def test_get_rows_bit_exact(ref, t):
    n, k = 40, 512
    raw = pkg.quantize.quantize(pkg.quantize.synthetic_weight(n, k, seed=t, std=1.0), t)
    table = pkg.QuantEmbedding(torch.from_numpy(raw).cuda(), t, n, k)
    ids = [3, 0, 39, 3, 17]
    got = table.gather(torch.tensor(ids, device="cuda")).cpu().numpy()
    want = ref.dequant_rows(t, raw, n, k)[ids]
    assert ref.same_bits(got, want)
    # strided output rows and an out-of-range id (a NaN row, no fault)
    out = torch.zeros(3, k + 64, device="cuda")
    table.gather(torch.tensor([1, n, -1], device="cuda"), out[:, :k])
    o = out.cpu().numpy()
    assert ref.same_bits(o[0, :k], ref.dequant_rows(t, raw, n, k)[1])
    assert np.isnan(o[1:, :k]).all() and (o[:, k:] == 0).all()


def test_loader_placement(tmp_path, ref):
    tensors = gm.make_model(seed=1, rope_freqs=True)
    extra = [("blk.0.ffn_gate_exps.weight", [256, 64, 4], 12,
              np.zeros(4 * 64 * 144, np.uint8)),
             ("v.patch_embd.weight", [32, 4], 0, np.zeros(128, np.float32)),
             ("blk.0.attn_q_norm.weight", [64], 1, np.arange(64, dtype=np.float16)),
             ("blk.0.bias16.weight", [64], 30,
              (np.arange(64, dtype=np.float32).view(np.uint32) >> 16).astype(np.uint16))]
    p = str(tmp_path / "m.gguf")
    gm.write_model(p, tensors, extra_tensors=extra)
    m = loader.load_gguf_model(p, "cuda")
    assert set(m.expert_tensors) == {"blk.0.ffn_gate_exps.weight"}
    assert m.expert_bytes == 4 * 64 * 144
    assert "v.patch_embd.weight" not in m.tensors
    assert "rope_freqs.weight" in m.host_tensors and "rope_freqs.weight" not in m.tensors
    f16 = m.tensors["blk.0.attn_q_norm.weight"]
    assert f16.data.dtype == torch.float32 and not f16.is_quantized
    assert torch.equal(f16.data.cpu(), torch.arange(64, dtype=torch.float32))
    assert torch.equal(m.tensors["blk.0.bias16.weight"].data.cpu(),
                       torch.arange(64, dtype=torch.float32))
    norm = m.tensors["blk.1.ffn_norm.weight"].data.cpu().numpy()
    assert np.array_equal(norm, tensors["blk.1.ffn_norm.weight"][3])
    emb = m.row_tables["token_embd.weight"]
    assert isinstance(emb, pkg.QuantEmbedding) and "token_embd.weight" not in m.tensors
    down = m.tensors["blk.1.ffn_down.weight"]
    assert down.is_quantized and down.dtype == "Q6_K"
    typ, n, k, raw = tensors["blk.1.ffn_down.weight"]
    assert ref.same_bits(down.data.dequant().cpu().numpy(), ref.dequant_rows(typ, raw, n, k))
    assert m.total_gpu_bytes >= sum(t.byte_length for t in m.tensors.values())


def test_tied_embeddings_feed_the_lm_head(tmp_path, ref):
    tensors = gm.make_model(seed=2, tied=True)
    p = str(tmp_path / "tied.gguf")
    gm.write_model(p, tensors)
    m = loader.load_gguf_model(p, "cuda")
    typ, n, k, raw = tensors["token_embd.weight"]
    w = m.tensors["token_embd.weight"].data
    assert (w.n, w.k) == (n, k)
    assert ref.same_bits(w.dequant().cpu().numpy(), ref.dequant_rows(typ, raw, n, k))
    assert isinstance(m.row_tables["token_embd.weight"], pkg.QuantEmbedding)


LOW_BIT = {"q": 11, "k": 10, "v": 23, "o": 2, "gate": 6, "up": 6, "down": 20, "embd": 11,
           "out": 10}          # Q3_K, Q2_K, IQ4_XS, Q4_0, Q5_0, IQ4_NL, Q3_K table, Q2_K head


GRID_MIX = {"q": 16, "k": 17, "v": 18, "o": 21, "gate": 22, "up": 29, "down": 16, "embd": 21,
            "out": 22}         # IQ2_XXS, IQ2_XS, IQ3_XXS, IQ3_S, IQ2_S, IQ1_M (fused decode step)


@pytest.mark.parametrize("variant", ["mixed_qkv", "uniform_tied", "low_bit", "grid"])
def test_decoder_from_gguf_matches_direct_build(tmp_path, variant):
    types = {"mixed_qkv": {}, "uniform_tied": {"v": 12, "down": 12, "embd": 14},
             "low_bit": LOW_BIT, "grid": GRID_MIX}[variant]
    tensors = gm.make_model(seed=4, types=types, tied=variant == "uniform_tied")
    p = str(tmp_path / "m.gguf")
    gm.write_model(p, tensors)
    model, loaded = gmodel.load_decoder(p, "cuda", max_seq=64)
    cfg = model.cfg
    lw = model.w.layers[0]
    if variant != "uniform_tied":
        assert lw.get("qkv_gg") is None and len(lw.qkv_parts) == 3
    else:
        assert lw.qkv_gg is not None
    direct = dec.QuantDecoder(cfg, gm.direct_weights(tensors, gm.TINY))
    assert model.fused and direct.fused           # every type has the fused step kernels
    prompt = torch.from_numpy(np.random.default_rng(7).integers(0, cfg.vocab, 24)).cuda()
    assert torch.equal(model.prefill(prompt), direct.prefill(prompt))
    a = model.generate(prompt, 10, graph=True)
    b = direct.generate(prompt, 10, graph=False)
    assert torch.equal(a["tokens"], b["tokens"])


def test_grid_model_fused_step_matches_unfused(tmp_path):
    """A model of the six grid-codebook types: the fused decode step (RMSNorm
    prologues, the attention merge inside the output projection, SwiGLU as the
    down projection's prologue, residual-accumulate epilogues) against the
    torch-glue step over plain projections, teacher-forced on the same tokens."""
    tensors = gm.make_model(seed=4, types=GRID_MIX)
    p = str(tmp_path / "g.gguf")
    gm.write_model(p, tensors)
    model, _ = gmodel.load_decoder(p, "cuda", max_seq=64)
    w = gm.direct_weights(tensors, gm.TINY)
    a, b = dec.QuantDecoder(model.cfg, w, fused=True), dec.QuantDecoder(model.cfg, w, fused=False)
    assert a.fused and not b.fused
    toks = np.random.default_rng(9).integers(0, model.cfg.vocab, 30).tolist()
    for m in (a, b):
        m.prefill(torch.tensor(toks[:20], device="cuda"), 0)
    pa, pb = torch.tensor([20], device="cuda"), torch.tensor([20], device="cuda")
    for t in toks[20:]:
        ga = a.step(torch.tensor([t], device="cuda"), pa).clone()[0]
        gb = b.step(torch.tensor([t], device="cuda"), pb).clone()[0]
        assert ((ga.double() - gb.double()).norm() / gb.double().norm()).item() < 1e-5
    assert torch.allclose(a.k_cache[:, :, :30], b.k_cache[:, :, :30], rtol=1e-5, atol=1e-5)


def test_decoder_from_gguf_matches_float64_reference(tmp_path):
    tensors = gm.make_model(seed=5, rope_freqs=True)
    p = str(tmp_path / "m.gguf")
    gm.write_model(p, tensors, extra_kv={"llama.rope.freq_base": 500000.0})
    model, _ = gmodel.load_decoder(p, "cuda", max_seq=64)
    cfg = model.cfg
    assert cfg.rope_base == 500000.0 and len(cfg.rope_freq_factors) == cfg.head_dim // 2
    r = Reference(cfg, model.w)
    prompt = torch.from_numpy(np.random.default_rng(8).integers(0, cfg.vocab, 36)).cuda()
    logits = model.prefill(prompt)[0]
    for pos, t in enumerate(prompt.tolist()):
        rl = r.token(t, pos)
    assert _rel(logits, rl) < 5e-3
    tok = torch.argmax(logits).view(1)
    pos = torch.tensor([prompt.numel()], device="cuda")
    for _ in range(4):
        t = int(tok.item())
        lg = model.step(tok, pos)[0]
        assert _rel(lg, r.token(t, int(pos.item()) - 1)) < 1e-3
