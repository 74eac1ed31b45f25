"""Benchmark of the GGUF dequant-matmul path on one MI355X.

Headline workload: Q4_K decode GEMV, M=1, K=4096, N=14336 (FFN gate/up), fp32
activations ~N(0,1), weights ~N(0,0.02) quantized to Q4_K.  One step = one
GEMV over one activation vector.  Weights are cold: step i reads weight copy
i mod P of P distinct copies (P * 33 MB > 512 MB, twice the 256 MB Infinity
Cache), so the bytes come from HBM.

Timing: the K timed steps are captured once as a HIP graph (one kernel per
step, as a decode loop issues them) and replayed once between two stream
synchronizations; HIP events on that stream bracket the replay.
``ms_per_step`` = replay time / K, which includes the launch gaps between
kernels, so ``roofline.achieved`` (algorithmic bytes per step / ms_per_step)
is a lower bound on the kernel's own rate.  The eager (one Python launch per
step) time is reported under ``secondary``.

Prints ONE JSON line.  Besides the headline it carries the other two parts of
the metric: ``prefill_gemm`` (Q4_K dequant-GEMM M=2048 K=4096 N=14336, fp16
activations, TFLOP/s against the dense fp16 MFMA peak) and ``decode`` (the
full synthetic Llama-style decoder: 32 layers, d_model 4096, 32/8 heads of
128, SwiGLU FFN 14336, vocab 151936, Q4_K attention and gate/up, Q6_K down and
LM head; 128 random prompt tokens then 256 greedy tokens; tok/s = generated
tokens / decode wall time, prefill excluded).  ``secondary`` holds the other
configurations of the path (Q4_K / Q5_K / Q6_K decode shapes and batch sizes,
the other GGML types at the headline shape, more prefill shapes, f32 prefill
activations).  ``cpu_baseline`` = the CPU restatement of the reference
path (the compiled C oracle, oracle/gguf_ref_c.c: Q4_K dequant fused with the
GEMV, OpenMP; numpy dequant + torch fp32 matmul when it is not built) on the
host threads, repeated for about 10 s, with two more entries: ``prefill`` (the Q4_K GEMM shape at
M=256) and ``decoder`` (the bench decoder in f32 on the host, ms/token over 8
greedy tokens).  Each carries the host CPU model string, the cores used and the
torch version.  ``roofline.traffic`` is read from the committed rocprofv3
counter summary of the headline kernel when present.
"""

from __future__ import annotations

import argparse
import importlib
import json
import math
import os
import platform
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0           # MI355X HBM3E, published
FP16_PEAK_TFLOPS = 2500.0       # MI355X dense fp16 MFMA, published
BLOCK = {8: (32, 34), 12: (256, 144), 13: (256, 176), 14: (256, 210), 2: (32, 18), 6: (32, 22),
         20: (32, 18), 23: (256, 136), 10: (256, 84), 11: (256, 110), 16: (256, 66),
         17: (256, 74), 22: (256, 82), 18: (256, 98), 21: (256, 110), 29: (256, 56)}


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=340)
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--pool", type=int, default=17, help="distinct weight copies (cold weights)")
    p.add_argument("--cpu-seconds", type=float, default=10.0)
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--no-secondary", action="store_true")
    p.add_argument("--only", default="", help="comma list of secondary groups to run")
    p.add_argument("--no-decoder", action="store_true")
    p.add_argument("--kernel-only", type=int, default=0, metavar="N",
                   help="profiling driver: N headline launches over the cold pool, then four "
                        "64 MiB device copies (counter calibration); prints no JSON")
    p.add_argument("--decode-tokens", type=int, default=256)
    return p.parse_args()


def graph_time(step, steps, warmup):
    """ms per step: ``steps`` launches captured as one graph, replayed once (timed)."""
    import torch
    for i in range(warmup):
        step(i)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(steps):
            step(i)
    g.replay()                      # untimed: first replay uploads the graph
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    g.replay()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps


def graph_time_median(step, steps, warmup, replays=3):
    """Like graph_time, but the median over ``replays`` timed replays of the graph."""
    import torch
    for i in range(warmup):
        step(i)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(steps):
            step(i)
    g.replay()
    torch.cuda.synchronize()
    times = []
    for _ in range(replays):
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record()
        g.replay()
        end.record()
        torch.cuda.synchronize()
        times.append(start.elapsed_time(end) / steps)
    return float(np.median(times))


def eager_time(step, steps, warmup):
    import torch
    for i in range(warmup):
        step(i)
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    for i in range(steps):
        step(warmup + i)
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps


def make_pool(pkg, t, n, k, copies, seed):
    """``copies`` distinct device copies of one quantized weight (row-tile layout):
    seeded N(0, 0.02) weights through the package quantizer; the raw bytes are
    returned for the CPU baseline."""
    w = pkg.quantize.synthetic_weight(n, k, seed=seed)
    raw = pkg.quantize.quantize(w, t)
    base = pkg.repack_gguf_for_gpu(t, raw, n, k, device="cuda")
    pool = [base] + [pkg.GGUFWeight(base.data.clone(), t, n, k) for _ in range(copies - 1)]
    return pool, raw


IQ_GRID = ((16, "iq2_xxs"), (17, "iq2_xs"), (22, "iq2_s"), (18, "iq3_xxs"), (21, "iq3_s"),
           (29, "iq1_m"))


def iq_pool(pkg, t, n, k, copies, seed):
    """``copies`` device copies of random IQ blocks (every bit pattern is a legal
    code) whose f16 d is 2^-8 (IQ1_M: spread over its scale words' top nibbles):
    the package has no quantizer for the grid types."""
    import torch
    block, size = BLOCK[t]
    rng = np.random.default_rng(seed)
    raw = rng.integers(0, 256, (n * (k // block), size), dtype=np.uint8)
    dh = int(np.array([2.0 ** -8], np.float16).view(np.uint16)[0])
    if t == 29:
        w = raw[:, 48:56].copy().view("<u2").astype(np.int64)
        for i in range(4):
            w[:, i] = (w[:, i] & 0x0FFF) | (((dh >> (4 * i)) & 0xF) << 12)
        raw[:, 48:56] = w.astype("<u2").view(np.uint8).reshape(-1, 8)
    else:
        raw[:, 0], raw[:, 1] = dh & 0xFF, dh >> 8
    base = pkg.repack_gguf_for_gpu(t, raw.reshape(-1), n, k, device="cuda")
    return [base] + [pkg.GGUFWeight(base.data.clone(), t, n, k) for _ in range(copies - 1)]


def matmul_case(pkg, t, m, n, k, pool, steps, warmup, xdtype="float32", eager=False,
                replays=1):
    import torch
    x = torch.from_numpy(pkg.quantize.synthetic_activations(m, k, seed=7)).cuda().to(
        getattr(torch, xdtype))
    y = torch.empty(m, n, device="cuda")
    P = len(pool)

    def step(i):
        pkg.dispatch_matmul_gguf(x, pool[i % P], y, m, n, k, "bench")

    ms = graph_time(step, steps, warmup) if replays == 1 else graph_time_median(step, steps, warmup,
                                                                               replays)
    wbytes = n * pkg.raw_row_bytes(t, k)
    algo = wbytes + m * k * x.element_size() + m * n * 4
    out = {"ms": ms, "bytes": algo, "gbs": algo / (ms * 1e-3) / 1e9,
           "tflops": 2.0 * m * n * k / (ms * 1e-3) / 1e12}
    if eager:
        out["eager_ms"] = eager_time(step, steps, warmup)
    return out


def _cpu_threads():
    """Host threads for the CPU baseline: the process's CPUs, capped by
    OMP_NUM_THREADS where that is set."""
    cores = len(os.sched_getaffinity(0))
    try:
        cap = int(os.environ.get("OMP_NUM_THREADS", "0"))
    except ValueError:
        cap = 0
    return min(cores, cap) if cap > 0 else cores


def _oracle_c():
    """The compiled C restatement of the oracle (oracle/liboracle.so), or None."""
    from oracle import build_oracle
    return build_oracle.load()


def cpu_baseline(pkg, raw, t, n, k, seconds, m=1):
    """CPU restatement of the reference path, repeated ~``seconds``: the compiled
    C oracle (Q4_K dequant fused with the GEMV, gcc -O3 AVX2, OpenMP over weight
    rows) on every host thread; without it, the numpy oracle's dequant + a torch
    fp32 matmul."""
    import torch
    from oracle import gguf_ref as ref
    cores = _cpu_threads()
    torch.set_num_threads(cores)
    x = pkg.quantize.synthetic_activations(m, k, seed=7).astype(np.float32)
    clib = _oracle_c() if t == 12 else None
    # distinct weight copies in turn (8 x 33 MB, beyond the host's last-level
    # caches), as the GPU line cycles through its cold pool
    pool = [np.array(raw, dtype=np.uint8, copy=True) for _ in range(8)] if clib is not None else []
    y = np.empty((m, n), np.float32)
    xt = torch.from_numpy(x)
    times, t_deq, t_mm = [], [], []
    t_start = time.perf_counter()
    it = 0
    while it < 4 or (time.perf_counter() - t_start < seconds and it < 100000):
        t0 = time.perf_counter()
        if clib is not None:
            w8 = pool[it % len(pool)]
            assert clib.oracle_matmul_q4_k(w8.ctypes.data, n, k, x.ctypes.data, m, y.ctypes.data,
                                           cores) > 0
            t1 = t2 = time.perf_counter()
        else:
            w = torch.from_numpy(ref.dequant_rows(t, raw, n, k))
            t1 = time.perf_counter()
            torch.matmul(xt, w.T)
            t2 = time.perf_counter()
        if it >= 2:                                    # two warm-ups
            times.append(t2 - t0)
            t_deq.append(t1 - t0)
            t_mm.append(t2 - t1)
        it += 1
    tot = float(np.median(times))
    wbytes = n * pkg.raw_row_bytes(t, k)
    head = (f"the headline workload (Q4_K M={m} K={k} N={n}) {len(times)} times after 2 warm-ups "
            f"({time.perf_counter() - t_start:.1f} s): ")
    if clib is not None:
        how = (f"compiled C restatement of the oracle (oracle/gguf_ref_c.c: gcc -O3 "
               f"-march=x86-64-v3, OpenMP, {cores} threads), each weight superblock dequantized "
               f"and dotted with x at once, over {len(pool)} weight copies in turn; median "
               f"{tot * 1e3:.2f} ms per step")
    else:
        how = (f"numpy dequant to f32 + torch.matmul f32; median dequant "
               f"{np.median(t_deq) * 1e3:.1f} ms, matmul {np.median(t_mm) * 1e3:.1f} ms, total "
               f"{tot * 1e3:.1f} ms per step")
    return {
        "value": round(wbytes / tot / 1e9, 3),
        "unit": "GB/s",
        "cores": cores,
        "kind": "port",
        "sample": head + how,
        "ms_per_step": round(tot * 1e3, 3),
        "cpu": cpu_model(),
        "torch": torch.__version__,
    }


def cpu_model():
    """The host CPU's model string (/proc/cpuinfo), else what platform reports."""
    try:
        with open("/proc/cpuinfo", encoding="utf-8") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


def cpu_prefill_baseline(pkg, raw, t, n, k, m, reps=5):
    """The prefill path on the host: oracle dequant (blocks -> f32 [N, K]; the
    compiled C restatement on every host thread when built, else numpy) + torch
    fp32 matmul of M fp16 activations upcast to f32; median of ``reps`` after 2
    warm-ups."""
    import torch
    from oracle import gguf_ref as ref
    cores = _cpu_threads()
    torch.set_num_threads(cores)
    x = torch.from_numpy(pkg.quantize.synthetic_activations(m, k, seed=7)).half().float()
    clib = _oracle_c() if t == 12 else None
    rawc = np.ascontiguousarray(raw, dtype=np.uint8)
    wbuf = np.empty((n, k), np.float32)
    t_deq, t_mm = [], []
    for it in range(reps + 2):
        t0 = time.perf_counter()
        if clib is not None:
            assert clib.oracle_dequant_rows_q4_k(rawc.ctypes.data, n, k, wbuf.ctypes.data, cores) > 0
            w = torch.from_numpy(wbuf)
        else:
            w = torch.from_numpy(ref.dequant_rows(t, raw, n, k))
        t1 = time.perf_counter()
        torch.matmul(x, w.T)
        t2 = time.perf_counter()
        if it >= 2:
            t_deq.append(t1 - t0)
            t_mm.append(t2 - t1)
    deq, mm = float(np.median(t_deq)), float(np.median(t_mm))
    flop = 2.0 * m * n * k
    return {
        "value": round(flop / (deq + mm) / 1e12, 4),
        "unit": "TFLOP/s",
        "cores": cores,
        "kind": "port",
        "sample": (f"Q4_K dequant-GEMM M={m} (the GPU line is M=2048) K={k} N={n}, fp16 "
                   f"activations upcast to f32: {reps} runs after 2 warm-ups; "
                   f"{'compiled C oracle dequant (OpenMP)' if clib is not None else 'numpy oracle dequant'}"
                   f" + torch f32 matmul; median dequant "
                   f"{deq * 1e3:.1f} ms + f32 matmul {mm * 1e3:.1f} ms "
                   f"({flop / mm / 1e12:.3f} TFLOP/s for the matmul alone)"),
        "ms_per_step": round((deq + mm) * 1e3, 3),
        "cpu": cpu_model(),
        "torch": torch.__version__,
    }


class CpuDecoder:
    """The bench decoder on the host in f32: weights dequantized once by the
    oracle (the CPU restatement of the reference dequant), projections as
    torch fp32 matmuls, norm / RoPE / attention / SwiGLU as plain torch ops
    (the same functions as the GPU decoder's prefill path).  Layers share one
    dequantized layer set, as the GPU run's layers share one quantized set;
    each layer's 0.9 GB still streams from DRAM (far beyond the caches)."""

    def __init__(self, cfg, w, norms, final_norm):
        import torch
        dec = importlib.import_module("artifex-assistantv5_amd.decoder")
        self.cfg, self.w, self.dec = cfg, w, dec
        self.norms, self.final_norm = norms, final_norm
        self.cos, self.sin = dec.rope_tables(cfg, "cpu")
        self.k = [[] for _ in range(cfg.n_layers)]
        self.v = [[] for _ in range(cfg.n_layers)]
        self.torch = torch

    def forward(self, tokens, pos0):
        """Run token ids ``tokens`` at positions pos0.. and return the last
        position's logits."""
        torch, cfg, dec, w = self.torch, self.cfg, self.dec, self.w
        M, nh, nkv, hd = len(tokens), cfg.n_heads, cfg.n_kv_heads, cfg.head_dim
        grp = nh // nkv
        pos = torch.arange(pos0, pos0 + M)
        cos, sin = self.cos[pos], self.sin[pos]
        x = w["embed"][torch.as_tensor(tokens)]
        for l in range(cfg.n_layers):
            an, fn = self.norms[l]
            qkv = dec.rms_norm(x, an, cfg.eps) @ w["qkv"].T
            q = dec.apply_rope(qkv[:, :nh * hd].view(M, nh, hd), cos, sin)
            k = dec.apply_rope(qkv[:, nh * hd:(nh + nkv) * hd].view(M, nkv, hd), cos, sin)
            self.k[l].append(k)
            self.v[l].append(qkv[:, (nh + nkv) * hd:].view(M, nkv, hd))
            K, V = torch.cat(self.k[l]), torch.cat(self.v[l])          # [T, nkv, hd]
            T = K.shape[0]
            qg = q.view(M, nkv, grp, hd).permute(1, 0, 2, 3).reshape(nkv, M * grp, hd)
            s = torch.matmul(qg, K.permute(1, 2, 0)) / math.sqrt(hd)   # [nkv, M*grp, T]
            mask = torch.arange(T)[None, :] > pos[:, None]              # [M, T]
            s = s.masked_fill(mask.repeat_interleave(grp, dim=0)[None], float("-inf"))
            o = torch.matmul(torch.softmax(s, dim=-1), V.permute(1, 0, 2))
            o = o.view(nkv, M, grp, hd).permute(1, 0, 2, 3).reshape(M, nh * hd)
            x = x + o @ w["o"].T
            h = dec.rms_norm(x, fn, cfg.eps)
            g, u = h @ w["gate"].T, h @ w["up"].T
            x = x + (u * torch.nn.functional.silu(g)) @ w["down"].T
        return dec.rms_norm(x[-1:], self.final_norm, cfg.eps) @ w["lm"].T


def cpu_decoder_baseline(pkg, prompt_len=16, n_new=8, lm_head_unique_rows=16384):
    """The bench decoder (``decoder_case``) on the host: the same configuration
    and quantized layer set (same seeds), dequantized once at load by the
    oracle; ``prompt_len`` prompt tokens, then ``n_new`` greedy tokens timed one
    by one (ms/token = median)."""
    import torch
    from oracle import gguf_ref as ref
    dec = importlib.import_module("artifex-assistantv5_amd.decoder")
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    cfg = dec.DecoderConfig()
    d, hd, q = cfg.d_model, cfg.head_dim, pkg.quantize
    t0 = time.perf_counter()

    def deq(t, n, k, seed):  # decoder.synthetic_weights' blocks for the same seed
        raw = q.quantize(q.synthetic_weight(n, k, seed=seed), t)
        return torch.from_numpy(ref.dequant_rows(t, raw, n, k))

    w = {"qkv": torch.cat([deq(cfg.attn_type, cfg.n_heads * hd, d, 1),
                           deq(cfg.attn_type, cfg.n_kv_heads * hd, d, 2),
                           deq(cfg.attn_type, cfg.n_kv_heads * hd, d, 3)]),
         "o": deq(cfg.attn_type, d, cfg.n_heads * hd, 4),
         "gate": deq(cfg.gate_up_type, cfg.ffn, d, 5),
         "up": deq(cfg.gate_up_type, cfg.ffn, d, 6),
         "down": deq(cfg.down_type, d, cfg.ffn, 7)}
    lm = deq(cfg.lm_head_type, lm_head_unique_rows, d, 99)
    w["lm"] = lm.repeat(-(-cfg.vocab // lm_head_unique_rows), 1)[:cfg.vocab].contiguous()
    w["embed"] = w["lm"]                                   # tied embedding table
    g = torch.Generator().manual_seed(0)
    norms = [(1.0 + 0.02 * torch.randn(d, generator=g), 1.0 + 0.02 * torch.randn(d, generator=g))
             for _ in range(cfg.n_layers)]
    final_norm = 1.0 + 0.02 * torch.randn(d, generator=g)
    t_load = time.perf_counter() - t0
    m = CpuDecoder(cfg, w, norms, final_norm)
    prompt = np.random.default_rng(0).integers(0, cfg.vocab, prompt_len).tolist()
    with torch.no_grad():
        t1 = time.perf_counter()
        tok = int(m.forward(prompt, 0).argmax())
        t_pre = time.perf_counter() - t1
        steps = []
        for i in range(n_new):
            t2 = time.perf_counter()
            tok = int(m.forward([tok], prompt_len + i).argmax())
            steps.append(time.perf_counter() - t2)
    ms = float(np.median(steps)) * 1e3
    return {
        "value": round(1e3 / ms, 3),
        "unit": "tok/s",
        "cores": cores,
        "kind": "port",
        "sample": (f"the bench decoder (32 layers, d 4096, 32/8 x 128, FFN 14336, vocab 151936, "
                   f"Q4_K attention and gate/up, Q6_K down and LM head) in f32 on the host: "
                   f"weights dequantized once at load ({t_load:.1f} s, one shared layer set), "
                   f"{prompt_len}-token prompt ({t_pre * 1e3:.0f} ms), then {n_new} greedy tokens "
                   f"(the GPU line decodes 256); median {ms:.1f} ms per token"),
        "ms_per_token": round(ms, 2),
        "cpu": cpu_model(),
        "torch": torch.__version__,
    }


def decoder_case(pkg, n_new):
    """Full synthetic decoder: 128-token random prompt then ``n_new`` greedy tokens."""
    import torch
    dec = importlib.import_module("artifex-assistantv5_amd.decoder")
    cfg = dec.DecoderConfig()
    t0 = time.perf_counter()
    w = dec.synthetic_weights(cfg, seed=0, lm_head_unique_rows=16384)
    torch.cuda.synchronize()
    t_w = time.perf_counter() - t0
    m = dec.QuantDecoder(cfg, w)
    prompt = torch.from_numpy(np.random.default_rng(0).integers(0, cfg.vocab, 128)).cuda()
    m.generate(prompt, 16)                              # warm-up (kernels, graph capture)
    r = m.generate(prompt, n_new)
    bpt = cfg.weight_bytes_per_token()
    ceiling = HBM_PEAK_GBS * 1e9 / bpt
    out = {
        "tok_s": round(r["tok_s"], 1),
        "ms_per_token": round(1e3 / r["tok_s"], 3),
        "weight_bytes_per_token": bpt,
        "weight_gbs": round(bpt * r["tok_s"] / 1e9, 1),
        "hbm_ceiling_tok_s": round(ceiling, 1),
        "frac_of_ceiling": round(r["tok_s"] / ceiling, 4),
        "prefill_ms": round(r["prefill_s"] * 1e3, 2),
        "prefill_tok_s": round(r["prefill_tok_s"], 1),
        "decode_steps_timed": r["decode_steps"],
        "workload": ("32 layers, d 4096, 32/8 heads x 128, SwiGLU 14336, vocab 151936; Q4_K "
                     "q/k/v/o and gate/up, Q6_K down and LM head; 128 random prompt ids then "
                     f"{n_new} greedy tokens, batch 1, each decode step one HIP graph replay"),
        "weights": ("seeded N(0,0.02) quantized with the package quantizer; the 32 layers hold "
                    "separate device copies of one quantized layer set, the LM head repeats "
                    "16384 quantized rows (every byte still streamed from HBM)"),
        "weight_setup_s": round(t_w, 1),
    }
    del m, w
    torch.cuda.empty_cache()
    return out


def traffic_from_profile():
    """HBM bytes per launch of the headline kernel from the committed rocprofv3
    FETCH_SIZE / WRITE_SIZE summary (profiles/q4k_decode_m1_k4096_n14336_traffic.json)."""
    f = os.path.join(ROOT, "profiles", "q4k_decode_m1_k4096_n14336_traffic.json")
    try:
        with open(f, encoding="utf-8") as fh:
            return json.load(fh).get("traffic_bytes_per_launch")
    except (OSError, ValueError):
        return None


def secondary_cases(pkg, args, pool, secondary):
    import torch
    only = set(filter(None, args.only.split(",")))

    def want(name):
        return not args.no_secondary and (not only or name in only)

    t = 12
    if want("gemv_batch"):
        for mm in (8, 32):
            r = matmul_case(pkg, t, mm, 14336, 4096, pool, 170, 5, replays=3)
            secondary[f"q4k_decode_m{mm}_gate_up_gbs"] = round(r["gbs"], 1)
    if want("down"):
        dpool, _ = make_pool(pkg, t, 4096, 14336, args.pool, seed=2)
        for mm in (1, 8, 32):
            r = matmul_case(pkg, t, mm, 4096, 14336, dpool, 170, 5, replays=3)
            secondary[f"q4k_decode_m{mm}_down_gbs"] = round(r["gbs"], 1)
        del dpool
    if want("batch_q6q8"):
        # decode (M = 1, 8, 32) and prefill (M = 2048, f16) of the path's other two types
        # (Q6_K, Q8_0) at the FFN shapes
        for tt, name in ((14, "q6k"), (8, "q8_0")):
            for (nn, kk), shape in (((14336, 4096), "gate_up"), ((4096, 14336), "down")):
                bpool, _ = make_pool(pkg, tt, nn, kk, 10, seed=40 + tt)
                for mm in (1, 8, 32):
                    r = matmul_case(pkg, tt, mm, nn, kk, bpool, 170, 5, replays=3)
                    secondary[f"{name}_decode_m{mm}_{shape}_gbs"] = round(r["gbs"], 1)
                if shape == "gate_up":
                    r = matmul_case(pkg, tt, 2048, nn, kk, bpool[:2], 10, 2, xdtype="float16")
                    secondary[f"{name}_gemm_m2048_n14336_tflops"] = round(r["tflops"], 1)
                    secondary[f"{name}_gemm_m2048_n14336_frac_fp16_peak"] = round(
                        r["tflops"] / FP16_PEAK_TFLOPS, 4)
                del bpool
    if want("q8"):
        qpool, _ = make_pool(pkg, 8, 4096, 4096, 32, seed=4)
        r = matmul_case(pkg, 8, 1, 4096, 4096, qpool, 320, 10, replays=3)
        secondary["q8_0_decode_m1_gbs"] = round(r["gbs"], 1)
        secondary["q8_0_decode_m1_frac_hbm"] = round(r["gbs"] / HBM_PEAK_GBS, 4)
        del qpool
    if want("small_blocks"):
        for tt, name in ((2, "q4_0"), (6, "q5_0"), (20, "iq4_nl"), (23, "iq4_xs"), (10, "q2_k"), (11, "q3_k")):
            spool, _ = make_pool(pkg, tt, 14336, 4096, 20, seed=8 + tt)
            r = matmul_case(pkg, tt, 1, 14336, 4096, spool, 280, 10, replays=3)
            secondary[f"{name}_decode_m1_gbs"] = round(r["gbs"], 1)
            secondary[f"{name}_decode_m1_frac_hbm"] = round(r["gbs"] / HBM_PEAK_GBS, 4)
            if tt in (23, 10, 11):
                r = matmul_case(pkg, tt, 2048, 14336, 4096, spool[:2], 10, 2, xdtype="float16")
                secondary[f"{name}_gemm_m2048_n14336_tflops"] = round(r["tflops"], 1)
                secondary[f"{name}_gemm_m2048_n14336_frac_fp16_peak"] = round(
                    r["tflops"] / FP16_PEAK_TFLOPS, 4)
            del spool
    if want("iq"):
        for tt, name in IQ_GRID:
            ipool = iq_pool(pkg, tt, 14336, 4096, 24, seed=20 + tt)
            for mm in (1, 8, 32):
                r = matmul_case(pkg, tt, mm, 14336, 4096, ipool, 240, 10, replays=3)
                secondary[f"{name}_decode_m{mm}_gbs"] = round(r["gbs"], 1)
            r = matmul_case(pkg, tt, 2048, 14336, 4096, ipool[:2], 10, 2, xdtype="float16")
            secondary[f"{name}_gemm_m2048_n14336_tflops"] = round(r["tflops"], 1)
            del ipool
    if want("q5k"):
        q5pool, _ = make_pool(pkg, 13, 14336, 4096, 14, seed=6)
        r = matmul_case(pkg, 13, 1, 14336, 4096, q5pool, 280, 10, replays=3)
        secondary["q5k_decode_m1_gbs"] = round(r["gbs"], 1)
        secondary["q5k_decode_m1_frac_hbm"] = round(r["gbs"] / HBM_PEAK_GBS, 4)
        r = matmul_case(pkg, 13, 2048, 14336, 4096, q5pool[:2], 10, 2, xdtype="float16")
        secondary["q5k_gemm_m2048_n14336_tflops"] = round(r["tflops"], 1)
        secondary["q5k_gemm_m2048_n14336_frac_fp16_peak"] = round(r["tflops"] / FP16_PEAK_TFLOPS, 4)
        del q5pool
    if want("lm_head"):
        dec = importlib.import_module("artifex-assistantv5_amd.decoder")
        lm = dec._tiled_rows(14, 16384, 151936, 4096, seed=5, device="cuda")
        lpool = [lm, pkg.GGUFWeight(lm.data.clone(), 14, 151936, 4096)]
        r = matmul_case(pkg, 14, 1, 151936, 4096, lpool, 40, 3, replays=3)
        secondary["q6k_lm_head_m1_gbs"] = round(r["gbs"], 1)
        secondary["q6k_lm_head_m1_frac_hbm"] = round(r["gbs"] / HBM_PEAK_GBS, 4)
        secondary["q6k_lm_head_weights"] = ("seeded N(0,0.02) weights quantized to Q6_K: 16384 "
                                            "rows repeated to 151936, each row's own bytes "
                                            "in HBM, 2 copies")
        del lpool, lm
    if want("prefill"):
        # the vendor's plain fp16 GEMM (hipBLASLt through torch.matmul, timed eagerly, not in
        # a graph) on the headline prefill shape: fp16 weights already dequantized, so a
        # ceiling for reference only
        xa = torch.randn(2048, 4096, device="cuda", dtype=torch.float16)
        wa = torch.randn(14336, 4096, device="cuda", dtype=torch.float16) * 0.02
        ms = min(eager_time(lambda i: torch.matmul(xa, wa.t()), 20, 3) for _ in range(3))
        secondary["torch_fp16_gemm_m2048_n14336_tflops"] = round(2.0 * 2048 * 14336 * 4096 /
                                                                 (ms * 1e-3) / 1e12, 1)
        del xa, wa
        for mm, nn in ((512, 4096), (512, 14336), (8192, 4096), (8192, 14336)):
            ppool = pool[:2] if nn == 14336 else make_pool(pkg, t, nn, 4096, 2, seed=3)[0]
            r = matmul_case(pkg, t, mm, nn, 4096, ppool, 10, 2, xdtype="float16")
            secondary[f"q4k_gemm_m{mm}_n{nn}_tflops"] = round(r["tflops"], 1)
            secondary[f"q4k_gemm_m{mm}_n{nn}_frac_fp16_peak"] = round(r["tflops"] / FP16_PEAK_TFLOPS, 4)
        # f32 activations (the decoder's prefill rows): staged once as an fp16 image in the
        # workspace, then the same GEMM
        for mm in (512, 2048):
            r = matmul_case(pkg, t, mm, 14336, 4096, pool[:2], 10, 2, xdtype="float32")
            secondary[f"q4k_gemm_m{mm}_n14336_f32x_tflops"] = round(r["tflops"], 1)


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this library runs on one GPU only; use --gpus 1 (the "
                                   "multi-GPU sharding of this path is a design note, not code)",
                          "n_gpus": args.gpus}))
        sys.exit(2)
    import torch
    pkg = importlib.import_module("artifex-assistantv5_amd")
    pkg.load_library()
    torch.cuda.set_device(0)

    t, m, n, k = 12, 1, 14336, 4096
    pool, raw = make_pool(pkg, t, n, k, args.pool, seed=1)
    if args.kernel_only:
        x = torch.from_numpy(pkg.quantize.synthetic_activations(m, k, seed=7)).cuda()
        y = torch.empty(m, n, device="cuda")
        a = torch.randn(16 * 2**20, device="cuda")
        b = torch.empty_like(a)
        torch.cuda.synchronize()
        for i in range(args.kernel_only):
            pkg.dispatch_matmul_gguf(x, pool[i % len(pool)], y, m, n, k, "profile")
        for _ in range(4):
            b.copy_(a)
        torch.cuda.synchronize()
        print(f"kernel-only: {args.kernel_only} launches + 4 x 64 MiB copies", flush=True)
        return
    head = matmul_case(pkg, t, m, n, k, pool, args.steps, args.warmup, eager=True)
    warm = matmul_case(pkg, t, m, n, k, pool[:1], args.steps, args.warmup)
    secondary = {"q4k_decode_m1_warm_gbs": round(warm["gbs"], 1),
                 "q4k_decode_m1_eager_ms_per_step": round(head["eager_ms"], 5)}
    secondary_cases(pkg, args, pool, secondary)
    gemm = matmul_case(pkg, t, 2048, n, k, pool[:2], 20, 2, xdtype="float16", replays=3)
    prefill = {"tflops": round(gemm["tflops"], 1), "peak": FP16_PEAK_TFLOPS, "unit": "TFLOP/s",
               "frac": round(gemm["tflops"] / FP16_PEAK_TFLOPS, 4),
               "ms_per_step": round(gemm["ms"], 4),
               "workload": "Q4_K dequant-GEMM M=2048 K=4096 N=14336, fp16 activations, f32 out",
               "timing": "median of 3 graph replays of 20 launches over 2 weight copies"}
    decode = None if args.no_decoder else decoder_case(pkg, args.decode_tokens)

    out = {
        "metric": "Q4_K GEMV weight GB/s (% HBM peak); prefill GEMM TFLOP/s; decode tok/s",
        "value": round(head["gbs"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(head["ms"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": ("q4_k weights (exact codes) x f32 activations entering the matrix cores as "
                  "f16 hi + lo parts of each power-of-two-scaled 256-element unit (22 "
                  "significant bits), f32 accumulate"),
        "data": "synthetic (seeded N(0,0.02) weights quantized to Q4_K, N(0,1) activations)",
        "config": {"workload": "Q4_K decode GEMV M=1 K=4096 N=14336 (FFN gate/up), cold weights",
                   "M": m, "K": k, "N": n, "weight_copies": args.pool,
                   "bytes_per_step": head["bytes"], "timing": "graph replay of the timed steps"},
        "roofline": {"bound": "hbm", "achieved": round(head["gbs"], 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(head["gbs"] / HBM_PEAK_GBS, 4),
                     "traffic": traffic_from_profile()},
        "prefill_gemm": prefill,
        "decode": decode,
        "secondary": secondary,
    }
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(pkg, raw, t, n, k, args.cpu_seconds)
        cpu["prefill"] = cpu_prefill_baseline(pkg, raw, t, n, k, m=256)
        if not args.no_decoder:
            cpu["decoder"] = cpu_decoder_baseline(pkg)
        out["cpu_baseline"] = cpu
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
