"""Benchmark of the GGUF dequant-matmul path on one MI355X.

Headline workload: Q4_K decode GEMV, M=1, K=4096, N=14336 (FFN gate/up), fp32
activations ~N(0,1), weights ~N(0,0.02) quantized to Q4_K.  One step = one
GEMV over one activation vector.  Weights are cold: every step reads a
different one of P distinct copies of the weight (P * 33 MB > 512 MB, more
than the 256 MB Infinity Cache), so the bytes come from HBM.

Prints ONE JSON line.  ``value`` = algorithmic bytes per step (weights + x +
y) / wall time per step, measured with HIP events on the stream the kernels
run on.  ``secondary`` holds the other configurations of the path.
``cpu_baseline`` = the CPU oracle (numpy dequant + torch fp32 matmul, all
host cores) on the same workload.
"""

from __future__ import annotations

import argparse
import importlib
import json
import os
import platform
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
FP16_PEAK_TFLOPS = 2500.0
Q4K_BYTES = 144 / 256
Q6K_BYTES = 210 / 256
Q8_BYTES = 34 / 32


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--pool", type=int, default=17, help="distinct weight copies (cold weights)")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--no-secondary", action="store_true")
    p.add_argument("--only", default="", help="comma list of secondary configs to run")
    return p.parse_args()


def time_steps(step, steps, warmup):
    """Run ``step(i)`` warmup + steps times; returns ms per timed step (HIP events)."""
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


def make_pool(pkg, t, n, k, copies, seed, quantized=True):
    """``copies`` distinct device copies of one quantized weight (row layout)."""
    import torch
    if quantized:
        w = pkg.quantize.synthetic_weight(n, k, seed=seed)
        raw = pkg.quantize.quantize(w, t)
        base = pkg.repack_gguf_for_gpu(t, raw, n, k, device="cuda")
    else:  # random block bytes with finite scales, drawn on the device
        block, size = {8: (32, 34), 12: (256, 144), 14: (256, 210)}[t]
        g = torch.Generator(device="cuda").manual_seed(seed)
        rawd = torch.randint(0, 256, (n * (k // block) * size,), dtype=torch.uint8, device="cuda",
                             generator=g)
        blocks = rawd.view(-1, size)
        for o in {8: [0], 12: [0, 2], 14: [208]}[t]:
            v = (torch.rand(blocks.shape[0], device="cuda", generator=g) * 0.003 + 0.0005).half()
            blocks[:, o:o + 2] = v.view(torch.uint8).view(-1, 2)
        base = pkg.repack_gguf_for_gpu(t, rawd, n, k)
        raw = None
    pool = [base] + [pkg.GGUFWeight(base.data.clone(), t, n, k) for _ in range(copies - 1)]
    return pool, raw


def gemv_case(pkg, t, m, n, k, pool, steps, warmup, xdtype="float32"):
    import torch
    x = torch.from_numpy(pkg.quantize.synthetic_activations(m, k, seed=7)).cuda().to(
        getattr(torch, xdtype))
    y = torch.empty(m, n, device="cuda")
    P = len(pool)

    def step(i):
        pkg.dispatch_matmul_gguf(x, pool[i % P], y, m, n, k, "bench")

    ms = time_steps(step, steps, warmup)
    wbytes = pool[0].n * pkg.raw_row_bytes(t, k)
    xbytes = m * k * x.element_size()
    algo = wbytes + xbytes + m * n * 4
    return {"ms": ms, "bytes": algo, "gbs": algo / (ms * 1e-3) / 1e9,
            "tflops": 2.0 * m * n * k / (ms * 1e-3) / 1e12}


def cpu_baseline(pkg, raw, t, n, k, m=1):
    """Oracle CPU path: numpy dequant (bit-exact restatement) + torch fp32 matmul."""
    import torch
    from oracle import gguf_ref as ref
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    x = torch.from_numpy(pkg.quantize.synthetic_activations(m, k, seed=7))
    times, t_deq, t_mm = [], [], []
    for it in range(7):
        t0 = time.perf_counter()
        w = torch.from_numpy(ref.dequant_rows(t, raw, n, k))
        t1 = time.perf_counter()
        torch.matmul(x, w.T)
        t2 = time.perf_counter()
        if it >= 2:
            times.append(t2 - t0)
            t_deq.append(t1 - t0)
            t_mm.append(t2 - t1)
    tot = float(np.median(times))
    wbytes = n * pkg.raw_row_bytes(t, k)
    return {
        "value": round(wbytes / tot / 1e9, 3),
        "unit": "GB/s",
        "cores": cores,
        "kind": "port",
        "sample": (f"Q4_K M={m} K={k} N={n}: numpy dequant to fp32 + torch.matmul fp32, "
                   f"median of 5 after 2 warm-ups; dequant {np.median(t_deq) * 1e3:.1f} ms, "
                   f"matmul {np.median(t_mm) * 1e3:.1f} ms, total {tot * 1e3:.1f} ms"),
        "cpu": platform.processor() or platform.machine(),
        "torch_threads": torch.get_num_threads(),
    }


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only; --gpus must be 1",
                          "n_gpus": args.gpus}))
        sys.exit(2)
    import torch
    pkg = importlib.import_module("artifex-assistantv5_amd")
    pkg.load_library()
    torch.cuda.set_device(0)

    t, m, n, k = 12, 1, 14336, 4096
    pool, raw = make_pool(pkg, t, n, k, args.pool, seed=1)
    head = gemv_case(pkg, t, m, n, k, pool, args.steps, args.warmup)
    # warm (cache-resident) figure for reference: one weight copy
    warm = gemv_case(pkg, t, m, n, k, pool[:1], args.steps, args.warmup)
    kernel_gbs = head["gbs"]

    secondary = {"q4k_gemv_m1_warm_gbs": round(warm["gbs"], 1)}
    only = set(filter(None, args.only.split(",")))

    def want(name):
        return not args.no_secondary and (not only or name in only)

    if want("gemv_batch"):
        for mm in (8, 32):
            r = gemv_case(pkg, t, mm, n, k, pool, max(20, args.steps // 4), 5)
            secondary[f"q4k_gemv_m{mm}_gate_up_gbs"] = round(r["gbs"], 1)
    if want("down"):
        dpool, _ = make_pool(pkg, t, 4096, 14336, args.pool, seed=2)
        for mm in (1, 8, 32):
            r = gemv_case(pkg, t, mm, 4096, 14336, dpool, max(20, args.steps // 4), 5)
            secondary[f"q4k_gemv_m{mm}_down_gbs"] = round(r["gbs"], 1)
        del dpool
    if want("prefill"):
        for mm, nn in ((512, 4096), (2048, 14336), (8192, 4096)):
            ppool = pool[:2] if nn == 14336 else make_pool(pkg, t, nn, 4096, 2, seed=3)[0]
            r = gemv_case(pkg, t, mm, nn, 4096, ppool, 10, 2, xdtype="float16")
            secondary[f"q4k_gemm_m{mm}_n{nn}_tflops"] = round(r["tflops"], 1)
            secondary[f"q4k_gemm_m{mm}_n{nn}_frac_fp16_peak"] = round(r["tflops"] / FP16_PEAK_TFLOPS, 4)
    if want("q8"):
        qpool, _ = make_pool(pkg, 8, 4096, 4096, 32, seed=4)
        r = gemv_case(pkg, 8, 1, 4096, 4096, qpool, args.steps, args.warmup)
        secondary["q8_0_gemv_m1_gbs"] = round(r["gbs"], 1)
        del qpool
    if want("lm_head"):
        lpool, _ = make_pool(pkg, 14, 151936, 4096, 2, seed=5, quantized=False)
        r = gemv_case(pkg, 14, 1, 151936, 4096, lpool, 20, 3)
        secondary["q6k_lm_head_m1_gbs"] = round(r["gbs"], 1)
        secondary["q6k_lm_head_weights"] = "random blocks with finite f16 scales"
        del lpool

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
        "dtype": "q4_k weights x f32 activations, f32 accumulate",
        "data": "synthetic (seeded N(0,0.02) weights quantized to Q4_K, N(0,1) activations)",
        "config": {"workload": "Q4_K decode GEMV M=1 K=4096 N=14336 (FFN gate/up), cold weights",
                   "M": m, "K": k, "N": n, "weight_copies": args.pool,
                   "bytes_per_step": head["bytes"]},
        "roofline": {"bound": "hbm", "achieved": round(kernel_gbs, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(kernel_gbs / HBM_PEAK_GBS, 4), "traffic": None},
        "secondary": secondary,
    }
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline(pkg, raw, t, n, k)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
