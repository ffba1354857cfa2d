"""Benchmark of the GGUF Q4_K_M quantized-linear hot path on one MI355X.

Headline (one JSON line on stdout): Q4_K dequant-GEMM at the Qwen-Image DiT shape
M=4096, K=3072, N=12288 (bf16 activations, fp32 bias) in TFLOP/s, with its fraction of the
MI355X bf16 dense MFMA peak. A step is one tc_qlinear_forward call on inputs already
resident in HBM (one fused dequant-GEMM kernel launch).

Secondary figures in the same line ("secondary"):
* config 1 (M=1024, N=K=3072 Q4_K + bias) TFLOP/s;
* config 2 text-encoder block at M=1 (q,k,v,o 3584x3584 Q4_K, gate/up 3584->18944 Q4_K,
  down 18944->3584 Q6_K): weight GB/s and fraction of 8 TB/s, rotating over 4 weight copies
  (644 MB > the 256 MB MALL) so that HBM, not the cache, serves the weights;
* the CPU baseline (cpu_baseline): the oracle's C decode (row-parallel, like RowDecodePool)
  to fp32 + torch.matmul fp32 on this host's cores, for a bounded sample of the headline
  workload, scaled to one full call.

Synthetic data: W ~ N(0, 0.02) fp32 quantized on the device, X ~ N(0, 1) bf16, bias ~ N(0, 0.01).
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

PEAK_BF16_TFLOPS = 2500.0   # MI355X dense bf16 MFMA (vendor)
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E (vendor)
Q4K, Q6K = 12, 14
BLOCK = {Q4K: 144, Q6K: 210}


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def make_linear(torch, gguf, qlinear, typ, n, k, seed, bias=True):
    g = torch.Generator(device="cuda").manual_seed(seed)
    w = torch.randn((n, k), generator=g, device="cuda") * 0.02
    blocks = gguf.quantize(w.contiguous(), typ)
    del w
    b = (torch.randn((n,), generator=g, device="cuda") * 0.01) if bias else None
    return qlinear.QuantizedLinear(blocks, typ, n, k, b), blocks


def time_steps(torch, fn, steps, warmup):
    """Per-step GPU time (ms) from event pairs recorded on the launch stream."""
    for _ in range(warmup):
        fn(0)
    torch.cuda.synchronize()
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    t0 = time.perf_counter()
    for i in range(steps):
        starts[i].record()
        fn(i)
        ends[i].record()
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) * 1e3
    per = [s.elapsed_time(e) for s, e in zip(starts, ends)]
    return per, wall


def cpu_baseline(m, n, k, threads, budget_s=12.0):
    """Oracle decode (C, `threads` row workers) + torch.matmul fp32 on CPU, scaled to one call."""
    import numpy as np
    import torch

    from oracle import oracle
    torch.set_num_threads(threads)
    rng = np.random.default_rng(0)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    blocks = oracle.quantize(Q4K, w)
    ms = 256
    x = torch.from_numpy(oracle.bf16_to_f32(oracle.bf16_bits(rng.standard_normal((ms, k)).astype(np.float32))))
    dec_t, mm_t = [], []
    t_end = time.perf_counter() + budget_s
    it = 0
    while it < 3 or (time.perf_counter() < t_end and it < 12):
        t0 = time.perf_counter()
        wd = oracle.decode_matrix(blocks, Q4K, n, k, threads=threads)
        t1 = time.perf_counter()
        _ = x @ torch.from_numpy(wd).T
        t2 = time.perf_counter()
        if it >= 1:  # first iteration is the warm-up
            dec_t.append(t1 - t0)
            mm_t.append(t2 - t1)
        it += 1
    t_dec, t_mm = statistics.median(dec_t), statistics.median(mm_t)
    t_call = t_dec + t_mm * (m / ms)
    return {
        "value": round(2.0 * m * n * k / t_call / 1e12, 4), "unit": "TFLOP/s", "cores": threads, "kind": "port",
        "sample": (f"oracle C decode of the full Q4_K W[{n},{k}] to fp32 ({threads} row workers) + torch.matmul fp32 "
                   f"of {ms} of the {m} rows, medians of {len(dec_t)} runs, scaled to one full call"),
        "decode_ms": round(t_dec * 1e3, 2), "gemm_ms_per_256_rows": round(t_mm * 1e3, 2),
        "call_ms": round(t_call * 1e3, 1),
    }


def bench_headline(torch, gguf, qlinear, g, args, dev_name):
    m, k, n = 4096, 3072, 12288
    lin, _ = make_linear(torch, gguf, qlinear, Q4K, n, k, seed=0)
    x = torch.randn((m, k), generator=g, device="cuda").to(torch.bfloat16)
    y = torch.empty((m, n), dtype=torch.bfloat16, device="cuda")
    per, wall = time_steps(torch, lambda i: lin(x, out=y), args.steps, args.warmup)
    kernel_ms = statistics.mean(per)
    tflops = 2.0 * m * n * k / (kernel_ms * 1e-3) / 1e12
    log(f"[headline] {dev_name}: gemm {m}x{n}x{k} mean {kernel_ms:.4f} ms  median {statistics.median(per):.4f} ms  "
        f"-> {tflops:.1f} TFLOP/s ({tflops / PEAK_BF16_TFLOPS:.1%} of bf16 peak); wall {wall / args.steps:.4f} ms/step")
    return kernel_ms, tflops


def bench_config1(torch, gguf, qlinear, g, args, out):
    lin1, _ = make_linear(torch, gguf, qlinear, Q4K, 3072, 3072, seed=0)
    x1 = torch.randn((1024, 3072), generator=g, device="cuda").to(torch.bfloat16)
    y1 = torch.empty((1024, 3072), dtype=torch.bfloat16, device="cuda")
    p1, _ = time_steps(torch, lambda i: lin1(x1, out=y1), args.steps, args.warmup)
    t1 = statistics.mean(p1)
    out["config1_gemm_1024x3072x3072"] = {"ms": round(t1, 4), "tflops": round(2 * 1024 * 3072 * 3072 / t1 / 1e9, 2)}
    log(f"[config1] {t1:.4f} ms {out['config1_gemm_1024x3072x3072']['tflops']} TFLOP/s")


def bench_config2(torch, gguf, qlinear, g, args, out, ms=(1, 8)):
    """Text-encoder block (7 linears) at small M, rotating 4 weight copies (> MALL)."""
    shapes = [("q", Q4K, 3584, 3584), ("k", Q4K, 3584, 3584), ("v", Q4K, 3584, 3584), ("o", Q4K, 3584, 3584),
              ("gate", Q4K, 18944, 3584), ("up", Q4K, 18944, 3584), ("down", Q6K, 3584, 18944)]
    copies = 4
    lins = [[make_linear(torch, gguf, qlinear, t, nn, kk, seed=100 + 10 * c + i, bias=False)[0]
             for i, (_, t, nn, kk) in enumerate(shapes)] for c in range(copies)]
    wbytes = sum(nn * kk // 256 * BLOCK[t] for _, t, nn, kk in shapes)
    for mm in ms:
        xs = {kk: torch.randn((mm, kk), generator=g, device="cuda").to(torch.bfloat16) for kk in (3584, 18944)}
        ys = {nn: torch.empty((mm, nn), dtype=torch.bfloat16, device="cuda") for nn in (3584, 18944)}

        def block(i, xs=xs, ys=ys):
            for lin_i, (_, _, nn, kk) in zip(lins[i % copies], shapes):
                lin_i(xs[kk], out=ys[nn])
        pb, _ = time_steps(torch, block, args.steps, args.warmup)
        tb = statistics.mean(pb)
        total = wbytes + sum(mm * (nn + kk) * 2 for _, _, nn, kk in shapes)
        gbs = total / (tb * 1e-3) / 1e9
        out[f"config2_block_m{mm}"] = {"ms": round(tb, 4), "GBps": round(gbs, 1),
                                       "frac_hbm": round(gbs / PEAK_HBM_GBS, 4), "bytes": total}
        log(f"[config2 m={mm}] block {tb:.4f} ms  {gbs:.0f} GB/s ({gbs / PEAK_HBM_GBS:.1%} of 8 TB/s)")


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--only", choices=["headline", "config1", "config2"], default=None,
                    help="run one workload only (profiling)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build runs the quantized-linear path on a single MI355X "
              f"(--gpus {args.gpus} is not supported; sharding is described in DESIGN.md)", file=sys.stderr)
        return 2

    import torch

    from turbocider_amd import gguf, qlinear
    torch.manual_seed(0)
    dev_name = torch.cuda.get_device_name(0)
    g = torch.Generator(device="cuda").manual_seed(1)
    want = (lambda name: args.only is None or args.only == name)

    m, k, n = 4096, 3072, 12288
    flops = 2.0 * m * n * k
    kernel_ms = tflops = float("nan")
    if want("headline"):
        kernel_ms, tflops = bench_headline(torch, gguf, qlinear, g, args, dev_name)
    secondary = {}
    if want("config1"):
        bench_config1(torch, gguf, qlinear, g, args, secondary)
    if want("config2"):
        bench_config2(torch, gguf, qlinear, g, args, secondary)

    cpu = None
    if not args.no_cpu_baseline:
        threads = len(os.sched_getaffinity(0))
        cpu = cpu_baseline(m, n, k, threads)
        log(f"[cpu] {cpu}")

    result = {
        "metric": "Q4_K_M dequant-GEMM TFLOP/s (M=4096, K=3072, N=12288)",
        "value": round(tflops, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(kernel_ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: W~N(0,0.02) fp32 quantized to Q4_K on device, X~N(0,1) bf16, bias~N(0,0.01)",
        "config": {"workload": "Qwen-Image DiT linear, Q4_K dequant-GEMM + bias", "m": m, "k": k, "n": n,
                   "weight_type": "Q4_K", "device": dev_name},
        "roofline": {"bound": "mfma", "achieved": round(tflops, 2), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(tflops / PEAK_BF16_TFLOPS, 4), "traffic": None,
                     "kernel": "k_gemm<12,true>", "flops_per_launch": flops},
        "cpu_baseline": cpu,
        "secondary": secondary,
    }
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
