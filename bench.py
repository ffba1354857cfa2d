"""Benchmark of the GGUF Q4_K_M quantized-linear hot path on one MI355X.

Headline (one JSON line on stdout): Q4_K dequant-GEMM at the Qwen-Image DiT shape
M=4096, K=3072, N=12288 (bf16 activations, fp32 bias) in TFLOP/s, with its fraction of the
MI355X bf16 dense MFMA peak. A step is one tc_qlinear_forward call on inputs already
resident in HBM (one fused dequant-GEMM kernel launch), timed with HIP events on the launch
stream.

Secondary figures in the same line ("secondary"), one per BASELINE config:
* config 1: M=1024, N=K=3072 Q4_K + bias, TFLOP/s;
* config 2: text-encoder block (q,k,v,o 3584x3584 Q4_K, gate/up 3584->18944 Q4_K, down
  18944->3584 Q6_K) at M in {1, 8, 64, 256}: block time and weight+activation GB/s, rotating
  over 4 weight copies (644 MB > the 256 MB MALL) so that HBM serves the weights. The 7
  launches are replayed from a HIP graph (the eager figure, bound by host launch cost, is
  reported beside it);
* config 3: Qwen-Image MMDiT block linears (image + text streams, adaLN at M=1) at 1024 and
  4096 image tokens: ms per block;
  plus the batched adaLN modulation of all 60 blocks (both streams) as one stacked launch
  against 120 separate ones: ms and weight GB/s;
* config 4: LTX-style video DiT block linears: ms per block;
* config 5: config-3 linears with a batch of 4 images, each with its own runtime LoRA
  (rank 16/64): ms per block and the LoRA share;
* decode: Q4_K 9728x2560 and Q6_K 2560x9728 to bf16 (the tensors of the reference's published
  CPU decode times) on the device and with the product's host decoder on one thread;
* the CPU baseline (cpu_baseline): the oracle's C decode (row-parallel, like RowDecodePool)
  to fp32 + torch.matmul fp32 on this host's cores, for a bounded sample of the headline
  workload, scaled to one full call; plus the oracle's one-thread decode of the two tensors
  above (interleaved arms, medians, output SHA-256) and the host's physical core count.
`--only copy` runs a plain device copy of known size (the calibration kernel for the
FETCH_SIZE / WRITE_SIZE counters); `--only adaln` runs the stacked adaLN GEMV alone (config 3's
M = 1 HBM-bound case, for its traffic counters).

Every timed workload is first run untimed for about a quarter of a second, so that the GPU is at
its sustained clock (it holds ~1.86 GHz under the headline GEMM) before the W warmup steps; then
exactly K steps are timed. Without it a short W (the driver uses 5, ~1.5 ms of GPU work) leaves
the clock ramp inside the timed steps.

Synthetic data: W ~ N(0, 0.02) fp32 quantized on the device, X ~ N(0, 1) bf16, bias ~ N(0, 0.01).
"""
from __future__ import annotations

import argparse
import json
import os
import re
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


def settle(torch, fn, seconds=0.25):
    """Untimed: run the step until `seconds` of wall time have passed (sustained clock)."""
    torch.cuda.synchronize()
    t_end = time.perf_counter() + seconds
    i = 0
    while time.perf_counter() < t_end:
        for _ in range(8):
            fn(i)
            i += 1
        torch.cuda.synchronize()


def time_steps(torch, fn, steps, warmup):
    """Per-step GPU time (ms) from event pairs recorded on the launch stream, after settle()."""
    settle(torch, fn)
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


def physical_cores(cpus) -> int:
    """Distinct (package, core) pairs among the logical CPUs `cpus` (from /proc/cpuinfo)."""
    seen, cpu, phys = set(), None, None
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines() + [""]:
            key, _, val = line.partition(":")
            key, val = key.strip(), val.strip()
            if key == "processor":
                cpu = int(val)
            elif key == "physical id":
                phys = val
            elif key == "core id" and cpu in cpus:
                seen.add((phys, val))
    except OSError:
        return len(cpus)
    return len(seen) or len(cpus)


def decode_probe_1t(samples=8):
    """One-thread decode to bf16 of the two tensors the reference publishes CPU decode times for
    (Q4_K blk.0.ffn_gate 9728x2560 and Q6_K blk.0.ffn_down 2560x9728, gguf-k-simd-20261001.json),
    with the oracle's C decode on synthetic N(0, 0.02) weights: 3 warmups per arm, the arms
    interleaved in the reference probe's pattern (gguf_decode_probe.cpp:74-101), medians, and the
    SHA-256 of each output."""
    import hashlib

    import numpy as np

    from oracle import oracle
    rng = np.random.default_rng(3)
    arms = {}
    for name, typ, n, k in (("q4k_9728x2560", Q4K, 9728, 2560), ("q6k_2560x9728", Q6K, 2560, 9728)):
        arms[name] = (typ, n, k, oracle.quantize(typ, (rng.standard_normal((n, k)) * 0.02).astype(np.float32)))

    def run(name):
        typ, n, k, blocks = arms[name]
        t0 = time.perf_counter()
        out = oracle.decode_matrix(blocks, typ, n, k, dtype=oracle.DTYPE_BF16, threads=1)
        return (time.perf_counter() - t0) * 1e3, out
    for _ in range(3):
        for name in arms:
            run(name)
    times = {name: [] for name in arms}
    digests = {}
    a, b = list(arms)
    for i in range(samples):
        for name in ((a, b) if i % 4 < 2 else (b, a)):
            t, out = run(name)
            times[name].append(t)
            digests[name] = hashlib.sha256(out.tobytes()).hexdigest()
    return {f"{name}_bf16_ms": round(statistics.median(times[name]), 2) for name in arms} | {
        "samples": samples, "warmups_per_arm": 3, "threads": 1, "output_sha256": digests,
        "reference_m4max_ms": {"q4k_scalar": 49.872, "q4k_neon": 4.707, "q6k_scalar": 51.223, "q6k_neon": 5.566}}


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
    cpus = os.sched_getaffinity(0)
    return {
        "value": round(2.0 * m * n * k / t_call / 1e12, 4), "unit": "TFLOP/s", "cores": threads, "kind": "port",
        "physical_cores": physical_cores(cpus), "logical_cpus": len(cpus),
        "sample": (f"oracle C decode of the full Q4_K W[{n},{k}] to fp32 ({threads} row workers) + torch.matmul fp32 "
                   f"of {ms} of the {m} rows, medians of {len(dec_t)} runs, scaled to one full call"),
        "decode_ms": round(t_dec * 1e3, 2), "gemm_ms_per_256_rows": round(t_mm * 1e3, 2),
        "call_ms": round(t_call * 1e3, 1),
        "decode_1t": decode_probe_1t(),
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


def time_graph(torch, fn, steps, warmup, variants=1):
    """Capture fn(v) for v < variants into one HIP graph each (after eager warm-up: any
    workspace is allocated before capture); replay `steps` times with per-replay events."""
    for v in range(variants):
        for _ in range(max(1, warmup)):
            fn(v)
    settle(torch, fn)
    side = torch.cuda.Stream()
    graphs = []
    for v in range(variants):
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gr, stream=side):
            fn(v)
        graphs.append(gr)
    torch.cuda.synchronize()
    for i in range(warmup):
        graphs[i % variants].replay()
    torch.cuda.synchronize()
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    for i in range(steps):
        starts[i].record()
        graphs[i % variants].replay()
        ends[i].record()
    torch.cuda.synchronize()
    return [s.elapsed_time(e) for s, e in zip(starts, ends)]


def bench_config2(torch, gguf, qlinear, g, args, out, ms=(1, 8, 64, 256)):
    """Text-encoder block (7 linears), rotating 4 weight copies (> MALL)."""
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
        pe, _ = time_steps(torch, block, args.steps, args.warmup)
        pg = time_graph(torch, block, args.steps, args.warmup, variants=copies)
        te, tg = statistics.mean(pe), statistics.mean(pg)
        total = wbytes + sum(mm * (nn + kk) * 2 for _, _, nn, kk in shapes)
        gbs = total / (tg * 1e-3) / 1e9
        out[f"config2_block_m{mm}"] = {"ms": round(tg, 4), "GBps": round(gbs, 1), "frac_hbm": round(gbs / PEAK_HBM_GBS, 4),
                                       "bytes": total, "ms_eager": round(te, 4),
                                       "tflops": round(2 * mm * sum(nn * kk for _, _, nn, kk in shapes) / tg / 1e9, 2)}
        log(f"[config2 m={mm}] block {tg:.4f} ms (graph; eager {te:.4f} ms)  {gbs:.0f} GB/s "
            f"({gbs / PEAK_HBM_GBS:.1%} of 8 TB/s)")
        if mm in (1, 8, 64, 256):
            # The same block with the projections of a shared activation fused
            # (Weights::project_many: q/k/v, gate/up), as the text encoder calls them.
            o_qkv = [torch.empty((mm, 3584), dtype=torch.bfloat16, device="cuda") for _ in range(3)]
            o_gu = [torch.empty((mm, 18944), dtype=torch.bfloat16, device="cuda") for _ in range(2)]

            def fused(i, xs=xs, ys=ys, o_qkv=o_qkv, o_gu=o_gu):
                ls = lins[i % copies]
                qlinear.forward_many(ls[0:3], xs[3584], outs=o_qkv)
                ls[3](xs[3584], out=ys[3584])
                qlinear.forward_many(ls[4:6], xs[3584], outs=o_gu)
                ls[6](xs[18944], out=ys[3584])
            pf = time_graph(torch, fused, args.steps, args.warmup, variants=copies)
            tf = statistics.mean(pf)
            gbf = total / (tf * 1e-3) / 1e9
            out[f"config2_block_m{mm}_fused"] = {"ms": round(tf, 4), "GBps": round(gbf, 1),
                                                 "frac_hbm": round(gbf / PEAK_HBM_GBS, 4), "bytes": total}
            log(f"[config2 m={mm} fused qkv/gate-up] block {tf:.4f} ms (graph)  {gbf:.0f} GB/s "
                f"({gbf / PEAK_HBM_GBS:.1%} of 8 TB/s)")


def mmdit_linears(n_img, n_txt):
    """Qwen-Image-style MMDiT block (hidden 3072, MLP 12288): per stream q+k fused (Q4_K),
    v (Q6_K), out, MLP up/down (Q6_K on the image stream's down: half of ffn_down), and the
    adaLN modulation 3072->18432 at M=1. Entries: (name, type, n, k, m)."""
    lins = []
    for s, m in (("img", n_img), ("txt", n_txt)):
        lins += [(f"{s}.qk", Q4K, 6144, 3072, m), (f"{s}.v", Q6K, 3072, 3072, m), (f"{s}.out", Q4K, 3072, 3072, m),
                 (f"{s}.mlp_up", Q4K, 12288, 3072, m),
                 (f"{s}.mlp_down", Q6K if s == "img" else Q4K, 3072, 12288, m),
                 (f"{s}.adaln", Q4K, 18432, 3072, 1)]
    return lins


def ltx_linears(n_vid=4004, n_txt=128):
    """LTX-style video DiT block (hidden 4096, MLP 16384): qkv, out, ff up/down over the video
    tokens plus the text tokens, cross-attention kv at M=128; Q6_K interleaved (v part and ff
    down)."""
    m = n_vid + n_txt
    return [("qk", Q4K, 8192, 4096, m), ("v", Q6K, 4096, 4096, m), ("out", Q4K, 4096, 4096, m),
            ("ff_up", Q4K, 16384, 4096, m), ("ff_down", Q6K, 4096, 16384, m), ("xattn_kv", Q4K, 8192, 4096, n_txt)]


def stream_plan(lins):
    """The dual-stream schedule of an MMDiT block's linears (names "img.X" / "txt.X"): each
    pair of the same type and K as one grouped launch (qlinear.forward_group), the two streams'
    M = 1 adaLN modulations (one timestep embedding) as one fused GEMV (forward_many), the rest
    one launch each. Entries: ("group" | "many" | "one", indices into lins)."""
    names = {nm: i for i, (nm, *_rest) in enumerate(lins)}
    plan, done = [], set()
    for i, (nm, t, n, k, m) in enumerate(lins):
        if i in done:
            continue
        j = names.get("txt." + nm[4:]) if nm.startswith("img.") else None
        if j is not None and lins[j][1] == t and lins[j][3] == k:
            plan.append(("many" if m == 1 and lins[j][4] == 1 else "group", (i, j)))
            done.update((i, j))
        else:
            plan.append(("one", (i,)))
            done.add(i)
    return plan


def bench_block(torch, gguf, qlinear, g, args, name, lins, out, lora_images=0, streams=False):
    made = [make_linear(torch, gguf, qlinear, t, n, k, seed=200 + i)[0] for i, (_, t, n, k, _) in enumerate(lins)]
    xs = [torch.randn((m, k), generator=g, device="cuda").to(torch.bfloat16) for (_, _, _, k, m) in lins]
    ys = [torch.empty((m, n), dtype=torch.bfloat16, device="cuda") for (_, _, n, _, m) in lins]
    adapters = [() for _ in lins]
    if lora_images:
        rng_ranks = (16, 64, 16, 64)
        for i, (_, _, n, k, m) in enumerate(lins):
            if m < lora_images:
                continue
            per = m // lora_images
            ads = []
            for img in range(lora_images):
                r = rng_ranks[img % 4]
                a = (torch.randn((r, k), generator=g, device="cuda") / r ** 0.5).to(torch.bfloat16)
                b = (torch.randn((n, r), generator=g, device="cuda") * 0.01).to(torch.bfloat16)
                ads.append(qlinear.LoRAAdapter(a, b, 0.5 + img / 4.0, img * per, per))
            adapters[i] = tuple(ads)

    def block(_i):
        for lin, x, y, ad in zip(made, xs, ys, adapters):
            lin(x, ad, out=y)
    p = time_graph(torch, block, args.steps, args.warmup)
    t = statistics.mean(p)
    flops = sum(2.0 * m * n * k for (_, _, n, k, m) in lins)
    out[name] = {"ms": round(t, 4), "tflops": round(flops / t / 1e9, 2), "linears": len(lins)}
    log(f"[{name}] block {t:.4f} ms  {flops / t / 1e9:.1f} TFLOP/s over {len(lins)} linears")
    if streams:
        # The same linears with the image and text streams grouped (one adaLN embedding).
        plan = stream_plan(lins)
        launches = []
        for kind, idx in plan:
            if kind == "group":
                launches.append(lambda i=idx: qlinear.forward_group([made[j] for j in i], [xs[j] for j in i],
                                                                    outs=[ys[j] for j in i]))
            elif kind == "many":
                launches.append(lambda i=idx: qlinear.forward_many([made[j] for j in i], xs[i[0]],
                                                                   outs=[ys[j] for j in i]))
            else:
                launches.append(lambda i=idx: made[i[0]](xs[i[0]], out=ys[i[0]]))
        grouped = sum(1 for kind, idx in plan if kind == "group" and
                      qlinear.forward_group([made[j] for j in idx], [xs[j] for j in idx],
                                            outs=[ys[j] for j in idx])[1])

        def block_streams(_i):
            for launch in launches:
                launch()
        p2 = time_graph(torch, block_streams, args.steps, args.warmup)
        t2 = statistics.mean(p2)
        out[name].update({"ms_streams_grouped": round(t2, 4), "tflops_streams_grouped": round(flops / t2 / 1e9, 2),
                          "grouped_launches": grouped})
        log(f"[{name}] streams grouped ({grouped} grouped GEMMs, adaLN fused): block {t2:.4f} ms  "
            f"{flops / t2 / 1e9:.1f} TFLOP/s")
    return t


def bench_adaln(torch, gguf, qlinear, g, args, out, blocks=60):
    """Batched adaLN modulation of a 60-block MMDiT: every block's image- and text-stream
    modulation (3072 -> 18432 Q4_K, M = 1) reads the same timestep embedding; stacked
    (Weights.bind_stacked) they run as one GEMV launch over 2 * 60 * 18432 rows (3.8 GB of
    weights), against the same 120 projections launched one by one from a HIP graph."""
    n, k = 18432, 3072
    W = qlinear.Weights()
    names = []
    for b in range(blocks):
        for s in ("img", "txt"):
            lin, blk = make_linear(torch, gguf, qlinear, Q4K, n, k, seed=5000 + 2 * b + (s == "txt"))
            W.bind(f"blocks.{b}.{s}_mod", blk, Q4K, n, k, lin.bias)
            del lin
            names.append(f"blocks.{b}.{s}_mod")
    W.bind_stacked("modulation", names)
    x = torch.randn((1, k), generator=g, device="cuda").to(torch.bfloat16)
    stacked = W._linears["modulation"]
    y = torch.empty((1, stacked.n), dtype=torch.bfloat16, device="cuda")
    wbytes = len(names) * n * k // 256 * BLOCK[Q4K]
    p1, _ = time_steps(torch, lambda i: stacked(x, out=y), args.steps, args.warmup)
    members = [W._linears[nm] for nm in names]
    ys = [y[:, i * n:(i + 1) * n] for i in range(len(names))]
    outs = [torch.empty((1, n), dtype=torch.bfloat16, device="cuda") for _ in names]

    def each(_i):
        for lin, o in zip(members, outs):
            lin(x, out=o)
    p2 = time_graph(torch, each, max(5, args.steps // 5), max(1, args.warmup // 5))
    t1, t2 = statistics.mean(p1), statistics.mean(p2)
    out["config3_adaln_60_blocks"] = {"ms_stacked": round(t1, 4), "GBps_stacked": round(wbytes / t1 / 1e6, 1),
                                      "frac_hbm": round(wbytes / t1 / 1e6 / PEAK_HBM_GBS, 4),
                                      "ms_per_projection_launches": round(t2, 4),
                                      "GBps_per_projection_launches": round(wbytes / t2 / 1e6, 1),
                                      "weight_bytes": wbytes}
    log(f"[adaLN x{len(names)}] stacked {t1:.4f} ms ({wbytes / t1 / 1e6:.0f} GB/s); "
        f"{len(names)} launches {t2:.4f} ms ({wbytes / t2 / 1e6:.0f} GB/s)")
    del ys


def bench_decode(torch, gguf, args, out):
    """Decode to bf16 of the two tensors the reference publishes CPU decode times for (Q4_K
    9728x2560, Q6_K 2560x9728): on the device (tc_gguf_decode_device, synchronous: each step
    includes the host read-back of the error word) and with the product's host decoder on one
    thread (tc_gguf_decode_host, median of 5 after one warmup)."""
    import numpy as np
    for name, typ, n, k in (("q4k_9728x2560", Q4K, 9728, 2560), ("q6k_2560x9728", Q6K, 2560, 9728)):
        g = torch.Generator(device="cuda").manual_seed(n + k)
        blocks = gguf.quantize(torch.randn((n, k), generator=g, device="cuda") * 0.02, typ)
        dst = torch.empty((n, k), dtype=torch.bfloat16, device="cuda")
        pm = gguf.PackedMatrix(blocks, typ, n, k)
        tgt = gguf.DecodeTarget(dst, gguf.DecodeDType.bf16, 2 * k, 2)
        per, _ = time_steps(torch, lambda i: gguf.decode_into(pm, gguf.DecodeSlice(0, n, 0, k), tgt),
                            args.steps, args.warmup)
        t = statistics.median(per)
        nbytes = blocks.numel() + 2 * n * k
        host_blocks = blocks.cpu().numpy()
        host_out = np.empty((n, k), dtype=np.uint16)
        hp = gguf.PackedMatrix(host_blocks, typ, n, k)
        ht = gguf.DecodeTarget(host_out, gguf.DecodeDType.bf16, 2 * k, 2)
        host = []
        for i in range(6):
            t0 = time.perf_counter()
            gguf.decode_cpu_into(hp, gguf.DecodeSlice(0, n, 0, k), ht)
            if i:
                host.append((time.perf_counter() - t0) * 1e3)
        same = bool(np.array_equal(host_out, dst.cpu().view(torch.int16).numpy().view(np.uint16)))
        out[f"decode_{name}_bf16"] = {"device_ms": round(t, 4), "device_GBps": round(nbytes / t / 1e6, 1),
                                      "host_1t_ms": round(statistics.median(host), 2), "host_equals_device": same}
        log(f"[decode {name}] device {t:.4f} ms ({nbytes / t / 1e6:.0f} GB/s incl. the error read-back); "
            f"host 1 thread {statistics.median(host):.1f} ms; outputs equal: {same}")


def bench_copy(torch, args, out, nbytes=1 << 30):
    """Plain device copy of known size: the calibration kernel for the HBM byte counters."""
    src = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    dst = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    p, _ = time_steps(torch, lambda i: dst.copy_(src), args.steps, args.warmup)
    t = statistics.mean(p)
    out["copy_1GiB"] = {"ms": round(t, 4), "bytes_read": nbytes, "bytes_written": nbytes,
                        "GBps": round(2 * nbytes / t / 1e6, 1)}
    log(f"[copy] {nbytes} B: {t:.4f} ms  {2 * nbytes / t / 1e6:.0f} GB/s (read + write)")


def traffic_from_profile():
    """HBM bytes per headline launch measured by FETCH_SIZE + WRITE_SIZE (scaled by the copy
    calibration), as recorded in profiles/gemm_q4k_northstar.md; None when absent."""
    path = ROOT / "profiles" / "gemm_q4k_northstar.md"
    if not path.exists():
        return None
    m = re.search(r"^traffic_bytes_per_launch:\s*([0-9]+)", path.read_text(), re.M)
    return int(m.group(1)) if m else None


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--only", choices=["headline", "config1", "config2", "config3", "config4", "config5", "decode",
                                       "copy", "adaln"],
                    default=None, help="run one workload only (profiling)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build runs the quantized-linear path on a single MI355X "
              f"(--gpus {args.gpus} is not supported: no multi-GPU path is built)", file=sys.stderr)
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
    if want("config3"):
        bench_block(torch, gguf, qlinear, g, args, "config3_mmdit_block_img1024", mmdit_linears(1024, 256), secondary,
                    streams=True)
        bench_block(torch, gguf, qlinear, g, args, "config3_mmdit_block_img4096", mmdit_linears(4096, 256), secondary,
                    streams=True)
        bench_adaln(torch, gguf, qlinear, g, args, secondary)
    if want("config4"):
        bench_block(torch, gguf, qlinear, g, args, "config4_ltx_block", ltx_linears(), secondary)
    if want("config5"):
        lins = [(nm, t, n, k, 4 * m if m > 1 else 1) for (nm, t, n, k, m) in mmdit_linears(1280, 0) if m > 0]
        t0 = bench_block(torch, gguf, qlinear, g, args, "config5_mmdit_4img_no_lora", lins, secondary)
        t1 = bench_block(torch, gguf, qlinear, g, args, "config5_mmdit_4img_lora", lins, secondary, lora_images=4)
        secondary["config5_mmdit_4img_lora"]["lora_share"] = round((t1 - t0) / t1, 4)
    if want("decode"):
        bench_decode(torch, gguf, args, secondary)
    if args.only == "copy":
        bench_copy(torch, args, secondary)
    if args.only == "adaln":
        bench_adaln(torch, gguf, qlinear, g, args, secondary)

    cpu = None
    if not args.no_cpu_baseline and want("headline"):
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
                     "frac": round(tflops / PEAK_BF16_TFLOPS, 4), "traffic": traffic_from_profile(),
                     "kernel": "k_gemm<Q4_K, unsplit, 256-row tile> (bias in the epilogue)", "flops_per_launch": flops,
                     "algorithmic_bytes_per_launch": n * k // 256 * BLOCK[Q4K] + 2 * m * k + 2 * m * n + 4 * n},
        "cpu_baseline": cpu,
        "secondary": secondary,
    }
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
