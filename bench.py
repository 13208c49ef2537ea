#!/usr/bin/env python3
"""Benchmark of the hot path on one MI355X.

The headline line times BASELINE config 2 -- the bf16 GEMM C[4096,12288] = A[4096,4096] @
B[4096,12288], fp32 accumulation, bf16 C (Qwen3-8B gate/up projection shape) -- as K back-to-back
launches over inputs resident in HBM, bracketed by torch.cuda.synchronize().  ``value`` is TFLOP/s
(2*M*N*K flops per step).  The same JSON line carries, under ``kernels``, each other BASELINE config
measured the same way (RMSNorm GB/s, fp8 GEMM TFLOP/s, flash-attention TFLOP/s, Qwen3-8B layer
latency) and the single-token decode path (the decode layer's largest GEMV and the decode attention
in GB/s, the 8-launch decode layer's latency), each with its roofline fraction, and
``cpu_baseline`` times the CPU golden (the oracle, torch-CPU) on this host's cores: the headline's
figure at top level and, under ``configs``, one entry per BASELINE config (a bounded sample of each
workload, on all host threads and on one thread).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--only gemm_bf16,...]
       python bench.py --decode-sweep   (decode attention over cache lengths; its own JSON line)
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO / "pytorchsim-triton-backend_amd"))
sys.path.insert(0, str(REPO))

PEAK_BF16_TFLOPS = 2500.0   # MI355X dense bf16 MFMA
PEAK_FP8_TFLOPS = 5000.0    # MI355X dense fp8 MFMA
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


SETTLE_S = 0.3   # untimed run-in before the warmup steps (set from --settle)


def timed(fn, steps: int, warmup: int):
    """Run fn() back to back for SETTLE_S seconds (the GPU raises its clock over the first ~50 ms of
    sustained load; the timed steps should see the sustained clock, not the ramp), then warmup
    times, then time `steps` launches with HIP events on torch's current stream (the stream every
    ptb_amd op launches on).  Returns (ms per step, wall ms per step)."""
    import torch

    t_end = time.perf_counter() + SETTLE_S
    while time.perf_counter() < t_end:
        for _ in range(4):
            fn()
        torch.cuda.synchronize()
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record()
    for _ in range(steps):
        fn()
    stop.record()
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) * 1e3 / steps
    return start.elapsed_time(stop) / steps, wall


def timed_graph(fn, calls: int, replays: int):
    """The device time of fn() by HIP-graph replay: `calls` consecutive calls captured once (so a
    function that cycles through input copies keeps reading HBM), the graph replayed for SETTLE_S
    seconds, then `replays` replays timed with HIP events.  Without the host's per-launch cost this
    is what a serving loop that replays a captured step sees.  Returns ms per call."""
    import torch

    cur = torch.cuda.current_stream()
    side = torch.cuda.Stream()
    side.wait_stream(cur)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side), torch.cuda.graph(g, stream=side):
        for _ in range(calls):
            fn()
    cur.wait_stream(side)
    g.replay()
    torch.cuda.synchronize()
    t_end = time.perf_counter() + SETTLE_S
    while time.perf_counter() < t_end:
        g.replay()
        torch.cuda.synchronize()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(replays):
        g.replay()
    stop.record()
    torch.cuda.synchronize()
    return start.elapsed_time(stop) / (replays * calls)


def bench_gemm_bf16(steps, warmup):
    import torch
    from ptb_amd import ops

    m, k, n = 4096, 4096, 12288
    g = torch.Generator().manual_seed(0)
    a = (torch.randn(m, k, generator=g) / 64.0).to(torch.bfloat16).cuda()
    b = (torch.randn(k, n, generator=g) / 64.0).to(torch.bfloat16).cuda()
    c = torch.empty(m, n, dtype=torch.bfloat16, device="cuda")
    ms, wall = timed(lambda: ops.gemm(a, b, out=c), steps, warmup)
    flops = 2.0 * m * n * k
    tf = flops / (ms * 1e-3) / 1e12
    return {
        "name": "gemm_bf16", "config": "BASELINE config 2: bf16 [4096x4096]@[4096x12288]",
        "us": ms * 1e3, "wall_us": wall * 1e3, "tflops": tf,
        "roofline": {"bound": "mfma", "achieved": tf, "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                     "frac": tf / PEAK_BF16_TFLOPS},
        "flops": flops,
    }


def bench_rmsnorm(steps, warmup):
    import torch
    from ptb_amd import ops

    rows, cols = 2048, 4096
    copies = 16   # 16 x 33.5 MB cycles through > the 256 MB last-level cache: every call reads HBM
    g = torch.Generator().manual_seed(0)
    xs = [torch.randn(rows, cols, generator=g).to(torch.bfloat16).cuda() for _ in range(copies)]
    w = (torch.randn(cols, generator=g) * 0.02 + 1.0).cuda()
    ys = [torch.empty_like(x) for x in xs]
    it = [0]

    def step():
        i = it[0] % copies
        it[0] += 1
        ops.rmsnorm(xs[i], w, 1e-6, out=ys[i])

    ms, wall = timed(step, steps * 4, warmup)
    nbytes = 2 * rows * cols * 2 + cols * 4
    gbs = nbytes / (ms * 1e-3) / 1e9

    # the practical ceiling: a device copy (hipMemcpyAsync) of the same bytes, x -> y, same cycling
    def copy_step():
        i = it[0] % copies
        it[0] += 1
        ys[i].copy_(xs[i])

    copy_ms, _ = timed(copy_step, steps * 4, warmup)

    # the library's own stream of the same bytes: ptb_add_scalar_bf16 reads and writes 2 B per
    # element over the same [2048, 4096] bf16 tensors, same cycling
    def same_bytes_step():
        i = it[0] % copies
        it[0] += 1
        ops.add_scalar(xs[i], 1.0, out=ys[i])

    same_ms, _ = timed(same_bytes_step, steps * 4, warmup)
    return {"name": "rmsnorm", "config": "BASELINE config 1: x bf16 [2048x4096], w fp32",
            "us": ms * 1e3, "wall_us": wall * 1e3, "gbs": gbs,
            "roofline": {"bound": "hbm", "achieved": gbs, "peak": PEAK_HBM_GBS, "unit": "GB/s",
                         "frac": gbs / PEAK_HBM_GBS},
            "device_copy_us": copy_ms * 1e3, "vs_device_copy": copy_ms / ms,
            "same_bytes_us": same_ms * 1e3, "vs_same_bytes": same_ms / ms,
            "same_bytes_frac": (nbytes - cols * 4) / (same_ms * 1e-3) / 1e9 / PEAK_HBM_GBS}


def bench_gemm_fp8(steps, warmup):
    import torch
    from ptb_amd import ops

    m, k, n = 2048, 12288, 4096
    g = torch.Generator().manual_seed(0)
    x = torch.randn(m, k, generator=g).to(torch.bfloat16).cuda()
    w = (torch.randn(k, n, generator=g) * 0.02).cuda()
    wq_t, sw = ops.quant_weight_e4m3(w)
    xq, sx = ops.quant_rows_e4m3(x)
    c = torch.empty(m, n, dtype=torch.bfloat16, device="cuda")
    ms, wall = timed(lambda: ops.gemm_fp8(xq, sx, wq_t, sw, out=c), steps, warmup)
    qms, _ = timed(lambda: ops.quant_rows_e4m3(x), steps, warmup)
    flops = 2.0 * m * n * k
    tf = flops / (ms * 1e-3) / 1e12
    qbytes = m * k * 2 + m * k + m * 4
    return {"name": "gemm_fp8", "config": "BASELINE config 4: e4m3 [2048x12288]@[12288x4096] + scales",
            "us": ms * 1e3, "wall_us": wall * 1e3, "tflops": tf,
            "roofline": {"bound": "mfma", "achieved": tf, "peak": PEAK_FP8_TFLOPS, "unit": "TFLOP/s",
                         "frac": tf / PEAK_FP8_TFLOPS},
            "quantise_us": qms * 1e3, "quantise_gbs": qbytes / (qms * 1e-3) / 1e9}


def bench_attention(steps, warmup):
    import torch
    from ptb_amd import ops

    hq, hkv, s, d = 32, 8, 4096, 128
    g = torch.Generator().manual_seed(0)
    q = torch.randn(hq, s, d, generator=g).to(torch.bfloat16).cuda()
    k = torch.randn(hkv, s, d, generator=g).to(torch.bfloat16).cuda()
    v = torch.randn(hkv, s, d, generator=g).to(torch.bfloat16).cuda()
    o = torch.empty_like(q)
    ms, wall = timed(lambda: ops.flash_attention(q, k, v, hq, hkv, True, out=o), steps, warmup)
    flops = 4.0 * hq * d * s * (s + 1) / 2
    tf = flops / (ms * 1e-3) / 1e12
    return {"name": "flash_attention", "config": "BASELINE config 3: causal GQA 32/8 heads, S 4096, D 128",
            "us": ms * 1e3, "wall_us": wall * 1e3, "tflops": tf,
            "roofline": {"bound": "mfma", "achieved": tf, "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                         "frac": tf / PEAK_BF16_TFLOPS}}


def bench_layer(steps, warmup):
    import torch
    from ptb_amd import qwen3

    t = 2048
    layer = qwen3.Qwen3Layer(qwen3.random_weights(device="cuda"))
    g = torch.Generator().manual_seed(1)
    x = torch.randn(t, 4096, generator=g).to(torch.bfloat16).cuda()
    y = torch.empty_like(x)
    ms, wall = timed(lambda: layer.forward(x, out=y), max(5, steps // 5), max(2, warmup // 5))
    work = qwen3.layer_work(t)
    roof_us = sum(max(f / (PEAK_BF16_TFLOPS * 1e12), b / (PEAK_HBM_GBS * 1e9)) for _, f, b in work) * 1e6
    flops = sum(f for _, f, _ in work)
    return {"name": "qwen3_8b_layer", "config": "BASELINE config 5: Qwen3-8B decoder layer prefill T=S=2048",
            "us": ms * 1e3, "wall_us": wall * 1e3, "tflops": flops / (ms * 1e-3) / 1e12,
            # the reference's layer is 14 launches of different bounds: frac = the sum of their
            # roofline times (max of MFMA time and HBM time each) over the measured layer latency;
            # the forward issues them fused into 8 kernels
            "roofline": {"bound": "mixed", "roofline_us": roof_us, "measured_us": ms * 1e3, "unit": "us",
                         "frac": roof_us / (ms * 1e3)},
            "launches": qwen3.PREFILL_KERNELS, "reference_launches": len(work)}


def bench_gemv(steps, warmup):
    """The decode layer's largest GEMV (K06 of qwen3_8b_layer_decode_1x<S>_bf16): the post-attention
    RMSNorm folded into gu = ((x + a) * r * w_post) Wgu, W [4096, 24576] bf16 streamed once."""
    import torch
    from ptb_amd import ops

    k, n = 4096, 24576
    g = torch.Generator().manual_seed(0)
    copies = 3   # 3 x 201 MB cycles through more than the 256 MB last-level cache
    ws = [(torch.randn(k, n, generator=g) * 0.02).to(torch.bfloat16).cuda() for _ in range(copies)]
    x = torch.randn(k, generator=g).to(torch.bfloat16).cuda()
    a = torch.randn(k, generator=g).to(torch.bfloat16).cuda()
    gw = (torch.randn(k, generator=g) * 0.02 + 1).to(torch.bfloat16).cuda()
    ss = ops.sumsq(x, a)
    y = torch.empty(n, dtype=torch.bfloat16, device="cuda")
    from ptb_amd import _lib
    work = torch.empty(_lib.load().ptb_gemv_workspace_bytes(k, n), dtype=torch.uint8, device="cuda")
    it = [0]

    def step():
        i = it[0] % copies
        it[0] += 1
        ops.gemv_rmsnorm(x, ss, gw, ws[i], add=a, out=y, workspace=work)

    eager_ms, wall = timed(step, steps * 4, warmup)
    ms = timed_graph(step, copies, max(4, steps))
    nbytes = 2.0 * (k * n + 3 * k + n) + 4
    gbs = nbytes / (ms * 1e-3) / 1e9
    return {"name": "gemv_decode", "config": "decode K06: ((x+a)*rsqrt(ss/4096+eps)*w) @ Wgu[4096x24576], bf16",
            "us": ms * 1e3, "timing": "hip graph replay", "eager_us": eager_ms * 1e3, "wall_us": wall * 1e3,
            "gbs": gbs,
            "roofline": {"bound": "hbm", "achieved": gbs, "peak": PEAK_HBM_GBS, "unit": "GB/s",
                         "frac": gbs / PEAK_HBM_GBS}}


def bench_attention_decode(steps, warmup):
    """attention_decode_32x8x4096_bf16: one token, 32 query heads over an [8, 4096, 128] K/V cache."""
    import torch
    from ptb_amd import ops

    hkv, g, s, d = 8, 4, 4096, 128
    gen = torch.Generator().manual_seed(0)
    copies = 12   # 12 x 16.8 MB of K/V: past the last-level cache
    kvs = [(torch.randn(hkv, s, d, generator=gen).to(torch.bfloat16).cuda(),
            torch.randn(hkv, s, d, generator=gen).to(torch.bfloat16).cuda()) for _ in range(copies)]
    q = torch.randn(hkv, g, d, generator=gen).to(torch.bfloat16).cuda()
    o = torch.empty_like(q)
    from ptb_amd import _lib
    work = torch.empty(_lib.load().ptb_attn_decode_workspace_bytes(hkv, g, s), dtype=torch.uint8, device="cuda")
    it = [0]

    def step():
        k, v = kvs[it[0] % copies]
        it[0] += 1
        ops.attention_decode(q, k, v, out=o, workspace=work)

    eager_ms, wall = timed(step, steps * 4, warmup)
    ms = timed_graph(step, copies, max(4, steps))
    nbytes = 2.0 * (2 * hkv * s * d + 2 * hkv * g * d)
    gbs = nbytes / (ms * 1e-3) / 1e9
    return {"name": "attention_decode", "config": "attention_decode_32x8x4096_bf16: 1 token, 32/8 heads, S 4096",
            "us": ms * 1e3, "timing": "hip graph replay", "eager_us": eager_ms * 1e3, "wall_us": wall * 1e3,
            "gbs": gbs,
            "roofline": {"bound": "hbm", "achieved": gbs, "peak": PEAK_HBM_GBS, "unit": "GB/s",
                         "frac": gbs / PEAK_HBM_GBS}}


def decode_sweep(steps, warmup):
    """Decode attention over cache lengths 512 .. 32768 (8 kv heads, 4 query rows each, D 128): time
    per call, GB/s and the fraction of 8 TB/s at each length, cycling enough K/V copies (>= 400 MB)
    that every call reads HBM.  A time that does not grow with the bytes names launch and latency,
    not bandwidth, as the limit."""
    import torch
    from ptb_amd import _lib, ops

    hkv, g, d = 8, 4, 128
    gen = torch.Generator().manual_seed(0)
    q = torch.randn(hkv, g, d, generator=gen).to(torch.bfloat16).cuda()
    o = torch.empty_like(q)
    rows = []
    for s in (512, 1024, 2048, 4096, 8192, 16384, 32768):
        copies = max(3, int(400e6 // (2 * 2 * hkv * s * d)))
        kvs = [(torch.randn(hkv, s, d, generator=gen).to(torch.bfloat16).cuda(),
                torch.randn(hkv, s, d, generator=gen).to(torch.bfloat16).cuda()) for _ in range(copies)]
        work = torch.empty(max(1, _lib.load().ptb_attn_decode_workspace_bytes(hkv, g, s)), dtype=torch.uint8,
                           device="cuda")
        it = [0]

        def step():
            k, v = kvs[it[0] % copies]
            it[0] += 1
            ops.attention_decode(q, k, v, out=o, workspace=work)

        eager_ms, _ = timed(step, steps * 4, warmup)
        ms = timed_graph(step, copies, max(4, steps))
        nbytes = 2.0 * (2 * hkv * s * d + 2 * hkv * g * d)
        gbs = nbytes / (ms * 1e-3) / 1e9
        rows.append({"seq": s, "us": ms * 1e3, "eager_us": eager_ms * 1e3, "gbs": gbs, "frac": gbs / PEAK_HBM_GBS,
                     "copies": copies})
        log(f"[sweep] S={s}: {ms * 1e3:.2f} us by graph replay ({eager_ms * 1e3:.2f} us eager), {gbs:.0f} GB/s")
        del kvs
        torch.cuda.empty_cache()
    return rows


def bench_decode_layer(steps, warmup):
    """qwen3_8b_layer_decode_1x4096_bf16: the bundle's 8-launch decode layer over a 4096-token cache
    (issued here as 5 fused steps, 10 kernels: each GEMV and the attention keep their finish pass)."""
    import torch
    from ptb_amd import qwen3

    layer = qwen3.Qwen3DecodeLayer(qwen3.random_weights(device="cuda"))
    g = torch.Generator().manual_seed(1)
    s = 4096
    x = torch.randn(4096, generator=g).to(torch.bfloat16).cuda()
    kc = torch.randn(8, s, 128, generator=g).to(torch.bfloat16).cuda()
    vc = torch.randn(8, s, 128, generator=g).to(torch.bfloat16).cuda()
    cos_t, sin_t = qwen3.rope_tables(s + 1, 128, 1.0e6, "cuda")
    cos, sin = cos_t[s].contiguous(), sin_t[s].contiguous()
    y = torch.empty_like(x)
    step = lambda: layer.forward(x, kc, vc, cos, sin, out=y)  # noqa: E731
    eager_ms, wall = timed(step, steps, warmup)
    ms = timed_graph(step, 4, max(4, steps // 4))
    # bytes the layer must move: every weight once plus the K/V cache
    nbytes = 2.0 * (4096 * 4096 * 2 + 4096 * 24576 + 12288 * 4096) + 2.0 * 2 * 8 * s * 128
    roof_us = nbytes / (PEAK_HBM_GBS * 1e9) * 1e6
    return {"name": "qwen3_8b_decode_layer", "config": "qwen3_8b_layer_decode_1x4096_bf16: 1 token, cache 4096",
            "us": ms * 1e3, "timing": "hip graph replay", "eager_us": eager_ms * 1e3, "wall_us": wall * 1e3,
            "gbs": nbytes / (ms * 1e-3) / 1e9,
            "roofline": {"bound": "hbm", "roofline_us": roof_us, "measured_us": ms * 1e3, "unit": "us",
                         "frac": roof_us / (ms * 1e3)},
            # GEMV partial + finish passes (the gate/up finish inside the down projection's prologue)
            # and attention's partial + merge passes, for the reference's 8 launches
            "launches": 9, "reference_launches": 8}


def _trial_seconds(fn, min_s: float) -> float:
    """Seconds per call of fn over one trial: at least one call, repeated until min_s has passed."""
    t0 = time.perf_counter()
    reps = 0
    while True:
        fn()
        reps += 1
        if time.perf_counter() - t0 >= min_s:
            return (time.perf_counter() - t0) / reps


def _median_seconds(fn, trials: int, min_s: float) -> float:
    ts = sorted(_trial_seconds(fn, min_s) for _ in range(trials))
    return ts[len(ts) // 2]


def golden_gemm_fp32(a, b, residual=None):
    """The reference's CPU golden for its GEMMs: torch.matmul on fp32 operands
    (tests/cases/smoke/gemm.py:45-47, tests/cases/mechanism/ops/ops_bf16_matmul.py's reference),
    with the bf16 kernel's residual add and single bf16 rounding."""
    import torch

    acc = torch.matmul(a.float(), b.float())
    if residual is not None:
        acc = acc + residual.float()
    return acc.to(torch.bfloat16)


def golden_gemm_fp8_fp32(aq, sa, wq_t, sw):
    """The reference's fp8 golden: torch.matmul of the e4m3 operands upcast to fp32
    (tests/cases/mechanism/ops/ops_fp8_e4m3_dot.py:41-44), then the per-token x per-channel scale
    epilogue (tests/cases/workloads/int8_dequant_matmul.py:59-69)."""
    import torch

    acc = torch.matmul(aq.float(), wq_t.float().t())
    return ((acc * sa[:, None]) * sw[None, :]).to(torch.bfloat16)


def cpu_baselines() -> list:
    """The reference's CPU golden for each BASELINE config, timed on this host on a bounded sample
    of each workload, on all host threads (median of 3 trials, 1 for the layer) and on one thread
    (median of 3, 1 for the layer).  GEMMs (config 2, the fp8 dot of config 4, the layer's
    projections) are the reference's golden, torch.matmul on fp32 operands; the vector ops and
    attention are the oracle's torch-CPU restatements (the fp64 GEMM sums of the oracle stay the
    parity checker only).  Throughput is the sample's algorithmic work over its time, in the GPU
    line's unit; the layer also gives its latency."""
    import torch
    import oracle
    from ptb_amd import qwen3

    bf = torch.bfloat16
    threads = len(os.sched_getaffinity(0))
    g = torch.Generator().manual_seed(0)
    out = []

    def leg(name, unit, work, sample_all, sample_one, fn_all, fn_one, trials=3, min_s=1.0,
            golden="oracle (torch-CPU fp32)"):
        """work(sample) -> algorithmic units of one call (GB or GFLOP); fn_*() runs the sample."""
        rec = {"config": name, "unit": unit, "cores": threads, "kind": "port", "golden": golden}
        for key, n, fn, samp in (("all", threads, fn_all, sample_all), ("one", 1, fn_one, sample_one)):
            torch.set_num_threads(n)
            if trials > 1:
                fn()   # warm (allocations)
            sec = _median_seconds(fn, trials, min_s if key == "all" else 0.0)
            rate = work(samp) / sec / (1e3 if unit == "TFLOP/s" else 1.0)
            rec["value" if key == "all" else "value_1_thread"] = rate
            rec["sample" if key == "all" else "sample_1_thread"] = f"{samp['what']}: {sec * 1e3:.1f} ms per call"
        rec["trials"] = trials
        torch.set_num_threads(threads)
        log(f"[bench] cpu {name}: {rec['value']:.4g} {unit} on {threads} threads, "
            f"{rec['value_1_thread']:.4g} on 1")
        return rec

    # config 1: RMSNorm, the whole workload
    x = torch.randn(2048, 4096, generator=g).to(bf)
    w = torch.randn(4096, generator=g) * 0.02 + 1.0
    s1 = {"what": "the whole 2048x4096 RMSNorm", "bytes": 2 * 2048 * 4096 * 2 + 4096 * 4}
    out.append(leg("1 rmsnorm", "GB/s", lambda s: s["bytes"] / 1e9, s1, s1,
                   lambda: oracle.rmsnorm(x, w, 1e-6), lambda: oracle.rmsnorm(x, w, 1e-6)))
    # config 2: bf16 GEMM, rows of A against all of B
    a = (torch.randn(4096, 4096, generator=g) / 64).to(bf)
    b = (torch.randn(4096, 12288, generator=g) / 64).to(bf)
    s2a = {"what": "256 of 4096 rows of A @ B[4096x12288]", "rows": 256}
    s2o = {"what": "32 of 4096 rows of A @ B[4096x12288]", "rows": 32}
    out.append(leg("2 gemm_bf16", "TFLOP/s", lambda s: 2.0 * s["rows"] * 4096 * 12288 / 1e9, s2a, s2o,
                   lambda: golden_gemm_fp32(a[:256], b), lambda: golden_gemm_fp32(a[:32], b),
                   golden="fp32 torch"))
    del a, b
    # config 3: causal GQA attention, one kv head with its 4 query heads (1/8 of the heads), full S
    q = torch.randn(4, 4096, 128, generator=g).to(bf)
    k = torch.randn(1, 4096, 128, generator=g).to(bf)
    v = torch.randn(1, 4096, 128, generator=g).to(bf)
    s3 = {"what": "4 of 32 query heads (one kv head), S 4096, causal", "heads": 4}
    att = lambda: oracle.flash_attention(q, k, v, 4, 1, True)  # noqa: E731
    out.append(leg("3 flash_attention", "TFLOP/s", lambda s: 4.0 * s["heads"] * 128 * 4096 * 4097 / 2 / 1e9,
                   s3, s3, att, att))
    # config 4: per-token quantise + fp8 GEMM, rows of x against the whole packed weight
    xs = torch.randn(64, 12288, generator=g).to(bf)
    wq, sw = oracle.quant_weight_e4m3(torch.randn(12288, 4096, generator=g) * 0.02)
    s4a = {"what": "quantise + e4m3 GEMM of 64 of 2048 rows against W[12288x4096]", "rows": 64}
    s4o = {"what": "quantise + e4m3 GEMM of 16 of 2048 rows against W[12288x4096]", "rows": 16}

    def fp8(rows):
        aq, sa = oracle.quant_rows_e4m3(xs[:rows])
        golden_gemm_fp8_fp32(aq, sa, wq, sw)

    out.append(leg("4 gemm_fp8", "TFLOP/s", lambda s: 2.0 * s["rows"] * 12288 * 4096 / 1e9, s4a, s4o,
                   lambda: fp8(64), lambda: fp8(16), golden="fp32 torch (quantiser: oracle)"))
    del wq, sw
    # config 5: the layer; all threads run T = 2048, one thread the first 256 tokens (a causal
    # layer's first rows are exactly a shorter sequence)
    wts = qwen3.random_weights()
    xt = torch.randn(2048, 4096, generator=torch.Generator().manual_seed(1)).to(bf)
    cos, sin = oracle.rope_tables(2048, 128, 1.0e6)
    lay = lambda t: oracle.qwen3_layer(xt[:t], wts, cos[:t], sin[:t], bq=min(t, 1024),  # noqa: E731
                                       gemm_fn=golden_gemm_fp32)
    flops = lambda s: sum(f for _, f, _ in qwen3.layer_work(s["t"])) / 1e9  # noqa: E731
    s5a = {"what": "the whole layer, T = S = 2048", "t": 2048}
    s5o = {"what": "the layer over the first 256 tokens", "t": 256}
    rec = leg("5 qwen3_8b_layer", "TFLOP/s", flops, s5a, s5o, lambda: lay(2048), lambda: lay(256),
              trials=1, min_s=0.0, golden="fp32 torch GEMMs, oracle vector ops and attention")
    rec["layer_us"] = flops(s5a) / rec["value"] * 1e3   # GFLOP / (TFLOP/s) = ms
    out.append(rec)
    return out


def pmc_driver(which: str) -> None:
    """What the committed rocprofv3 --pmc summaries were collected on: the BASELINE-shaped kernel
    launched 5 times, then a 256 MiB device copy as the calibration dispatch for FETCH_SIZE /
    WRITE_SIZE (its true traffic is 256 MiB each way)."""
    import torch
    from ptb_amd import ops

    g = torch.Generator().manual_seed(0)
    if which == "gemm_bf16":
        a = (torch.randn(4096, 4096, generator=g) / 64).to(torch.bfloat16).cuda()
        b = (torch.randn(4096, 12288, generator=g) / 64).to(torch.bfloat16).cuda()
        c = torch.empty(4096, 12288, dtype=torch.bfloat16, device="cuda")
        run = lambda: ops.gemm(a, b, out=c)  # noqa: E731
    elif which == "gemm_fp8":
        x = torch.randn(2048, 12288, generator=g).to(torch.bfloat16).cuda()
        wq, sw = ops.quant_weight_e4m3((torch.randn(12288, 4096, generator=g) * 0.02).cuda())
        xq, sx = ops.quant_rows_e4m3(x)
        c = torch.empty(2048, 4096, dtype=torch.bfloat16, device="cuda")
        run = lambda: ops.gemm_fp8(xq, sx, wq, sw, out=c)  # noqa: E731
    elif which == "flash_attention":
        q = torch.randn(32, 4096, 128, generator=g).to(torch.bfloat16).cuda()
        k = torch.randn(8, 4096, 128, generator=g).to(torch.bfloat16).cuda()
        v = torch.randn(8, 4096, 128, generator=g).to(torch.bfloat16).cuda()
        o = torch.empty_like(q)
        run = lambda: ops.flash_attention(q, k, v, 32, 8, True, out=o)  # noqa: E731
    elif which == "rmsnorm":
        x = torch.randn(2048, 4096, generator=g).to(torch.bfloat16).cuda()
        w = (torch.randn(4096, generator=g) * 0.02 + 1).cuda()
        y = torch.empty_like(x)
        run = lambda: ops.rmsnorm(x, w, 1e-6, out=y)  # noqa: E731
    elif which == "quant_rows":
        x = torch.randn(2048, 12288, generator=g).to(torch.bfloat16).cuda()
        run = lambda: ops.quant_rows_e4m3(x)  # noqa: E731
    elif which == "gemv_decode":
        from ptb_amd import _lib
        wg = (torch.randn(4096, 24576, generator=g) * 0.02).to(torch.bfloat16).cuda()
        x = torch.randn(4096, generator=g).to(torch.bfloat16).cuda()
        a = torch.randn(4096, generator=g).to(torch.bfloat16).cuda()
        gw = (torch.randn(4096, generator=g) * 0.02 + 1).to(torch.bfloat16).cuda()
        ss = ops.sumsq(x, a)
        y = torch.empty(24576, dtype=torch.bfloat16, device="cuda")
        ws = torch.empty(_lib.load().ptb_gemv_workspace_bytes(4096, 24576), dtype=torch.uint8, device="cuda")
        run = lambda: ops.gemv_rmsnorm(x, ss, gw, wg, add=a, out=y, workspace=ws)  # noqa: E731
    elif which == "attention_decode":
        from ptb_amd import _lib
        q = torch.randn(8, 4, 128, generator=g).to(torch.bfloat16).cuda()
        k = torch.randn(8, 4096, 128, generator=g).to(torch.bfloat16).cuda()
        v = torch.randn(8, 4096, 128, generator=g).to(torch.bfloat16).cuda()
        o = torch.empty_like(q)
        ws = torch.empty(_lib.load().ptb_attn_decode_workspace_bytes(8, 4, 4096), dtype=torch.uint8, device="cuda")
        run = lambda: ops.attention_decode(q, k, v, out=o, workspace=ws)  # noqa: E731
    else:
        raise SystemExit(f"unknown --pmc-driver {which}")
    for _ in range(5):
        run()
    src = torch.ones(64 * 1024 * 1024, dtype=torch.float32, device="cuda")
    torch.empty_like(src).copy_(src)
    torch.cuda.synchronize()
    print(f"pmc driver {which}: done", flush=True)


def profiled_traffic(name: str):
    """HBM bytes per launch of the headline kernel from its committed rocprofv3 --pmc summary
    (FETCH_SIZE and WRITE_SIZE, scaled by the 256 MiB copy's readings), or None."""
    path = REPO / "profiles" / f"{name}.md"
    if not path.exists():
        return None
    for line in path.read_text().splitlines():
        if line.startswith("traffic_bytes_per_launch ="):
            return int(float(line.split("=")[1]))
    return None


BENCHES = {
    "gemm_bf16": bench_gemm_bf16,
    "rmsnorm": bench_rmsnorm,
    "gemm_fp8": bench_gemm_fp8,
    "flash_attention": bench_attention,
    "qwen3_8b_layer": bench_layer,
    "gemv_decode": bench_gemv,
    "attention_decode": bench_attention_decode,
    "qwen3_8b_decode_layer": bench_decode_layer,
}


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--only", default="", help="comma-separated subset of " + ",".join(BENCHES))
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--pmc-driver", help="run one kernel 5x plus a 256 MiB copy (for rocprofv3 --pmc) and exit")
    ap.add_argument("--decode-sweep", action="store_true",
                    help="time decode attention over cache lengths 512..32768, print one JSON line and exit")
    ap.add_argument("--settle", type=float, default=SETTLE_S,
                    help="seconds of untimed back-to-back launches before the warmup steps")
    args = ap.parse_args(argv)
    globals()["SETTLE_S"] = max(0.0, args.settle)
    if args.pmc_driver:
        pmc_driver(args.pmc_driver)
        return 0
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (asked for --gpus {args.gpus}); sharding the "
              "path over several GPUs is a design, not a benchmarked configuration.", file=sys.stderr)
        return 2

    import torch

    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        return 1
    from ptb_amd import _lib

    _lib.load()   # fail loudly when the HIP library is missing
    if args.decode_sweep:
        print(json.dumps({"decode_sweep": decode_sweep(args.steps, args.warmup)}), flush=True)
        return 0
    names = [n for n in (args.only.split(",") if args.only else BENCHES) if n]
    results = {}
    for name in names:
        log(f"[bench] {name} ...")
        results[name] = BENCHES[name](args.steps, args.warmup)
        r = results[name]
        log(f"[bench] {name}: {r['us']:.1f} us/launch, roofline frac {r['roofline']['frac']:.3f}")

    head = results.get("gemm_bf16") or next(iter(results.values()))
    cpu = None
    if not args.no_cpu:
        log("[bench] cpu baselines (the oracle on this host's cores) ...")
        per_config = cpu_baselines()
        c2 = next(r for r in per_config if r["config"].startswith("2 "))
        cpu = {"value": c2["value"], "unit": c2["unit"], "cores": c2["cores"], "kind": "port",
               "golden": c2["golden"], "sample": c2["sample"], "value_1_thread": c2["value_1_thread"],
               "sample_1_thread": c2["sample_1_thread"], "configs": per_config}
    kernels = []
    for r in results.values():
        kernels.append({k: v for k, v in r.items() if not k.startswith("_")})
    line = {
        "metric": "TFLOP/s or GB/s (% MI355X roofline) per kernel; Qwen3-8B layer latency",
        "value": head.get("tflops", head.get("gbs")),
        "unit": "TFLOP/s" if "tflops" in head else "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": head["us"] / 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded randn, BASELINE.json shapes)",
        "config": ({"workload": "BASELINE config 2: bf16 GEMM C[4096,12288] = A[4096,4096] @ B[4096,12288], "
                                "fp32 accumulation, bf16 C", "M": 4096, "K": 4096, "N": 12288,
                    "settle_s": SETTLE_S}
                   if "gemm_bf16" in results else {"workload": head["config"], "settle_s": SETTLE_S}),
        "roofline": (dict(head["roofline"], traffic=profiled_traffic("gemm_bf16_4096x4096x12288"))
                     if "gemm_bf16" in results else dict(head["roofline"], traffic=None)),
        "cpu_baseline": cpu,
        "kernels": kernels,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
