"""Validation-suite entry points on the GPU: time the bundle's workloads with the HIP kernels.

Mirrors the reference's runners, ``validation/{vector,gemm,attention,layer,qwen3_8b}/
simulate_shapes.py`` (shared runner validation/gemm/simulate_shapes.py:265-319, 426-502): the same
suite KEYS name a workload, every distinct kernel of a workload runs once per launch count, and
``results.json`` -- rewritten after every workload -- holds per workload the keys, ``kernel`` (the
workload name), ``rc``, ``failed_step``, ``us`` and per kernel its launches.  Where the reference
reads TOGSim cycles, this runner reads hipEvent time of back-to-back launches on inputs drawn by
the specs' seeded ``make_inputs`` convention, and adds TFLOP/s, GB/s and the MI355X roofline
fraction per kernel.  ``--shard K/N`` and ``--merge`` split and join runs as the reference's do.

    python -m ptb_amd.validation qwen3_8b --bundle <reference>/validation/pytorchsim --out results.json
    python -m ptb_amd.validation gemm --manifests bundle_manifests.json.gz --out results.json

``--manifests`` reads the workloads from a manifests file (tests/golden/extract_bundle.py writes
one for the whole bundle) where the bundle's directory tree is not at hand.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

from . import bundle, contract, kernels

MI355X = {"name": "MI355X (gfx950)", "peak_bf16_tflops": 2500.0, "peak_fp8_tflops": 5000.0, "hbm_gbs": 8000.0}
SUITES = tuple(bundle.SUITE_KEYS)

#: --ci caps (reference: validation/layer/simulate_shapes.py:13 CI_TOKENS, :26 CI_OPS; validation/gemm/
#: simulate_shapes.py:58-59 the table of Qwen3-30B-A3B GEMM shapes whose M the cap limits, and CI_M)
CI_TOKENS = 4096
CI_OPS = ("dispatch", "combine", "router_post", "gmm_gate_up", "gmm_down")
CI_M = 4096
CAPPED_TABLE = os.path.join("gemm", "tpu_v6e_qwen3moe_torchxla.csv")


def read_capped(path) -> frozenset:
    """The (M, K, N) shapes a measured GEMM table holds: the gemm suite's --ci caps these by M."""
    import csv

    with open(path, newline="") as fh:
        return frozenset(tuple(int(r[k]) for k in ("M", "K", "N")) for r in csv.DictReader(fh))


def _tokens(keys) -> int:
    """A layer workload's tokens: a layer's context S, an op's T (validation/layer/simulate_shapes.py:16-18)."""
    return int(keys["S"]) if keys["section"] == "layer" else int(keys["T"])


def under_ci_cap(suite, keys, capped=frozenset()) -> bool:
    """Whether the suite's --ci times a workload with these keys.  layer: a layer or one of CI_OPS of at most
    CI_TOKENS tokens (validation/layer/simulate_shapes.py:30-32); qwen3_8b: a layer of at most CI_TOKENS tokens
    (validation/qwen3_8b/simulate_shapes.py:27-30); gemm: a shape of the `capped` table at M <= CI_M, any other
    shape always (validation/gemm/simulate_shapes.py:408-411); vector and attention have no cap."""
    if suite == "layer":
        return (keys["section"] == "layer" or keys["name"] in CI_OPS) and _tokens(keys) <= CI_TOKENS
    if suite == "qwen3_8b":
        return keys["section"] == "layer" and _tokens(keys) <= CI_TOKENS
    if suite == "gemm":
        shape = tuple(int(keys[k]) for k in ("M", "K", "N"))
        return shape not in capped or shape[0] <= CI_M
    return True


def cost(suite, keys) -> int:
    """What a workload is ranked by when shards are planned: attention the scores it computes
    (validation/attention/simulate_shapes.py:13-17), the layer suites the query-key pairs of a layer or an op's
    tokens (validation/layer/simulate_shapes.py:21-23), any other suite the product of its numeric keys
    (validation/gemm/simulate_shapes.py:171-179)."""
    if suite == "attention":
        hq, sq = int(keys["Hq"]), int(keys["S"])
        return hq * sq * (sq + 1) // 2 if keys["kind"] == "prefill" else hq * sq
    if suite in ("layer", "qwen3_8b"):
        return int(keys["T"]) * int(keys["S"]) if keys["section"] == "layer" else int(keys["T"])
    n = 1
    for v in keys.values():
        n *= int(v) if str(v).isdigit() else 1
    return n


def shard(ws, k, n, suite) -> list:
    """Part `k` (0-based) of `n`, by longest processing time: the workloads, costliest first (ties in key order),
    each go to the part with the least cost so far (ties to the lower part), so the parts are disjoint, cover the
    set and are fixed (validation/gemm/simulate_shapes.py:182-196)."""
    if not 0 <= k < n:
        raise ValueError(f"--shard {k}/{n}: K must be in 0..N-1")
    names = bundle.SUITE_KEYS[suite]

    def order(w):
        return (-cost(suite, w.keys), tuple((0, int(w.keys[c])) if str(w.keys[c]).isdigit() else (1, w.keys[c])
                                            for c in names))
    load, mine = [0] * n, []
    for w in sorted(ws, key=order):
        i = min(range(n), key=lambda j: (load[j], j))
        load[i] += cost(suite, w.keys)
        if i == k:
            mine.append(w)
    return mine


def time_kernel(bk, reps: int = 20, warmup: int = 3, seed: int = 0, settle: float = 0.02, graph: bool = True,
                recorded: dict | None = None) -> dict:
    """Run one bundle kernel on the GPU and time it; returns its record.  `recorded` holds the
    arguments the spec takes from its recorded inputs (the MoE kernels' index tables)."""
    import torch

    plan = kernels.resolve(bk.spec, bk.source)
    host = contract.seeded_inputs(bk.spec, torch, seed, recorded=recorded)
    tensors = {}
    for a in bk.spec.args:
        if a.name in host:
            tensors[a.name] = host[a.name].to("cuda")
        else:
            tensors[a.name] = torch.empty(a.numel, dtype=getattr(torch, a.dtype), device="cuda")
    # the clock needs tens of ms of load to leave idle: run the kernel for `settle` seconds first
    t_end = time.perf_counter() + settle
    while True:
        for _ in range(max(1, warmup)):
            kernels.run(plan, tensors)
        torch.cuda.synchronize()
        if time.perf_counter() >= t_end:
            break
    eager_us = _time(lambda: [kernels.run(plan, tensors) for _ in range(reps)], torch) / reps
    # the same launches captured once as a HIP graph and replayed: the device time without the
    # host's per-launch cost (which sets the time of kernels shorter than a Python call)
    us, timing = eager_us, "eager"
    if graph:
        try:
            side = torch.cuda.Stream()
            side.wait_stream(torch.cuda.current_stream())
            g = torch.cuda.CUDAGraph()
            with torch.cuda.stream(side), torch.cuda.graph(g, stream=side):
                for _ in range(reps):
                    kernels.run(plan, tensors)
            torch.cuda.current_stream().wait_stream(side)
            g.replay()
            torch.cuda.synchronize()
            us = min(_time(g.replay, torch) for _ in range(3)) / reps
            timing = "graph"
        except Exception:  # noqa: BLE001 - a kernel that cannot be captured keeps its eager time
            torch.cuda.synchronize()
    flops, nbytes = kernels.work_of(plan)
    tflops = flops / (us * 1e-6) / 1e12
    gbs = nbytes / (us * 1e-6) / 1e9
    roof_us = max(flops / (MI355X["peak_bf16_tflops"] * 1e12), nbytes / (MI355X["hbm_gbs"] * 1e9)) * 1e6
    return {"dir": bk.dir, "name": bk.spec.name, "launches": bk.launches, "family": plan.family, "us": us,
            "eager_us": eager_us, "timing": timing, "flops": flops, "bytes": nbytes,
            "tflops": tflops, "gbs": gbs, "roofline_us": roof_us, "roofline_frac": roof_us / us if us else None}


def _time(fn, torch) -> float:
    """Microseconds fn() takes on the current stream, by HIP events."""
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    fn()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1e3


def _recorded_for(w, bk, recorded_path):
    """The recorded inputs of one kernel: from a recorded-inputs file, or from the ``*_inputs.pt``
    beside the spec when the workload was read from the bundle itself."""
    if not (bk.spec.extra or {}).get("recorded"):
        return None
    if recorded_path:
        return bundle.read_recorded(recorded_path, w.name, bk.dir)
    if w.path:
        import torch

        d = os.path.join(w.path, bk.dir)
        pts = [f for f in os.listdir(d) if f.endswith("_inputs.pt")]
        if len(pts) == 1:
            return torch.load(os.path.join(d, pts[0]), weights_only=True)
    raise FileNotFoundError(f"{w.name}/{bk.dir}: recorded inputs needed (--recorded)")


def run_workload(w, reps: int = 20, warmup: int = 3, settle: float = 0.02, graph: bool = True,
                 recorded_path: str | None = None) -> dict:
    got = dict(w.keys, kernel=w.name, rc=0, failed_step=None, kernels=[])
    t0 = time.monotonic()
    step = "resolve"
    try:
        for bk in w.kernels:
            step = bk.dir
            got["kernels"].append(time_kernel(bk, reps, warmup, settle=settle, graph=graph,
                                              recorded=_recorded_for(w, bk, recorded_path)))
        got["us"] = sum(k["us"] * k["launches"] for k in got["kernels"])
        got["roofline_us"] = sum(k["roofline_us"] * k["launches"] for k in got["kernels"])
    except Exception as e:  # noqa: BLE001 - a workload's failure is recorded, never lost
        got.update(rc=f"{type(e).__name__}: {e}", failed_step=step)
    got["wall_s"] = round(time.monotonic() - t0, 1)
    return got


def write_results(path, suite, done, total, part=None) -> None:
    keys = bundle.SUITE_KEYS[suite]
    shapes = sorted(done, key=lambda r: tuple(str(r.get(k)) for k in keys))
    res = {"machine": MI355X, "suite": suite, "expected": total, "shapes": shapes}
    if part:
        res["shard"] = part
    tmp = path + ".tmp"
    with open(tmp, "w") as fh:
        json.dump(res, fh, indent=1)
    os.replace(tmp, path)


def merge(paths, out) -> int:
    """The results.json of shard runs as one run's at `out`: the parts must come from one suite and machine and
    must not overlap; expected is the whole set's.  1 if a workload is missing (validation/gemm/
    simulate_shapes.py:322-352)."""
    parts = []
    for p in paths:
        with open(p) as fh:
            parts.append(json.load(fh))
    suite = parts[0]["suite"]
    if any(p["suite"] != suite or p["machine"] != parts[0]["machine"] for p in parts):
        raise ValueError("shards of different suites or machines")
    names = [s["kernel"] for p in parts for s in p["shapes"]]
    if len(names) != len(set(names)):
        raise ValueError("shards overlap: " + ", ".join(sorted({k for k in names if names.count(k) > 1})))
    shapes = [s for p in parts for s in p["shapes"]]
    plan = parts[0].get("shard")
    expected = plan["total"] if isinstance(plan, dict) else parts[0]["expected"]
    write_results(out, suite, shapes, expected)
    return 0 if len(shapes) == expected else 1


def parse_where(items):
    out = {}
    for it in items or ():
        k, _, v = it.partition("=")
        out[k] = v
    return out


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description="time a validation suite's bundle workloads on the GPU")
    ap.add_argument("suite", choices=SUITES)
    ap.add_argument("--bundle", required=False, help="the reference's validation/pytorchsim directory")
    ap.add_argument("--manifests", required=False, help="a manifests file (.json or .json.gz) instead of --bundle")
    ap.add_argument("--out", default="results.json")
    ap.add_argument("--where", action="append", help="key=value filter on the workload's keys (repeatable)")
    ap.add_argument("--only", action="append", help="workload name (repeatable)")
    ap.add_argument("--ci", action="store_true", help="only the workloads under the suite's CI cap, where it has one")
    ap.add_argument("--shard", help="K/N: time part K (0-based) of N disjoint parts of the set")
    ap.add_argument("--merge", nargs="+", help="join shard results.json files into --out")
    ap.add_argument("--reps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--settle", type=float, default=0.02, help="seconds of back-to-back launches before timing")
    ap.add_argument("--eager", action="store_true", help="time Python launches only (no HIP graph replay)")
    ap.add_argument("--recorded", help="recorded-inputs file (.npz) for kernels whose specs take recorded inputs")
    args = ap.parse_args(argv)
    if args.merge:
        return merge(args.merge, args.out)
    if bool(args.bundle) == bool(args.manifests):
        ap.error("give one of --bundle or --manifests (unless --merge)")
    from . import _lib

    _lib.load()
    if args.bundle:
        ws = bundle.load_bundle(args.bundle, args.suite, parse_where(args.where) or None)
        table = os.path.join(os.path.dirname(os.path.abspath(args.bundle)), CAPPED_TABLE)
        capped = read_capped(table) if args.suite == "gemm" and os.path.isfile(table) else frozenset()
        if args.ci and args.suite == "gemm" and not capped:
            raise SystemExit(f"--ci: the gemm suite's cap reads {table}, which is not there")
        for w in ws:
            w.ci = under_ci_cap(w.suite, w.keys, capped)
    else:
        ws = bundle.workloads_from_manifests(bundle.read_manifests(args.manifests), args.suite,
                                             parse_where(args.where) or None)
    if args.only:
        ws = [w for w in ws if w.name in set(args.only)]
    if args.ci:
        skipped = [w.name for w in ws if not w.ci]
        ws = [w for w in ws if w.ci]
        print(f"--ci: {len(ws)} workloads, {len(skipped)} over the CI cap left out: {' '.join(skipped)}", flush=True)
    part = None
    if args.shard:
        k, n = (int(x) for x in args.shard.split("/"))
        total = len(ws)
        try:
            ws = shard(ws, k, n, args.suite)
        except ValueError as e:
            raise SystemExit(str(e)) from None
        part = {"index": k, "of": n, "total": total}
    done = []
    write_results(args.out, args.suite, done, len(ws), part)
    for w in ws:
        r = run_workload(w, args.reps, args.warmup, args.settle, graph=not args.eager, recorded_path=args.recorded)
        done.append(r)
        write_results(args.out, args.suite, done, len(ws), part)
        print(f"{w.name}: rc={r['rc']} us={r.get('us', float('nan')):.1f}", flush=True)
    return 0 if all(r["rc"] == 0 for r in done) else 1


if __name__ == "__main__":
    sys.exit(main())
