"""Validation reports: a suite's ``results.json`` (``python -m ptb_amd.validation``) set against the
measured TPU v6e rows the reference's validation tables hold -> ``results.csv``, ``summary.md`` and
a self-contained ``report.html`` (inline SVG, nothing fetched).

The shape of the reports follows the reference's ``validation/{gemm,vector,attention,layer,qwen3_8b}/
emit_report.py``: one row per workload joined to its measured row by the suite's keys, the measured
time as those reports take it (``latency_ns`` less the measuring framework's lead-in where the table
records one: ``module_gap_us`` for GEMM, validation/gemm/emit_report.py:36-43; ``lead_in_ns`` for the
load and softmax tables, validation/vector/emit_report.py:64-77), headline chips, the failures shown
and not dropped, the largest outliers, and with ``--baseline`` each workload against an earlier run.
Where the reference puts TOGSim's simulated time beside the measured one, these reports put the time
the HIP kernels took on the MI355X (HIP-graph replay of back-to-back launches, so a kernel shorter
than a host launch is timed by the device and not by the host; ``mi355x_eager_us`` keeps the
Python-launched time), and add each workload's share of the MI355X roofline.

    python -m ptb_amd.report gemm --results results.json --out report/ --real-dir <reference>/validation
"""
from __future__ import annotations

import argparse
import csv
import datetime
import html
import json
import math
import os
import sys

from .bundle import SUITE_KEYS

WORST = 10

#: The measured tables each suite's report reads by default, relative to the reference's validation/
#: (the defaults of its emit_report.py --real / --softmax / --load / --attention options).
TABLES = {
    "gemm": ("gemm/tpu_v6e_torchxla.csv", "gemm/tpu_v6e_qwen3moe_torchxla.csv"),
    "vector": ("vector/tpu_v6e_softmax_pallas.csv", "vector/tpu_v6e_load_torchxla.csv"),
    "attention": ("attention/tpu_v6e_attention_torchxla.csv",),
    "qwen3_8b": ("qwen3_8b/tpu_v6e_qwen3_8b_layer_torchxla.csv",),
    "layer": ("layer/tpu_v6e_qwen3moe_layer_torchxla.csv",),
}
_INT_KEYS = {"M", "K", "N", "R", "C", "Hq", "Hkv", "S", "T"}

COLUMNS = ("workload", "kernels", "launches", "families", "flops", "bytes", "mi355x_us", "mi355x_eager_us", "timing",
           "v6e_us", "speedup",
           "mi355x_tflops", "mi355x_gbs", "roofline_us", "roofline_frac", "base_us", "vs_base", "v6e_status",
           "v6e_run_id", "rc", "failed_step")


def key_of(suite: str, row: dict) -> tuple:
    """The suite's key tuple of a results or table row (numbers as ints, names as text)."""
    out = []
    for k in SUITE_KEYS[suite]:
        v = row.get(k)
        if suite == "vector" and k == "program" and v is None:
            v = "softmax"          # the softmax tables have no program column
        out.append(int(v) if k in _INT_KEYS and v not in (None, "") else v)
    return tuple(out)


def measured_us(row: dict) -> float:
    """A measured row's time in us: its latency less the lead-in its table records (none for the
    attention and layer tables, which record no lead-in)."""
    us = int(row["latency_ns"]) / 1000
    if row.get("module_gap_us") not in (None, "") and "M" in row:
        us -= float(row["module_gap_us"])
    elif row.get("lead_in_ns") not in (None, ""):
        us -= float(row["lead_in_ns"]) / 1000
    return us


def measured(suite: str, paths) -> dict:
    """key -> measured row, from every table in `paths`; a key measured twice is refused, as the
    reference's measured() refuses it."""
    real = {}
    for path in paths:
        with open(path, newline="") as fh:
            for r in csv.DictReader(fh):
                k = key_of(suite, r)
                if any(v in (None, "") for v in k):
                    continue
                if k in real:
                    raise SystemExit(f"{k} is measured twice ({path})")
                real[k] = r
    return real


def kernel_work(k: dict) -> tuple:
    """(flops, bytes) of one kernel record: recorded by the runner, or recovered from its rates."""
    if "flops" in k and "bytes" in k:
        return float(k["flops"]), float(k["bytes"])
    us = k.get("us") or 0.0
    return k.get("tflops", 0.0) * us * 1e6, k.get("gbs", 0.0) * us * 1e3


def join_rows(suite: str, results: dict, real: dict, baseline: dict | None = None) -> list:
    """One row per workload of `results`: its kernels, work, MI355X time and roofline share, and the
    measured v6e time of the same key (None where the tables hold none)."""
    base = {}
    if baseline:
        base = {key_of(suite, s): s for s in baseline["shapes"]}
    rows = []
    for s in results["shapes"]:
        k = key_of(suite, s)
        ks = s.get("kernels") or []
        ok = s.get("rc") == 0
        flops = sum(kernel_work(x)[0] * x.get("launches", 1) for x in ks)
        nbytes = sum(kernel_work(x)[1] * x.get("launches", 1) for x in ks)
        us = s.get("us") if ok else None
        t = real.get(k)
        v6e = measured_us(t) if t else None
        b = base.get(k)
        base_us = b.get("us") if b and b.get("rc") == 0 else None
        row = dict(zip(SUITE_KEYS[suite], k))
        row.update({
            "workload": s.get("kernel"), "kernels": len(ks), "launches": sum(x.get("launches", 1) for x in ks),
            "families": " ".join(sorted({x.get("family", "?") for x in ks})), "flops": flops, "bytes": nbytes,
            "mi355x_us": us, "v6e_us": v6e,
            "mi355x_eager_us": sum(x["eager_us"] * x.get("launches", 1) for x in ks) if ok and all(
                "eager_us" in x for x in ks) else None,
            "timing": " ".join(sorted({x.get("timing", "eager") for x in ks})) if ok else None,
            "speedup": v6e / us if (us and v6e) else None,
            "mi355x_tflops": flops / us / 1e6 if (us and flops) else None,
            "mi355x_gbs": nbytes / us / 1e3 if (us and nbytes) else None,
            "roofline_us": s.get("roofline_us") if ok else None,
            "roofline_frac": (s["roofline_us"] / us) if (us and s.get("roofline_us")) else None,
            "base_us": base_us, "vs_base": us / base_us if (us and base_us) else None,
            "v6e_status": t.get("status") if t else None, "v6e_run_id": t.get("run_id") if t else None,
            "rc": s.get("rc"), "failed_step": s.get("failed_step")})
        rows.append(row)
    return rows


def geomean(xs):
    xs = [x for x in xs if x]
    return math.exp(sum(math.log(x) for x in xs) / len(xs)) if xs else None


def chips(rows) -> list:
    """The headline counts: (value, label)."""
    ran = [r for r in rows if r["mi355x_us"] is not None]
    paired = [r for r in ran if r["speedup"] is not None]
    fracs = sorted(r["roofline_frac"] for r in ran if r["roofline_frac"] is not None)
    gm = geomean([r["speedup"] for r in paired])
    out = [(f"{len(ran)} / {len(rows)}", "ran on MI355X"),
           (f"{sum(r['speedup'] > 1 for r in paired)} / {len(paired)}", "faster than measured v6e"),
           ("–" if gm is None else f"{gm:.2f}×", "speedup geomean (v6e ÷ MI355X)"),
           ("–" if not fracs else f"{fracs[len(fracs) // 2]:.3f}", "median roofline fraction")]
    failed = len(rows) - len(ran)
    if failed:
        out.append((f"{failed} / {len(rows)}", "failed or refused"))
    return out


def _fmt(v, spec=".3f"):
    return "–" if v is None else format(v, spec)


def emit_summary(suite: str, rows, meta) -> str:
    keys = SUITE_KEYS[suite]
    name = lambda r: "×".join(str(r[k]) for k in keys)  # noqa: E731
    cs = chips(rows)
    out = [f"### {suite} validation: MI355X (HIP) vs TPU v6e measured ({len(rows)} workloads) "
           f"@ `{meta.get('commit', 'unknown')[:12]}`", "",
           f"Ran on {meta.get('machine', 'MI355X')}; {meta.get('when', '')}.", "",
           "| " + " | ".join(label for _, label in cs) + " |", "|" + "---|" * len(cs),
           "| " + " | ".join(f"**{v}**" for v, _ in cs) + " |", ""]
    failed = [r for r in rows if r["mi355x_us"] is None]
    if failed:
        out += [f"**Failed or refused ({len(failed)})**:", ""]
        out += [f"- `{r['workload']}`: {r['failed_step'] or ''} {r['rc']}"[:240] for r in failed[:WORST]]
        if len(failed) > WORST:
            out.append(f"- … and {len(failed) - WORST} more (results.csv)")
        out.append("")
    paired = sorted((r for r in rows if r["speedup"] is not None), key=lambda r: r["speedup"])
    head = f"| {' × '.join(keys)} | kernels | v6e µs | MI355X µs | speedup | roofline frac |"
    line = "|---|---:|---:|---:|---:|---:|"
    row = lambda r: (f"| {name(r)} | {r['kernels']} | {r['v6e_us']:.2f} | {r['mi355x_us']:.2f} "  # noqa: E731
                     f"| {r['speedup']:.2f} | {_fmt(r['roofline_frac'])} |")
    if paired:
        out += [f"Slowest against v6e ({min(WORST, len(paired))} of {len(paired)}):", "", head, line]
        out += [row(r) for r in paired[:WORST]] + [""]
        out += [f"Fastest against v6e ({min(5, len(paired))}):", "", head, line]
        out += [row(r) for r in paired[::-1][:5]] + [""]
    by_fam = {}
    for r in rows:
        if r["roofline_frac"] is not None:
            by_fam.setdefault(r["families"], []).append(r)
    if by_fam:
        out += ["Roofline fraction by kernel families (median; largest workload's fraction):", "",
                "| families | workloads | median | largest workload |", "|---|---:|---:|---:|"]
        for fam, rs in sorted(by_fam.items()):
            fr = sorted(x["roofline_frac"] for x in rs)
            big = max(rs, key=lambda x: x["flops"] + x["bytes"])
            out.append(f"| {fam} | {len(rs)} | {fr[len(fr) // 2]:.3f} | {big['roofline_frac']:.3f} ({name(big)}) |")
        out.append("")
    moved = [r for r in rows if r["vs_base"] is not None]
    if moved:
        out += [f"Against the baseline run: {sum(r['vs_base'] < 0.97 for r in moved)} faster, "
                f"{sum(r['vs_base'] > 1.03 for r in moved)} slower (±3%), geomean "
                f"{geomean([r['vs_base'] for r in moved]):.3f} (this ÷ baseline).", ""]
    return "\n".join(out) + "\n"


def emit_csv(path: str, suite: str, rows) -> None:
    cols = list(SUITE_KEYS[suite]) + list(COLUMNS)
    with open(path, "w", newline="") as fh:
        w = csv.DictWriter(fh, fieldnames=cols, extrasaction="ignore")
        w.writeheader()
        w.writerows(rows)


def _scatter(rows, w=520, h=420, pad=50) -> str:
    """Inline SVG: MI355X µs against v6e µs on log axes, the diagonal = same time."""
    pts = [(r["v6e_us"], r["mi355x_us"], r["workload"]) for r in rows if r["speedup"] is not None]
    if not pts:
        return "<p>No workload has both times.</p>"
    lo = math.log10(min(min(a, b) for a, b, _ in pts)) - 0.1
    hi = math.log10(max(max(a, b) for a, b, _ in pts)) + 0.1

    def xy(a, b):
        x = pad + (math.log10(a) - lo) / (hi - lo) * (w - 2 * pad)
        y = h - pad - (math.log10(b) - lo) / (hi - lo) * (h - 2 * pad)
        return x, y

    out = [f'<svg width="{w}" height="{h}" xmlns="http://www.w3.org/2000/svg" font-size="11">',
           f'<rect x="{pad}" y="{pad}" width="{w - 2 * pad}" height="{h - 2 * pad}" fill="none" stroke="#999"/>']
    (x0, y0), (x1, y1) = xy(10 ** lo, 10 ** lo), xy(10 ** hi, 10 ** hi)
    out.append(f'<line x1="{x0:.1f}" y1="{y0:.1f}" x2="{x1:.1f}" y2="{y1:.1f}" stroke="#bbb" stroke-dasharray="4"/>')
    for d in range(math.ceil(lo), math.floor(hi) + 1):
        x, _ = xy(10 ** d, 10 ** lo)
        _, y = xy(10 ** lo, 10 ** d)
        out.append(f'<text x="{x:.1f}" y="{h - pad + 14}" text-anchor="middle">{10 ** d:g}</text>')
        out.append(f'<text x="{pad - 6}" y="{y + 4:.1f}" text-anchor="end">{10 ** d:g}</text>')
    for a, b, n in pts:
        x, y = xy(a, b)
        col = "#2a7" if b < a else "#c33"
        out.append(f'<circle cx="{x:.1f}" cy="{y:.1f}" r="3" fill="{col}"><title>{html.escape(n)}: v6e {a:.2f} µs, '
                   f'MI355X {b:.2f} µs</title></circle>')
    out.append(f'<text x="{w / 2}" y="{h - 12}" text-anchor="middle">TPU v6e measured µs</text>')
    out.append(f'<text x="14" y="{h / 2}" transform="rotate(-90 14 {h / 2})" text-anchor="middle">MI355X µs</text>')
    out.append("</svg>")
    return "\n".join(out)


def emit_html(suite: str, rows, meta) -> str:
    cols = list(SUITE_KEYS[suite]) + ["workload", "kernels", "families", "v6e_us", "mi355x_us", "speedup",
                                      "mi355x_tflops", "mi355x_gbs", "roofline_frac", "rc"]
    head = "".join(f"<th>{html.escape(c)}</th>" for c in cols)
    body = []
    for r in rows:
        cells = []
        for c in cols:
            v = r.get(c)
            cells.append(f"<td>{html.escape(_fmt(v) if isinstance(v, float) else str('–' if v is None else v))}</td>")
        body.append("<tr>" + "".join(cells) + "</tr>")
    cs = "".join(f'<div class="chip"><b>{html.escape(v)}</b><br>{html.escape(label)}</div>' for v, label in chips(rows))
    return f"""<!doctype html><html><head><meta charset="utf-8"><title>{suite} validation: MI355X vs v6e</title>
<style>body{{font-family:sans-serif;margin:20px}} table{{border-collapse:collapse;font-size:12px}}
td,th{{border:1px solid #ccc;padding:2px 6px;text-align:right}} .chip{{display:inline-block;border:1px solid #aaa;
border-radius:6px;padding:6px 10px;margin:4px;text-align:center}}</style></head><body>
<h2>{html.escape(suite)} validation: MI355X (HIP kernels) against TPU v6e measured</h2>
<p>commit {html.escape(meta.get('commit', 'unknown'))} · {html.escape(meta.get('machine', ''))} · {html.escape(meta.get('when', ''))}</p>
{cs}
<h3>Time per workload</h3>{_scatter(rows)}
<h3>Workloads</h3><table><tr>{head}</tr>{''.join(body)}</table></body></html>
"""


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description="MI355X validation results against the measured v6e tables")
    ap.add_argument("suite", choices=tuple(SUITE_KEYS))
    ap.add_argument("--results", required=True, help="results.json of python -m ptb_amd.validation")
    ap.add_argument("--out", required=True, help="report.html, summary.md and results.csv go here")
    ap.add_argument("--real", nargs="+", help="measured tables (csv); default: the suite's tables under --real-dir")
    ap.add_argument("--real-dir", help="the reference's validation/ directory holding the measured tables")
    ap.add_argument("--baseline", help="an earlier results.json to set each workload against")
    ap.add_argument("--commit", default="unknown")
    args = ap.parse_args(argv)
    paths = args.real or ([os.path.join(args.real_dir, t) for t in TABLES[args.suite]] if args.real_dir else [])
    if not paths:
        ap.error("give --real tables or --real-dir")
    with open(args.results) as fh:
        results = json.load(fh)
    if results.get("suite") != args.suite:
        ap.error(f"{args.results} holds suite {results.get('suite')!r}, not {args.suite!r}")
    baseline = None
    if args.baseline:
        with open(args.baseline) as fh:
            baseline = json.load(fh)
    rows = join_rows(args.suite, results, measured(args.suite, paths), baseline)
    machine = results.get("machine", {})
    meta = {"commit": args.commit, "machine": machine.get("name", "MI355X") if isinstance(machine, dict) else str(machine),
            "when": datetime.date.today().isoformat()}
    os.makedirs(args.out, exist_ok=True)
    with open(os.path.join(args.out, "summary.md"), "w") as fh:
        fh.write(emit_summary(args.suite, rows, meta))
    emit_csv(os.path.join(args.out, "results.csv"), args.suite, rows)
    with open(os.path.join(args.out, "report.html"), "w") as fh:
        fh.write(emit_html(args.suite, rows, meta))
    print(f"{args.suite}: {len(rows)} workloads -> {args.out}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
