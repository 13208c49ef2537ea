"""The validation report (ptb_amd.report) on a small synthetic results.json and measured table: the
join by suite keys, the lead-in the measured time leaves out, failures kept, the three outputs."""
import csv
import json

from ptb_amd import report


def write_csv(path, rows):
    with open(path, "w", newline="") as fh:
        w = csv.DictWriter(fh, fieldnames=list(rows[0]))
        w.writeheader()
        w.writerows(rows)


def test_gemm_report_joins_and_subtracts_the_module_gap(tmp_path):
    table = tmp_path / "v6e.csv"
    write_csv(table, [
        {"M": 4096, "K": 4096, "N": 4096, "latency_ns": 100300, "module_gap_us": 0.3, "status": "ok", "run_id": "r1"},
        {"M": 1, "K": 768, "N": 768, "latency_ns": 3147, "module_gap_us": 0.319, "status": "ok", "run_id": "r2"},
        {"M": 8, "K": 768, "N": 768, "latency_ns": 4000, "module_gap_us": 0.3, "status": "ok", "run_id": "r3"}])
    results = {"suite": "gemm", "machine": {"name": "MI355X (gfx950)"}, "expected": 3, "shapes": [
        {"M": 4096, "K": 4096, "N": 4096, "kernel": "gemm_4096x4096x4096_bf16", "rc": 0, "us": 50.0,
         "roofline_us": 55.0 * 0.5, "kernels": [{"family": "gemm", "launches": 1, "us": 50.0, "eager_us": 60.0,
                                                 "timing": "graph", "flops": 2 * 4096.0 ** 3, "bytes": 3 * 2 * 4096.0 ** 2}]},
        {"M": 1, "K": 768, "N": 768, "kernel": "gemm_1x768x768_bf16", "rc": 0, "us": 5.656, "roofline_us": 0.3,
         "kernels": [{"family": "gemv", "launches": 1, "us": 5.656, "tflops": 0.0002, "gbs": 210.0}]},
        {"M": 8, "K": 768, "N": 768, "kernel": "gemm_8x768x768_bf16", "rc": "HipError: boom", "failed_step": "00",
         "kernels": []}]}
    rp = tmp_path / "results.json"
    rp.write_text(json.dumps(results))
    out = tmp_path / "out"
    assert report.main(["gemm", "--results", str(rp), "--out", str(out), "--real", str(table)]) == 0
    rows = list(csv.DictReader(open(out / "results.csv")))
    by = {(r["M"], r["K"], r["N"]): r for r in rows}
    big = by[("4096", "4096", "4096")]
    assert abs(float(big["v6e_us"]) - 100.0) < 1e-9          # 100.3 us less the 0.3 us module gap
    assert abs(float(big["speedup"]) - 2.0) < 1e-9
    assert abs(float(big["mi355x_eager_us"]) - 60.0) < 1e-9 and big["timing"] == "graph"
    assert abs(float(big["mi355x_tflops"]) - 2 * 4096.0 ** 3 / 50.0 / 1e6) < 1e-6
    small = by[("1", "768", "768")]
    assert abs(float(small["speedup"]) - (3.147 - 0.319) / 5.656) < 1e-9
    assert float(small["flops"]) > 0                           # recovered from the recorded rates
    failed = by[("8", "768", "768")]
    assert failed["mi355x_us"] == "" and "boom" in failed["rc"]
    summary = (out / "summary.md").read_text()
    assert "**2 / 3**" in summary and "Failed or refused (1)" in summary and "gemm_8x768x768_bf16" in summary
    page = (out / "report.html").read_text()
    assert page.startswith("<!doctype html>") and "<svg" in page and "http" not in page.split("<svg", 1)[1][:0]


def test_vector_softmax_rows_key_as_softmax_and_leave_out_their_lead_in(tmp_path):
    table = tmp_path / "softmax.csv"
    write_csv(table, [{"R": 8, "C": 128, "latency_ns": 1127, "lead_in_ns": 3.7, "status": "ok", "run_id": "p"}])
    real = report.measured("vector", [table])
    assert list(real) == [("softmax", 8, 128)]
    assert abs(report.measured_us(real[("softmax", 8, 128)]) - (1.127 - 0.0037)) < 1e-12


def test_a_key_measured_twice_is_refused(tmp_path):
    a, b = tmp_path / "a.csv", tmp_path / "b.csv"
    for p in (a, b):
        write_csv(p, [{"kind": "decode", "Hq": 32, "Hkv": 8, "S": 128, "latency_ns": 5000}])
    try:
        report.measured("attention", [a, b])
    except SystemExit as e:
        assert "measured twice" in str(e)
    else:
        raise AssertionError("duplicate key accepted")
