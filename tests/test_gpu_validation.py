"""The validation runner (python -m ptb_amd.validation) end to end on the GPU: each suite's
workloads timed from the manifests fixture into results.json, --ci, --shard K/N and --merge
(reference: validation/gemm/simulate_shapes.py:322-352, :426-502, validation/layer/
simulate_shapes.py:30-32)."""
import json
from pathlib import Path

import pytest

from ptb_amd import validation

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden"
MAN = str(GOLDEN / "bundle_manifests.json.gz")
REC = str(GOLDEN / "recorded_inputs.npz")
QUICK = ["--reps", "3", "--warmup", "1", "--settle", "0"]


def run(tmp_path, name, argv):
    out = tmp_path / f"{name}.json"
    rc = validation.main(argv + ["--out", str(out)])
    return rc, json.loads(out.read_text())


@pytest.mark.parametrize("suite,names", [
    ("vector", ["vector_softmax_8x128_bf16", "vector_sum_16x128_bf16", "vector_slice_8x128_bf16"]),
    ("gemm", ["gemm_8x768x2048_bf16"]),
    ("attention", ["attention_decode_16x8x128_bf16", "attention_prefill_16x8x128_bf16"]),
    ("layer", ["layer_op_router_post_1x0_bf16", "layer_op_dispatch_1x0_bf16"]),
    ("qwen3_8b", ["qwen3_8b_layer_decode_1x128_bf16"]),
])
def test_each_suite_times_its_workloads(tmp_path, suite, names):
    argv = [suite, "--manifests", MAN, "--recorded", REC] + QUICK + sum((["--only", n] for n in names), [])
    rc, res = run(tmp_path, suite, argv)
    assert rc == 0
    assert res["suite"] == suite and res["expected"] == len(names)
    assert sorted(s["kernel"] for s in res["shapes"]) == sorted(names)
    for s in res["shapes"]:
        assert s["rc"] == 0 and s["failed_step"] is None, s
        assert s["us"] > 0 and s["roofline_us"] > 0 and s["kernels"]
        assert all(k["us"] > 0 and k["launches"] >= 1 for k in s["kernels"])


def test_ci_keeps_the_capped_workloads(tmp_path):
    """layer suite, ops at T = 1: --ci keeps exactly the MoE ops (CI_OPS) and drops the dense ones."""
    argv = ["layer", "--manifests", MAN, "--recorded", REC, "--ci", "--where", "section=op", "--where", "T=1"]
    rc, res = run(tmp_path, "ci", argv + QUICK)
    assert rc == 0
    assert sorted(s["name"] for s in res["shapes"]) == sorted(validation.CI_OPS)
    assert all(s["rc"] == 0 for s in res["shapes"])


def test_shards_merge_into_the_whole_set(tmp_path):
    """Two 0-based shards of the M = 8 GEMMs run separately, then --merge joins them; a missing part
    makes --merge exit 1."""
    parts = []
    for k in range(2):
        rc, res = run(tmp_path, f"part{k}", ["gemm", "--manifests", MAN, "--where", "M=8", "--shard", f"{k}/2"] + QUICK)
        assert rc == 0 and len(res["shapes"]) == 1
        assert res["shard"] == {"index": k, "of": 2, "total": 2}
        parts.append(str(tmp_path / f"part{k}.json"))
    merged = tmp_path / "merged.json"
    assert validation.main(["gemm", "--merge", *parts, "--out", str(merged)]) == 0
    res = json.loads(merged.read_text())
    assert res["expected"] == 2
    assert sorted(s["kernel"] for s in res["shapes"]) == ["gemm_8x2048x768_bf16", "gemm_8x768x2048_bf16"]
    assert validation.main(["gemm", "--merge", parts[0], "--out", str(tmp_path / "short.json")]) == 1
