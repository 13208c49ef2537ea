"""CPU tests of the host-side boundary: spec/manifest round trips, the seeded-input convention,
kernel-family resolution of the bundle's kernels, verify semantics, the launcher registry and the
device's error paths.  No GPU is touched."""
import json
from pathlib import Path

import numpy as np
import pytest
import torch

from ptb_amd import bundle, contract, device, kernels, launcher, verify
from ptb_amd.contract import Arg, KernelSpec

GOLDEN = Path(__file__).resolve().parent / "golden"
MANIFESTS = bundle.read_manifests(GOLDEN / "bundle_manifests.json.gz")


def spec_of(workload, i):
    return contract.spec_from_manifest(MANIFESTS[workload]["kernels"][i])


def test_arg_and_spec_basics():
    a = Arg("x", "in", "bfloat16", (4, 8))
    assert a.numel == 32 and a.nbytes == 64
    with pytest.raises(ValueError):
        Arg("x", "sideways", "bfloat16", (1,))
    with pytest.raises(ValueError):
        Arg("x", "in", "bfloat17", (1,))
    s = KernelSpec(name="k", signature={}, constexprs={}, grid=(2,),
                   args=[Arg("x", "in", "bfloat16", (8,)), Arg("y", "inout", "float32", (8,)),
                         Arg("z", "out", "float32", (8,))])
    assert [a.name for a in s.inputs()] == ["x", "y"]
    assert [a.name for a in s.outputs()] == ["y", "z"]
    assert s.parallel_axes == ("x",)
    with pytest.raises(ValueError):
        KernelSpec(name="k", signature={}, constexprs={}, grid=(1,),
                   args=[Arg("x", "in", "bfloat16", (8,)), Arg("x", "out", "bfloat16", (8,))])


def test_manifest_round_trip_keeps_scalars_and_hints():
    man = MANIFESTS["qwen3_8b_layer_prefill_2048x2048_bf16"]["kernels"][0]
    spec = contract.spec_from_manifest(man)
    again = spec.manifest()
    assert again["name"] == man["name"] and again["args"] == man["args"] and again["grid"] == man["grid"]
    assert spec.scalar_values == {"xnumel": 2048, "r0_numel": 4096}


def test_seeded_inputs_follow_the_spec_convention():
    """One generator, randn per read argument in order, cast (validation/pytorchsim/*/_spec.py:28-36)."""
    spec = spec_of("attention_prefill_24x8x1024_bf16", 0)
    got = contract.seeded_inputs(spec, torch, seed=0)
    g = torch.Generator().manual_seed(0)
    for a in spec.inputs():
        want = torch.randn(a.numel, generator=g).to(torch.bfloat16)
        assert torch.equal(got[a.name], want), a.name
    assert list(got) == [a.name for a in spec.inputs()]   # o_ptr is inout: drawn too


@pytest.mark.parametrize("workload", sorted(MANIFESTS))
def test_every_fixture_kernel_resolves_to_its_recorded_family(workload):
    for man in MANIFESTS[workload]["kernels"]:
        if man["family"] is None:
            with pytest.raises(kernels.UnsupportedKernel):
                kernels.resolve(contract.spec_from_manifest(man))
            continue
        plan = kernels.resolve(contract.spec_from_manifest(man))
        assert plan.family == man["family"], man["name"]
        flops, nbytes = kernels.work_of(plan)
        assert nbytes > 0


def test_fixture_covers_the_whole_bundle():
    """All 502 workloads; the only kernels no HIP family serves are the Qwen3-30B-A3B MoE layer
    suite's routing / grouped-GEMM kernels (validation/layer)."""
    assert len(MANIFESTS) == 502
    suites = {}
    for w in MANIFESTS.values():
        suites[w["suite"]] = suites.get(w["suite"], 0) + 1
        for m in w["kernels"]:
            assert m["family"] is not None or w["suite"] == "layer", m["name"]
    assert suites == {"vector": 228, "gemm": 110, "attention": 56, "layer": 96, "qwen3_8b": 12}


def test_workloads_from_manifests_filters_like_the_bundle_reader():
    ws = bundle.workloads_from_manifests(MANIFESTS, "gemm", {"M": 4096})
    assert ws and all(w.suite == "gemm" and str(w.keys["M"]) == "4096" for w in ws)
    w = bundle.workloads_from_manifests(MANIFESTS, "qwen3_8b", {"T": 2048, "name": "prefill"})
    assert [x.name for x in w] == ["qwen3_8b_layer_prefill_2048x2048_bf16"]
    assert len(w[0].order) == 14 and sum(k.launches for k in w[0].kernels) == 14
    assert all(kernels.resolve(k.spec, k.source).family for k in w[0].kernels)


def test_every_workload_resolves_from_its_manifest_alone():
    """The validation runner's --manifests path: no Triton source, only the manifest's hints."""
    for w in bundle.workloads_from_manifests(MANIFESTS):
        for bk in w.kernels:
            if w.suite == "layer" and bk.spec.extra["hints"] == {} and MANIFESTS[w.name]["kernels"][
                    [k.dir for k in w.kernels].index(bk.dir)]["family"] is None:
                continue
            assert kernels.resolve(bk.spec, bk.source).family, (w.name, bk.dir)


def test_qwen3_layer_plans_match_the_model_shapes():
    fams = {m["dir"][:2]: kernels.resolve(contract.spec_from_manifest(m))
            for m in MANIFESTS["qwen3_8b_layer_prefill_2048x2048_bf16"]["kernels"]}
    assert fams["00"].params == dict(rows=2048, cols=4096, eps=1e-6, x="in_ptr0", w="in_ptr1", y="out_ptr1")
    assert (fams["01"].params["m"], fams["01"].params["k"], fams["01"].params["n"]) == (2048, 4096, 4096)
    assert (fams["09"].params["n"], fams["11"].params["k"]) == (24576, 12288)
    assert fams["08"].params["residual"] == "in_ptr0" and fams["11"].params["residual"] == "in_ptr0"
    assert fams["02"].params["heads"] == 32 and fams["04"].params["heads"] == 8
    assert (fams["05"].params["d0"], fams["05"].params["d1"]) == (2048, 8)      # [T,8,D] -> [8,T,D]
    assert (fams["07"].params["d0"], fams["07"].params["d1"]) == (32, 2048)     # [32,T,D] -> [T,32,D]
    assert fams["06"].params["hkv"] == 8 and fams["06"].params["causal"]
    assert fams["10"].params["inter"] == 12288
    order = MANIFESTS["qwen3_8b_layer_prefill_2048x2048_bf16"]["order"]
    assert [d[:2] for d in order] == ["00", "01", "02", "03", "04", "03", "05", "06", "07", "08", "00", "09",
                                      "10", "11"]


def test_index_expression_parser():
    src = ("    x0 = (xindex % 128)\n    x1 = ((xindex // 128) % 2048)\n    x2 = xindex // 262144\n"
           "    x3 = xindex\n    tmp0 = tl.load(in_ptr0 + (x0 + 128*x2 + 1024*x1), None)\n")
    assert kernels._permutation_from_source(src, 2048 * 8 * 128) == (2048, 8, 128)
    bad = src.replace("1024*x1", "1000*x1")
    with pytest.raises(kernels.UnsupportedKernel):
        kernels._permutation_from_source(bad, 2048 * 8 * 128)
    assert kernels._row_length_from_source("    x0 = (xindex % 12288)\n") == 12288


def test_unsupported_kernels_fail_loudly():
    s = KernelSpec(name="mystery", signature={}, constexprs={}, grid=(1,),
                   args=[Arg("a", "in", "int32", (8,)), Arg("b", "out", "int32", (8,))])
    with pytest.raises(kernels.UnsupportedKernel):
        kernels.resolve(s)
    dec = KernelSpec(name="_decode_kernel", signature={}, grid=(8,),
                     constexprs={"HQ": 32, "G": 4, "S": 128, "D": 128},
                     args=[Arg(n, "in", "bfloat16", (8,)) for n in ("q", "k", "v")] + [Arg("o", "out", "bfloat16", (8,))])
    with pytest.raises(kernels.UnsupportedKernel):
        kernels.resolve(dec)


def test_verify_report_matches_reference_semantics():
    want = np.array([1.0, 2.0, 3.0, np.nan])
    ok, lines = verify.compare_arrays("o", want.copy(), want, 1e-4, 1e-4)
    assert ok and "PASS" in lines[0]
    got = want.copy()
    got[1] = 2.5
    ok, lines = verify.compare_arrays("o", got, want, 1e-4, 1e-4)
    assert not ok
    assert "max_abs_err = 0.5" in lines[1] and "worst at flat index 1" in lines[2]
    assert lines[3].strip().startswith("1/4")


def test_verify_compare_decodes_bf16_bits(tmp_path):
    spec = KernelSpec(name="k", signature={}, constexprs={}, grid=(1,),
                      args=[Arg("x", "in", "bfloat16", (4,)), Arg("y", "out", "bfloat16", (4,))])
    y = torch.tensor([1.0, -2.0, 0.5, 3.0]).to(torch.bfloat16)
    path = tmp_path / "y.raw"
    verify.write_raw(path, spec.arg("y"), y.view(torch.int16).numpy().view(np.uint16))
    back = verify.read_raw(path, spec.arg("y"))
    assert back.dtype == np.uint16
    ok, _ = verify.compare(spec, {"y": back}, {"y": y}, torch)
    assert ok
    with pytest.raises(ValueError):
        verify.read_raw(path, Arg("y", "out", "bfloat16", (8,)))


def test_launcher_registry_and_grid_check():
    launcher.set_launcher(None)
    with pytest.raises(RuntimeError):
        launcher.registered_launcher()
    launcher.set_launcher(launcher.hip_launcher)
    assert launcher.registered_launcher() is launcher.hip_launcher
    launcher.set_launcher(None)
    spec = spec_of("vector_add1_1024x1024_bf16", 0)
    with pytest.raises(launcher.GridMismatch):
        launcher.launch(spec, {}, grid=(7, 1, 1))
    with pytest.raises(ValueError):   # CPU tensors are refused before any launch
        launcher.launch(spec, {"in_ptr0": torch.zeros(1048576, dtype=torch.bfloat16),
                               "out_ptr0": torch.zeros(1048576, dtype=torch.bfloat16)})


def test_device_registry_and_missing_inputs(tmp_path):
    dev = device.get("hip")
    assert dev.name == "hip"
    with pytest.raises(device.DeviceError):
        device.get("spike")
    man = MANIFESTS["vector_add1_1024x1024_bf16"]["kernels"][0]
    req = device.Launch(str(tmp_path), man, raw_paths={})
    with pytest.raises(device.DeviceError):
        dev.launch(req)


def test_grid_bound_and_refusal():
    """contract/kernel_object.py:93-107: the bound is kernel.json's grid_bound where stated (a null
    or absent grid_bound, or a null axis, is unbounded: :98-100), a spec's own grid when no manifest
    is launched; an axis past it, below 1, or past the 21-bit program id is refused."""
    spec = spec_of("qwen3_8b_layer_prefill_2048x2048_bf16", 0)
    assert contract.grid_bound(spec) == contract.grid3(spec.grid)
    man = spec.manifest()
    assert contract.grid_bound(dict(man, grid_bound=[16, None, 1])) == (16, None, 1)
    assert contract.grid_bound(dict(man, grid_bound=None)) == (None, None, None)
    assert contract.grid_bound({k: v for k, v in man.items() if k != "grid_bound"}) == (None, None, None)
    # an unbounded kernel object takes a grid past its own: refused later for the CPU tensors only
    cpu = {a.name: torch.zeros(a.numel, dtype=getattr(torch, a.dtype)) for a in spec.args}
    with pytest.raises(ValueError) as e:
        launcher.launch(dict(man, grid_bound=None), cpu, grid=(spec.grid[0] * 4, 3, 1))
    assert not isinstance(e.value, launcher.GridMismatch)
    with pytest.raises(launcher.GridMismatch):
        launcher.launch(dict(man, grid_bound=list(spec.grid)), cpu, grid=(spec.grid[0] + 1, 1, 1))
    assert contract.refuse_grid_past_bound("k", (8,), (8, 1, 1)) == (8, 1, 1)
    assert contract.refuse_grid_past_bound("k", (3, 1, 1), (8, 1, 1)) == (3, 1, 1)
    for g in [(9, 1, 1), (8, 2, 1), (0, 1, 1), (8, 1, 1 << 22)]:
        with pytest.raises(contract.ObjectError):
            contract.refuse_grid_past_bound("k", g, (8, 1, None))
    with pytest.raises(launcher.GridMismatch):
        launcher.launch(spec, {}, grid=(spec.grid[0] + 1, 1, 1))


def test_manifest_spec_disagreements_refused():
    """contract/kernel_object.py:264-286: a manifest from another compile is refused by name of what
    differs, before any tensor is looked at."""
    spec = spec_of("qwen3_8b_layer_prefill_2048x2048_bf16", 0)
    man = spec.manifest()
    assert contract.disagreements(man, spec) == []
    other = json.loads(json.dumps(man))
    other["grid"] = [spec.grid[0] * 2, 1, 1]
    other["args"][0]["shape"] = [other["args"][0]["shape"][0] + 1]
    assert contract.disagreements(other, spec) == ["grid3", "numel"]
    with pytest.raises(contract.ObjectError):
        launcher.launch(spec, {}, manifest=other)
    swapped = json.loads(json.dumps(man))
    swapped["args"][0], swapped["args"][1] = swapped["args"][1], swapped["args"][0]
    assert "argv_order" in contract.disagreements(swapped, spec)


def test_hip_launcher_maps_scalars_by_name():
    """driver.py:39-44: the launcher gets the call's arguments in signature order with constexprs
    dropped; the values that are not tensors bind to the kernel object's runtime scalars in order,
    all or none, and an unknown scalar name is refused."""
    spec = spec_of("qwen3_8b_layer_prefill_2048x2048_bf16", 0)   # rmsnorm: xnumel, r0_numel
    man = spec.manifest()
    names = [s["name"] for s in man["scalars"]]
    assert names == ["xnumel", "r0_numel"]
    with pytest.raises(contract.ObjectError):   # one scalar of two
        launcher.hip_launcher(None, json.dumps(man), spec.grid, [torch.zeros(1), torch.zeros(1), torch.zeros(1), 5])
    with pytest.raises(contract.ObjectError):   # a tensor missing
        launcher.hip_launcher(None, man, spec.grid, [torch.zeros(1), torch.zeros(1), 2048, 4096])
    with pytest.raises(contract.ObjectError):
        launcher._with_scalars(spec, {"ynumel": 3})
    s2 = launcher._with_scalars(spec, {"xnumel": 1024, "r0_numel": 4096})
    assert s2.scalar_values == {"xnumel": 1024, "r0_numel": 4096}
    assert spec.scalar_values["xnumel"] == 2048      # the spec itself is unchanged


def test_ci_caps_follow_the_reference_suites():
    """--ci: the layer suite times its layers and MoE ops up to 4096 tokens and none of the dense ops
    (validation/layer/test_cap.py:16-24); qwen3_8b only its layers; gemm caps the measured MoE shapes
    at M <= 4096; vector and attention have no cap."""
    from ptb_amd import validation as v

    assert v.under_ci_cap("layer", {"section": "layer", "name": "prefill", "T": 4096, "S": 4096})
    assert v.under_ci_cap("layer", {"section": "op", "name": "combine", "T": 4096, "S": 0})
    assert not v.under_ci_cap("layer", {"section": "op", "name": "combine", "T": 8192, "S": 0})
    assert not v.under_ci_cap("layer", {"section": "op", "name": "rmsnorm", "T": 128, "S": 0})
    assert not v.under_ci_cap("layer", {"section": "layer", "name": "prefill", "T": 8192, "S": 8192})
    assert not v.under_ci_cap("qwen3_8b", {"section": "op", "name": "rmsnorm", "T": 1, "S": 0})
    assert v.under_ci_cap("qwen3_8b", {"section": "layer", "name": "decode", "T": 1, "S": 4096})
    capped = frozenset({(8192, 2048, 128), (4096, 2048, 128)})
    assert not v.under_ci_cap("gemm", {"M": 8192, "K": 2048, "N": 128}, capped)
    assert v.under_ci_cap("gemm", {"M": 4096, "K": 2048, "N": 128}, capped)
    assert v.under_ci_cap("gemm", {"M": 8192, "K": 4096, "N": 4096}, capped)
    assert v.under_ci_cap("vector", {"program": "sum", "R": 16384, "C": 8192})
    # the manifests file records the flag: the layer suite's 12 layers and 5 MoE ops x 7 token counts,
    # and the four 8192-row GEMMs the measured MoE table holds
    ws = bundle.workloads_from_manifests(MANIFESTS)
    by = {}
    for w in ws:
        by.setdefault(w.suite, []).append(w)
    assert sum(w.ci for w in by["layer"]) == 12 + 5 * 7
    assert {w.name for w in by["layer"] if w.ci and w.keys["section"] == "op"} == {
        f"layer_op_{o}_{t}x0_bf16" for o in v.CI_OPS for t in (1, 128, 256, 512, 1024, 2048, 4096)}
    assert sorted(w.name for w in by["gemm"] if not w.ci) == [
        "gemm_8192x2048x128_bf16", "gemm_8192x2048x4096_bf16", "gemm_8192x2048x512_bf16",
        "gemm_8192x4096x2048_bf16"]
    assert all(w.ci for s in ("vector", "attention", "qwen3_8b") for w in by[s])
    for w in ws:
        assert w.ci == v.under_ci_cap(w.suite, w.keys, frozenset(
            (int(x.keys["M"]), int(x.keys["K"]), int(x.keys["N"])) for x in by["gemm"] if not x.ci)), w.name


def test_shards_are_disjoint_cover_the_set_and_balance_by_cost():
    """--shard K/N (0-based): longest processing time over each suite's cost (validation/gemm/
    simulate_shapes.py:182-196); --merge refuses overlapping parts and expects the whole set."""
    from ptb_amd import validation as v

    for suite, n in (("gemm", 4), ("attention", 3), ("layer", 5), ("vector", 7)):
        ws = bundle.workloads_from_manifests(MANIFESTS, suite)
        parts = [v.shard(ws, k, n, suite) for k in range(n)]
        names = [w.name for p in parts for w in p]
        assert sorted(names) == sorted(w.name for w in ws) and len(set(names)) == len(names)
        loads = [sum(v.cost(suite, w.keys) for w in p) for p in parts]
        # LPT: no part exceeds another by more than the costliest single workload
        assert max(loads) - min(loads) <= max(v.cost(suite, w.keys) for w in ws)
        assert [w.name for w in v.shard(ws, 1, n, suite)] == [w.name for w in parts[1]]
    ws = bundle.workloads_from_manifests(MANIFESTS, "attention")
    big = max(ws, key=lambda w: v.cost("attention", w.keys))
    assert big.keys["kind"] == "prefill" and int(big.keys["S"]) == 8192 and int(big.keys["Hq"]) == 64
    assert v.shard(ws, 0, 3, "attention")[0].name == big.name
    with pytest.raises(ValueError):
        v.shard(ws, 3, 3, "attention")
    with pytest.raises(ValueError):
        v.shard(ws, -1, 3, "attention")


def test_merge_expects_the_whole_set(tmp_path):
    from ptb_amd import validation as v

    def part(k, names):
        p = tmp_path / f"r{k}.json"
        p.write_text(json.dumps({"machine": v.MI355X, "suite": "gemm", "expected": len(names),
                                 "shard": {"index": k, "of": 2, "total": 3},
                                 "shapes": [{"M": 1, "K": 2, "N": i, "kernel": n, "rc": 0} for i, n in
                                            enumerate(names)]}))
        return str(p)
    out = str(tmp_path / "all.json")
    assert v.merge([part(0, ["a", "b"]), part(1, ["c"])], out) == 0
    assert json.loads(Path(out).read_text())["expected"] == 3
    assert v.merge([part(0, ["a"]), part(1, ["c"])], out) == 1
    with pytest.raises(ValueError, match="overlap"):
        v.merge([part(0, ["a", "b"]), part(1, ["b"])], out)
