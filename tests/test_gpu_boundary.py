"""The reference's boundary on the GPU: bundle kernels (as manifests) run through
ptb_amd.launcher / the set_launcher-compatible hook / HipDevice over .raw files, on the inputs the
specs' make_inputs draw, checked against the oracle (bf16 tolerance 2e-2; exact families
bit-equal; full-size GEMMs and attention on sampled rows / heads).  Every distinct kernel of every
bundle workload that a HIP family serves is run (586 kernels of the 502 workloads)."""
import json
import math
from pathlib import Path

import numpy as np
import pytest
import torch

import oracle
from helpers import assert_close, bits_equal
from ptb_amd import bundle, contract, device, kernels, launcher, verify

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden"
MANIFESTS = bundle.read_manifests(GOLDEN / "bundle_manifests.json.gz")
RECORDED = GOLDEN / "recorded_inputs.npz"


def plan_family(spec):
    return kernels.resolve(spec).family


def _unique_cases():
    """(workload, kernel index) of every kernel a HIP family serves, the first workload that launches
    each distinct kernel (same name, args, grid, constexprs and scalars) standing for the others."""
    seen, out = set(), []
    for w in sorted(MANIFESTS):
        for i, m in enumerate(MANIFESTS[w]["kernels"]):
            if m["family"] is None:
                continue
            key = json.dumps({k: m.get(k) for k in ("name", "args", "grid", "constexprs", "scalars")}, sort_keys=True)
            if key not in seen:
                seen.add(key)
                out.append((w, i))
    return out


CASES = _unique_cases()


def sample(n, k=8, seed=0):
    if n <= k:
        return torch.arange(n)
    g = torch.Generator().manual_seed(seed)
    return torch.unique(torch.cat([torch.tensor([0, n - 1]), torch.randint(0, n, (k,), generator=g)]))


def check_against_oracle(plan, host, got):
    """got: name -> CPU tensor (flat) from the GPU; host: the CPU inputs."""
    p, f = plan.params, plan.family
    if f == "gemm":
        m, k, n = p["m"], p["k"], p["n"]
        rows = sample(m, 16)
        a = host[p["a"]].view(m, k)[rows]
        r = host[p["residual"]].view(m, n)[rows] if p["residual"] else None
        want = oracle.gemm(a, host[p["b"]].view(k, n), r)
        scale = float(want.float().abs().mean()) + 1e-6
        assert_close(got[p["c"]].view(m, n)[rows], want, 2e-2, 2e-2 * scale, "gemm")
    elif f == "attention":
        bh, s, d, hkv = p["batch"] * p["hq"], p["seq"], p["head_dim"], p["batch"] * p["hkv"]
        q = host[p["q"]].view(bh, s, d)
        heads = sample(bh, 2)
        k = host[p["k"]].view(hkv, s, d)
        v = host[p["v"]].view(hkv, s, d)
        g = p["hq"] // p["hkv"]
        kv_of = [(h // p["hq"]) * p["hkv"] + (h % p["hq"]) // g for h in heads.tolist()]
        want = oracle.flash_attention(q[heads], k[kv_of], v[kv_of], len(kv_of), len(kv_of), p["causal"], p["scale"])
        assert_close(got[p["o"]].view(bh, s, d)[heads], want, 2e-2, 2e-2, "attention")
    elif f == "rmsnorm":
        want = oracle.rmsnorm(host[p["x"]].view(p["rows"], p["cols"]), host[p["w"]], p["eps"])
        assert_close(got[p["y"]].view(p["rows"], p["cols"]), want, 2e-2, 2e-2, "rmsnorm")
    elif f == "qk_norm_rope":
        t, h, d = p["tokens"], p["heads"], p["head_dim"]
        want = oracle.qk_norm_rope(host[p["x"]].view(t, h, d), host[p["w"]], host[p["cos"]].view(t, d),
                                   host[p["sin"]].view(t, d), p["eps"])
        assert_close(got[p["y"]].view(h, t, d), want, 2e-2, 2e-2, "qk_norm_rope")
    elif f == "transpose":
        want = oracle.transpose_heads(host[p["x"]].view(p["d0"], p["d1"], p["inner"]))
        assert bits_equal(got[p["y"]].view(p["d1"], p["d0"], p["inner"]), want)
    elif f == "silu_mul":
        want = oracle.silu_mul(host[p["x"]].view(p["rows"], 2 * p["inter"]))
        assert_close(got[p["y"]].view(p["rows"], p["inter"]), want, 2e-2, 2e-2, "silu_mul")
    elif f == "softmax":
        if p["out_f32"]:   # fp32 probabilities: the fp32 bar
            want = oracle.softmax_rows(host[p["x"]].view(p["rows"], p["cols"]), torch.float32)
            assert_close(got[p["y"]].view(p["rows"], p["cols"]), want, 1e-5, 1e-6, "softmax fp32 out")
        else:
            want = oracle.softmax_rows(host[p["x"]].view(p["rows"], p["cols"]))
            assert_close(got[p["y"]].view(p["rows"], p["cols"]), want, 2e-2, 2e-2, "softmax")
    elif f == "reduce":
        x = host[p["x"]]
        if p["op"] == "max":
            assert torch.equal(got[p["y"]], oracle.reduce_max(x))
        else:
            bound = 1e-6 * float(x.float().abs().sum()) + 1e-6
            assert abs(float(got[p["y"]]) - float(oracle.reduce_sum(x))) <= bound
    elif f == "add_scalar":
        assert bits_equal(got[p["y"]], oracle.add_scalar(host[p["x"]], p["s"]))
    elif f == "slice_add":
        assert torch.equal(got[p["y"]], oracle.slice_add(host[p["x"]], p["first"], p["count"], p["s"]))
    elif f == "sumsq":
        x = host[p["x"]]
        y = host[p["y"]] if p["y"] else None
        terms = (x.float() + (0 if y is None else y.float())).double().pow(2).sum()
        assert abs(float(got[p["out"]]) - float(oracle.sumsq(x, y))) <= 1e-6 * float(terms) + 1e-6
    elif f == "attention_decode":
        nkv, g, s, d = p["nkv"], p["group"], p["seq"], p["head_dim"]
        want = oracle.attention_decode(host[p["q"]].view(nkv, g, d), host[p["k"]].view(nkv, s, d),
                                       host[p["v"]].view(nkv, s, d), p["scale"])
        assert_close(got[p["o"]].view(nkv, g, d), want, 2e-2, 2e-2, "attention_decode")
    elif f == "gemv":
        k, n = p["k"], p["n"]
        w = host[p["w"]].view(k, n)
        if p["mode"] == "plain":
            want = oracle.gemv(host[p["x"]], w)
        elif p["mode"] == "rms":
            want = oracle.gemv_rmsnorm(host[p["x"]], host[p["ss"]], host[p["g"]], w,
                                       add=host[p["add"]] if p["add"] else None, eps=p["eps"])
        else:
            want = oracle.gemv_silu(host[p["x"]], w, host[p["res_a"]] if p["res_a"] else None,
                                    host[p["res_b"]] if p["res_b"] else None)
        finite = want.float().isfinite()
        scale = float(want.float()[finite].abs().mean()) + 1e-6 if bool(finite.any()) else 1.0
        assert_close(got[p["y"]], want, 2e-2, 2e-2 * scale, f"gemv {p['mode']}")
    elif f in MOE_FAMILIES:
        check_moe_against_oracle(plan, host, got)
    else:
        raise AssertionError(f"no oracle for {f}")


MOE_FAMILIES = {"fill_zero", "cast", "cumsum", "group_table", "count_le", "expert_count", "rank_select", "sort",
                "topk", "gather_rows", "rms_broadcast", "combine", "normalize_rows", "row_sum", "add", "rope",
                "rmsnorm_add", "grouped_mm"}


def check_moe_against_oracle(plan, host, got):
    """The MoE layer's kernels (integer and index results exact, bf16 within 2e-2 of the output's
    scale); `host` holds every argument's initial value (inout included)."""
    p, f = plan.params, plan.family
    if f == "fill_zero":
        assert not got[p["y"]].any()
    elif f == "cast":
        assert torch.equal(got[p["y"]], oracle.cast_i64_i32(host[p["x"]]))
    elif f == "cumsum":
        want = oracle.cumsum_int(host[p["x"]], got[p["y"]].dtype)
        assert torch.equal(got[p["y"]], want) and (not p["y2"] or torch.equal(got[p["y2"]], want))
    elif f == "group_table":
        for name, want in zip(("nonempty", "starts", "rows"), oracle.group_table(host[p["ends"]])):
            assert torch.equal(got[p[name]], want), name
    elif f == "count_le":
        assert torch.equal(got[p["y"]], oracle.count_le(host[p["x"]], p["m"]))
    elif f == "expert_count":
        counts, cum = oracle.expert_count(host[p["ids"]], p["e"])
        assert torch.equal(got[p["counts"]], counts) and torch.equal(got[p["cum"]], cum)
        if p["counts2"]:
            assert torch.equal(got[p["counts2"]], counts)
    elif f == "rank_select":
        assert torch.equal(got[p["y"]], oracle.rank_select(host[p["cum"]], host[p["ids"]], p["e"]))
    elif f == "sort":
        v, i = oracle.sort_rows(host[p["x"]], p["rows"], p["descending"])
        assert torch.equal(got[p["i"]], i) and bits_equal(got[p["v"]], v)
    elif f == "topk":
        v, i = oracle.topk_rows(host[p["x"]], p["e"], p["k"], p["largest"])
        assert torch.equal(got[p["i"]], i) and torch.equal(got[p["v"]], v)
    elif f == "gather_rows":
        assert bits_equal(got[p["y"]], oracle.gather_rows(host[p["slot"]], host[p["x"]], p["k"], p["cols"]))
    elif f == "rms_broadcast":
        want = oracle.rms_broadcast(host[p["x"]], host[p["a"]], host[p["ss"]], host[p["w"]], p["rows"], p["eps"])
        assert_close(got[p["y"]], want, 2e-2, 2e-2, "rms_broadcast")
    elif f == "combine":
        io = host[p["out"]] if p["h"] else None
        want = oracle.combine(host[p["ids"]], host[p["ends"]], host[p["counts"]], host[p["rank"]], host[p["y"]],
                              host[p["w"]], p["tokens"], p["k"], p["cols"],
                              wsum=host[p["wsum"]] if p["wsum"] else None, h=host[p["h"]] if p["h"] else None, io=io)
        finite = want.float().isfinite()
        scale = float(want.float()[finite].abs().mean()) + 1e-6 if bool(finite.any()) else 1.0
        assert_close(got[p["out"]], want, 2e-2, 2e-2 * scale, "combine")
    elif f == "normalize_rows":
        assert_close(got[p["y"]], oracle.normalize_rows(host[p["x"]], p["k"]), 2e-2, 2e-2, "normalize_rows")
    elif f == "row_sum":
        want = oracle.row_sum(host[p["x"]], p["rows"])
        bound = 1e-6 * host[p["x"]].float().abs().reshape(p["rows"], -1).sum(1) + 1e-6
        assert bool(((got[p["y"]] - want).abs() <= bound).all())
    elif f == "add":
        assert bits_equal(got[p["y"]], oracle.add_bf16(host[p["a"]], host[p["b"]]))
    elif f == "rope":
        want = oracle.rope(host[p["x"]], host[p["cos"]], host[p["sin"]], p["tokens"])
        assert_close(got[p["y"]], want, 2e-2, 2e-2, "rope")
    elif f == "rmsnorm_add":
        want = oracle.rmsnorm_add(host[p["x"]], host[p["a"]], host[p["w"]], p["eps"])
        assert_close(got[p["y"]], want, 2e-2, 2e-2, "rmsnorm_add")
    elif f == "grouped_mm":
        want = oracle.grouped_mm(host[p["a"]], host[p["b"]], host[p["group"]], host[p["start"]], host[p["rows"]],
                                 p["k"], p["n"], p["stride"], c=host[p["c"]])
        finite = want.float().isfinite()
        scale = float(want.float()[finite].abs().mean()) + 1e-6 if bool(finite.any()) else 1.0
        assert_close(got[p["c"]], want, 2e-2, 2e-2 * scale, "grouped_mm")


def _device_args(spec, host, fill=None):
    """The launch's device tensors: inputs (and in/out arguments) from host; pure outputs freshly
    allocated (NaN-poisoned by the conftest allocator) or, with fill, every byte set to fill."""
    dev = {}
    for a in spec.args:
        if a.name in host:
            dev[a.name] = host[a.name].cuda()
        else:
            dev[a.name] = torch.empty(a.numel, dtype=getattr(torch, a.dtype), device="cuda")
            if fill is not None:
                dev[a.name].view(torch.uint8).fill_(fill)
    return dev


@pytest.mark.parametrize("workload,index", CASES)
def test_bundle_kernel_through_launcher(workload, index):
    """Each distinct bundle kernel against the oracle, then once more over outputs poisoned with a
    different byte pattern: the two runs must agree byte for byte, so every output byte is written by
    the kernel (a missed write would keep each run's own poison) and the result does not depend on
    the order the programs ran in -- the missing / conflicting-write checks of the reference's
    functional runtime (runtime/spike.py:310-334)."""
    man = MANIFESTS[workload]["kernels"][index]
    spec = contract.spec_from_manifest(man)
    rec = bundle.read_recorded(RECORDED, workload, man["dir"]) if man["extra"].get("recorded") else None
    host = contract.seeded_inputs(spec, torch, seed=0, recorded=rec)
    print(f"[case] {workload}/{man['dir']} {plan_family(spec)}", flush=True)
    dev = _device_args(spec, host)
    plan = launcher.launch(spec, dev, grid=tuple(man["grid"]))
    torch.cuda.synchronize()
    got = {a.name: dev[a.name].cpu() for a in spec.outputs()}
    check_against_oracle(plan, host, got)
    again = _device_args(spec, host, fill=0x5A)
    launcher.launch(spec, again, grid=tuple(man["grid"]))
    torch.cuda.synchronize()
    for a in spec.outputs():
        first = got[a.name].contiguous().view(torch.uint8)
        second = again[a.name].cpu().contiguous().view(torch.uint8)
        assert torch.equal(first, second), f"{a.name}: the two runs differ (unwritten or order-dependent bytes)"


def test_hip_launcher_hook_takes_kernel_json():
    man = MANIFESTS["qwen3_8b_layer_prefill_512x512_bf16"]["kernels"][0]   # rmsnorm
    spec = contract.spec_from_manifest(man)
    host = contract.seeded_inputs(spec, torch, seed=3)
    args = [host[a.name].cuda() if a.name in host else torch.empty(a.numel, dtype=torch.bfloat16, device="cuda")
            for a in spec.args]
    launcher.set_launcher(launcher.hip_launcher)
    try:
        fn = launcher.registered_launcher()
        # signature order with constexprs dropped: the tensors, then xnumel and r0_numel by name
        fn(b"", json.dumps(man), tuple(man["grid"]), args + [man["scalars"][0]["default"], man["scalars"][1]["default"]])
    finally:
        launcher.set_launcher(None)
    torch.cuda.synchronize()
    p = kernels.resolve(spec).params
    want = oracle.rmsnorm(host["in_ptr0"].view(p["rows"], p["cols"]), host["in_ptr1"], 1e-6)
    assert_close(args[2].cpu().view(p["rows"], p["cols"]), want, 2e-2, 2e-2, "hook rmsnorm")


def test_hip_device_over_raw_files(tmp_path):
    """HipDevice reads .raw inputs, poisons outputs, runs, writes .raw outputs; the result equals
    the launcher's bit for bit, matches the oracle on sampled rows, and passes verify.compare (the
    reference verify's allclose and report) against the oracle's full output."""
    man = MANIFESTS["qwen3_8b_layer_prefill_512x512_bf16"]["kernels"][3]   # k/v projection GEMM
    spec = contract.spec_from_manifest(man)
    host = contract.seeded_inputs(spec, torch, seed=0)
    paths = {a.name: str(tmp_path / f"{a.name}.raw") for a in spec.args}
    for a in spec.inputs():
        verify.write_raw(paths[a.name], a, host[a.name].view(torch.int16).numpy().view(np.uint16))
    device.get("hip").launch(device.Launch(str(tmp_path), man, raw_paths=paths, grid=tuple(man["grid"])))
    out = spec.outputs()[0]
    raw = verify.read_raw(paths[out.name], out)
    got = torch.from_numpy(raw.view(np.int16).copy()).view(torch.bfloat16)
    dev = {a.name: (host[a.name].cuda() if a.name in host else torch.empty(a.numel, dtype=torch.bfloat16,
                                                                             device="cuda")) for a in spec.args}
    plan = launcher.launch(spec, dev)
    torch.cuda.synchronize()
    assert bits_equal(got, dev[out.name].cpu())
    check_against_oracle(plan, host, {out.name: got})
    p = plan.params
    want = oracle.gemm(host[p["a"]].view(p["m"], p["k"]), host[p["b"]].view(p["k"], p["n"])).reshape(-1)
    ok, report = verify.compare(spec, {out.name: raw}, {out.name: want}, torch, rtol=2e-2,
                                atol=2e-2 * float(want.float().abs().mean()))
    assert ok, report


def test_qwen3_layer_from_bundle_manifests_matches_composed_oracle():
    """The 14 launches of qwen3_8b_layer_prefill_512x512_bf16, chained the way the layer's data flows
    (K00 -> K01/K03 -> K02/K04/K05 -> K06 -> K07 -> K08 -> K00 -> K09 -> K10 -> K11), against the
    oracle's Qwen3 layer on the same weights."""
    w = MANIFESTS["qwen3_8b_layer_prefill_512x512_bf16"]
    specs = {m["dir"][:2]: contract.spec_from_manifest(m) for m in w["kernels"]}
    t, hidden, hq, hkv, d, inter = 512, 4096, 32, 8, 128, 12288
    g = torch.Generator().manual_seed(5)

    def rnd(*shape, std=0.02, mean=0.0):
        return (torch.randn(*shape, generator=g) * std + mean).to(torch.bfloat16)

    x = rnd(t, hidden, std=1.0)
    wts = {"w_in": rnd(hidden, mean=1.0), "wq": rnd(hidden, hq * d), "wk": rnd(hidden, hkv * d),
           "wv": rnd(hidden, hkv * d), "w_qn": rnd(d, mean=1.0), "w_kn": rnd(d, mean=1.0), "wo": rnd(hq * d, hidden),
           "w_post": rnd(hidden, mean=1.0), "wgu": rnd(hidden, 2 * inter), "wd": rnd(inter, hidden)}
    cos, sin = oracle.rope_tables(t, d, 1.0e6)
    cu = {k: v.cuda().reshape(-1) for k, v in wts.items()}

    def run(key, **named):
        spec = specs[key]
        tens = {}
        for a in spec.args:
            tens[a.name] = named[a.name] if a.name in named else torch.empty(
                a.numel, dtype=getattr(torch, a.dtype), device="cuda")
        launcher.launch(spec, tens)
        return tens[spec.outputs()[0].name]

    xc = x.cuda().reshape(-1)
    xn = run("00", in_ptr0=xc, in_ptr1=cu["w_in"])
    q = run("01", arg_A=xn, arg_B=cu["wq"])
    k = run("03", arg_A=xn, arg_B=cu["wk"])
    v = run("03", arg_A=xn, arg_B=cu["wv"])
    qh = run("02", in_ptr0=q, in_ptr1=cu["w_qn"], in_ptr2=cos.cuda().reshape(-1), in_ptr3=sin.cuda().reshape(-1))
    kh = run("04", in_ptr0=k, in_ptr1=cu["w_kn"], in_ptr2=cos.cuda().reshape(-1), in_ptr3=sin.cuda().reshape(-1))
    vh = run("05", in_ptr0=v)
    oh = run("06", q_ptr=qh, k_ptr=kh, v_ptr=vh, o_ptr=torch.empty_like(qh))
    o = run("07", in_ptr0=oh)
    h = run("08", in_ptr0=xc, arg_A=o, arg_B=cu["wo"])
    hn = run("00", in_ptr0=h, in_ptr1=cu["w_post"])
    gu = run("09", arg_A=hn, arg_B=cu["wgu"])
    a = run("10", in_ptr0=gu)
    y = run("11", in_ptr0=h, arg_A=a, arg_B=cu["wd"])
    torch.cuda.synchronize()
    want = oracle.qwen3_layer(x, wts, cos, sin, hq, hkv, d, 1e-6, bq=512)
    rms = float(want.float().pow(2).mean().sqrt())
    assert_close(y.cpu().view(t, hidden), want, 2e-2, 2e-2 * max(1.0, rms), "qwen3 layer from manifests")
    assert math.isfinite(rms)


def test_qwen3_decode_layer_from_bundle_manifests_matches_composed_oracle():
    """The 8 launches of qwen3_8b_layer_decode_1x128_bf16 chained the way the decode layer's data
    flows (K00 -> K01 -> K02 -> K03 over the cache -> K04 -> K05 -> K06 -> K07), against the
    oracle's decode layer on the same weights and cache."""
    w = MANIFESTS["qwen3_8b_layer_decode_1x128_bf16"]
    specs = {m["dir"][:2]: contract.spec_from_manifest(m) for m in w["kernels"]}
    s, hidden, hq, hkv, d, inter = 128, 4096, 32, 8, 128, 12288
    g = torch.Generator().manual_seed(6)

    def rnd(*shape, std=0.02, mean=0.0):
        return (torch.randn(*shape, generator=g) * std + mean).to(torch.bfloat16)

    x = rnd(hidden, std=1.0)
    wts = {"w_in": rnd(hidden, mean=1.0), "wq": rnd(hidden, hq * d), "w_qn": rnd(d, mean=1.0), "wo": rnd(hq * d, hidden),
           "w_post": rnd(hidden, mean=1.0), "wgu": rnd(hidden, 2 * inter), "wd": rnd(inter, hidden)}
    kc, vc = rnd(hkv, s, d, std=1.0), rnd(hkv, s, d, std=1.0)
    cos_t, sin_t = oracle.rope_tables(s + 1, d, 1.0e6)
    cos, sin = cos_t[s].contiguous(), sin_t[s].contiguous()
    cu = {k: v.cuda().reshape(-1) for k, v in wts.items()}

    def run(key, **named):
        spec = specs[key]
        tens = {}
        for a in spec.args:
            tens[a.name] = named[a.name] if a.name in named else torch.empty(
                a.numel, dtype=getattr(torch, a.dtype), device="cuda")
        launcher.launch(spec, tens)
        return tens[spec.outputs()[0].name]

    xc = x.cuda()
    ss = run("00", in_ptr0=xc)
    q = run("01", in_ptr0=xc, in_ptr1=ss, in_ptr2=cu["w_in"], in_ptr3=cu["wq"])
    qh = run("02", in_ptr0=q, in_ptr1=cu["w_qn"], in_ptr2=cos.cuda(), in_ptr3=sin.cuda())
    o = run("03", q_ptr=qh, k_ptr=kc.cuda().reshape(-1), v_ptr=vc.cuda().reshape(-1))
    a = run("04", in_ptr0=o, in_ptr1=cu["wo"])
    ss2 = run("05", in_ptr0=xc, in_ptr1=a)
    gu = run("06", in_ptr0=xc, in_ptr1=a, in_ptr2=ss2, in_ptr3=cu["w_post"], in_ptr4=cu["wgu"])
    y = run("07", in_ptr0=gu, in_ptr1=cu["wd"], in_ptr2=xc, in_ptr3=a)
    torch.cuda.synchronize()
    want = oracle.qwen3_decode_layer(x, wts, kc, vc, cos, sin, hq, hkv, d, 1e-6)
    rms = float(want.float().pow(2).mean().sqrt())
    assert_close(y.cpu(), want, 2e-2, 2e-2 * max(1.0, rms), "qwen3 decode layer from manifests")


# ---- the spec-driven C entries (ptb_<family>_args) on three bundle kernels ----------------------
def _bundle(workload, index, seed=0):
    man = MANIFESTS[workload]["kernels"][index]
    spec = contract.spec_from_manifest(man)
    host = contract.seeded_inputs(spec, torch, seed=seed)
    dev = {a.name: (host[a.name].cuda() if a.name in host
                    else torch.empty(a.numel, dtype=getattr(torch, a.dtype), device="cuda")) for a in spec.args}
    return man, spec, host, dev


def _roles(spec):
    return [a.role for a in spec.args]


def test_args_entry_rmsnorm_bundle_kernel():
    """L2048/00 through ptb_rmsnorm_args with the spec's tensors in spec order, ints [xnumel,
    r0_numel, programs] and the whole grid; then a grid of 3 of its 8 programs, which writes the
    first 3 * 256 rows only (the rest keeps its NaN poison)."""
    from ptb_amd import capi
    man, spec, host, dev = _bundle("qwen3_8b_layer_prefill_2048x2048_bf16", 0)
    rows, cols = 2048, 4096
    tens = [dev[a.name] for a in spec.args]
    capi.call_args("rmsnorm", tens, _roles(spec), [rows, cols, spec.grid[0]], [1e-6], spec.grid)
    torch.cuda.synchronize()
    want = oracle.rmsnorm(host["in_ptr0"].view(rows, cols), host["in_ptr1"], 1e-6)
    assert_close(dev["out_ptr1"].cpu().view(rows, cols), want, 2e-2, 2e-2, "rmsnorm_args")
    part = torch.full((rows * cols,), float("nan"), dtype=torch.bfloat16, device="cuda")
    capi.call_args("rmsnorm", tens[:2] + [part], _roles(spec), [rows, cols, spec.grid[0]], [1e-6], (3, 1, 1))
    torch.cuda.synchronize()
    got = part.cpu().view(rows, cols)
    assert_close(got[: 3 * 256], want[: 3 * 256], 2e-2, 2e-2, "rmsnorm_args partial grid")
    assert torch.isnan(got[3 * 256:].float()).all()


def test_args_entry_gemm_residual_bundle_kernel():
    """L2048/08 (o-projection + residual, args [in_ptr0 residual, arg_A, arg_B, out_ptr0]) through
    ptb_gemm_args; sampled rows against the oracle with the absolute floor scaled to the output."""
    from ptb_amd import capi
    man, spec, host, dev = _bundle("qwen3_8b_layer_prefill_2048x2048_bf16", 8)
    assert [a.name for a in spec.args] == ["in_ptr0", "arg_A", "arg_B", "out_ptr0"]
    m, k, n = 2048, 4096, 4096
    capi.call_args("gemm", [dev[a.name] for a in spec.args], _roles(spec), [m, n, k, spec.grid[0]], [], spec.grid)
    torch.cuda.synchronize()
    rows = sample(m, 16)
    want = oracle.gemm(host["arg_A"].view(m, k)[rows], host["arg_B"].view(k, n),
                       host["in_ptr0"].view(m, n)[rows])
    got = dev["out_ptr0"].cpu().view(m, n)[rows]
    assert_close(got, want, 2e-2, 2e-2 * float(want.float().abs().mean()), "gemm_args residual")


def test_args_entry_attention_bundle_kernel():
    """attention_prefill_32x8x4096_bf16's _prefill_kernel through ptb_flash_attn_args: ints [batch,
    HQ, HQ / G, S, D, CAUSAL], floats [SCALE] from its constexprs, grid (32, 1, 1)."""
    from ptb_amd import capi
    man, spec, host, dev = _bundle("attention_prefill_32x8x4096_bf16", 0)
    ce = man["constexprs"]
    hq, g, s, d = ce["HQ"], ce["G"], ce["S"], ce["D"]
    capi.call_args("flash_attn", [dev[a.name] for a in spec.args], _roles(spec),
                   [1, hq, hq // g, s, d, int(ce["CAUSAL"])], [ce["SCALE"]], spec.grid)
    torch.cuda.synchronize()
    heads = torch.tensor([0, 17])
    q = host["q_ptr"].view(hq, s, d)[heads]
    k = host["k_ptr"].view(hq // g, s, d)[heads // g]
    v = host["v_ptr"].view(hq // g, s, d)[heads // g]
    want = oracle.flash_attention(q, k, v, 2, 2, True, ce["SCALE"])
    got = dev["o_ptr"].cpu().view(hq, s, d)[heads]
    from helpers import assert_close_rows
    assert_close_rows(got, want, 2e-2, 2e-2, "flash_attn_args")


@pytest.mark.parametrize("workload,index", [
    ("gemm_1x2048x128_bf16", 0),                  # gemv, plain (the M = 1 mm template)
    ("qwen3_8b_layer_decode_1x1024_bf16", 0),     # sumsq of x
    ("qwen3_8b_layer_decode_1x1024_bf16", 1),     # gemv, RMSNorm prologue
    ("qwen3_8b_layer_decode_1x1024_bf16", 4),     # gemv, plain
    ("qwen3_8b_layer_decode_1x1024_bf16", 5),     # sumsq of x + a
    ("qwen3_8b_layer_decode_1x1024_bf16", 6),     # gemv, RMSNorm prologue over x + a
    ("qwen3_8b_layer_decode_1x1024_bf16", 7),     # gemv, silu prologue + two residuals
    ("layer_layer_decode_1x1024_bf16", 18),       # reduce (sum) over fp32
    ("vector_max_1024x1024_bf16", 0),             # reduce (max) over bf16
    ("vector_sum_1024x1024_bf16", 0),             # reduce (sum) over bf16
    ("vector_add1_1024x1024_bf16", 0),            # add_scalar
    ("vector_slice_4096x4096_bf16", 0),           # slice_add
])
def test_args_entry_more_families(workload, index):
    """The sumsq, gemv, reduce, add_scalar and slice_add kernels through their ptb_<family>_args
    entries, called directly with the spec's tensors (plus the entry's workspace descriptor) and
    the whole grid, against the oracle."""
    from ptb_amd import capi
    man, spec, host, dev = _bundle(workload, index)
    plan = kernels.resolve(spec)
    fam, names, ints, floats = capi.plan_args(plan, spec.grid[0])
    roles = {a.name: a.role for a in spec.args}
    ts, rs = [dev[n] for n in names], [roles[n] for n in names]
    ws = capi.workspace_for(plan, "cuda")
    if ws is not None:
        ts, rs = ts + [ws], rs + ["out"]
    print(f"[case] {workload}/{man['dir']} {plan.family} -> ptb_{fam}_args", flush=True)
    capi.call_args(fam, ts, rs, ints, floats, spec.grid)
    torch.cuda.synchronize()
    check_against_oracle(plan, host, {a.name: dev[a.name].cpu() for a in spec.outputs()})


def test_args_entry_rmsnorm_column_arm():
    """tests/cases/workloads/rmsnorm.py:44-57 (x, w, o, c all fp32, grid (1,)): o through the row
    norm, c = rsqrt(mean over the rows of x^2 + eps) through the column arm, both within the
    reference case's fp32 bar."""
    from ptb_amd import capi
    m, n, eps = 8, 64, 1e-5
    g = torch.Generator().manual_seed(0)
    x = torch.randn(m * n, generator=g)
    w = torch.randn(n, generator=g)
    o = torch.empty(m * n, device="cuda")
    c = torch.empty(n, device="cuda")
    capi.call_args("rmsnorm", [x.cuda(), w.cuda(), o, c], ["in", "in", "out", "out"], [m, n, 1], [eps], (1, 1, 1))
    torch.cuda.synchronize()
    xr = x.view(m, n).double()
    want_o = (xr * torch.rsqrt(xr.pow(2).mean(-1, keepdim=True) + eps) * w.double()).float()
    want_c = torch.rsqrt(xr.pow(2).mean(0) + eps).float()
    assert_close(o.cpu().view(m, n), want_o, 1e-5, 1e-6, "rmsnorm_args o")
    assert_close(c.cpu(), want_c, 1e-5, 1e-6, "rmsnorm_args c")
    assert_close(c.cpu(), oracle.col_rms_f32(x.view(m, n), eps), 1e-5, 1e-6, "rmsnorm_args c vs oracle")


def test_kernel_object_rebuilt_for_other_extents():
    """A kernel object rebuilt for a launch's own extents, as the reference's _Launcher hands it over
    (pytorchsim_triton_backend/driver.py:46-65, compiler.py:200-209: every argument's shape set to
    the call's storage span, the stated scalars to the call's values): L2048/00's RMSNorm rebuilt for
    1000 rows, with a null grid_bound, launched through the set_launcher hook over the grid
    Inductor gives 1000 rows (ceil(1000 / XBLOCK)) and over a larger one (programs past the rows
    are masked no-ops), both against the oracle."""
    man = json.loads(json.dumps(MANIFESTS["qwen3_8b_layer_prefill_2048x2048_bf16"]["kernels"][0]))
    rows, cols = 1000, 4096
    for a in man["args"]:
        a["shape"] = [cols] if a["name"] == "in_ptr1" else [rows * cols]
    man["grid_bound"] = None
    xblock = man["constexprs"]["XBLOCK"]
    g = torch.Generator().manual_seed(11)
    x = torch.randn(rows * cols, generator=g).to(torch.bfloat16)
    w = (torch.randn(cols, generator=g) * 0.1 + 1).to(torch.bfloat16)
    want = oracle.rmsnorm(x.view(rows, cols), w, 1e-6)
    for grid in ((-(-rows // xblock), 1, 1), (8, 1, 1), (13, 1, 1)):
        y = torch.empty(rows * cols, dtype=torch.bfloat16, device="cuda")
        launcher.hip_launcher(b"", json.dumps(man), grid, [x.cuda(), w.cuda(), y, rows, cols])
        torch.cuda.synchronize()
        assert_close(y.cpu().view(rows, cols), want, 2e-2, 2e-2, f"rebuilt rmsnorm grid {grid}")
    # a partial grid of the rebuilt kernel covers its leading XBLOCK-row blocks only
    y = torch.empty(rows * cols, dtype=torch.bfloat16, device="cuda")
    launcher.hip_launcher(b"", json.dumps(man), (2, 1, 1), [x.cuda(), w.cuda(), y, rows, cols])
    torch.cuda.synchronize()
    got = y.cpu().view(rows, cols)
    assert_close(got[: 2 * xblock], want[: 2 * xblock], 2e-2, 2e-2, "rebuilt rmsnorm partial grid")
    assert torch.isnan(got[2 * xblock:].float()).all()
