"""Read the reference's kernel bundle (``validation/pytorchsim/``) without running any of its code.

Each workload directory holds ``manifest.json`` -- ``{workload, suite, <keys>..., launches: [{kernel,
dir}], externs}`` -- and per launched kernel a ``<kernel>_spec.py`` (a ``KernelSpec(...)`` call with
literal arguments) beside ``<kernel>_triton.py`` (validation/gemm/simulate_shapes.py:363-405 loads
the same files).  The spec is parsed with :mod:`ast` (its keyword values are literals and ``Arg``
calls), never imported, so no reference module and no ``pytorchsim_triton_compiler`` is needed.
The Triton source is kept as text: the kernel families that need index facts read them from it.
"""
from __future__ import annotations

import ast
import gzip
import json
import os
import re
from dataclasses import dataclass, field

from .contract import Arg, KernelSpec, spec_from_manifest

SUITE_KEYS = {
    # validation/{vector,gemm,attention,layer,qwen3_8b}/simulate_shapes.py KEYS
    "vector": ("program", "R", "C"),
    "gemm": ("M", "K", "N"),
    "attention": ("kind", "Hq", "Hkv", "S"),
    "layer": ("section", "name", "T", "S"),
    "qwen3_8b": ("section", "name", "T", "S"),
}


@dataclass
class BundleKernel:
    dir: str
    spec: KernelSpec
    source: str          # the Triton kernel's text ("" when absent)
    launches: int = 1    # how many times the workload launches it


@dataclass
class Workload:
    name: str
    suite: str
    keys: dict
    kernels: list = field(default_factory=list)   # BundleKernel, in first-launch order
    order: list = field(default_factory=list)     # kernel dirs in launch order (repeats kept)
    path: str = ""
    ci: bool = True                               # under its suite's --ci cap (manifests files record it)


def _literal(node):
    if isinstance(node, ast.Call) and getattr(node.func, "id", None) == "Arg":
        vals = [ast.literal_eval(a) for a in node.args]
        kw = {k.arg: ast.literal_eval(k.value) for k in node.keywords}
        return Arg(*vals, **kw)
    if isinstance(node, (ast.List, ast.Tuple)):
        items = [_literal(e) for e in node.elts]
        return items if isinstance(node, ast.List) else tuple(items)
    return ast.literal_eval(node)


_SPEC_FIELDS = ("name", "signature", "constexprs", "args", "grid", "rtol", "atol", "parallel_axes", "extra",
                "graph_prefetch")


def parse_spec_text(text: str, where: str = "<spec>") -> KernelSpec:
    """The KernelSpec a reference kernel file declares as ``SPEC = KernelSpec(...)``, read from its
    text.  Keyword arguments that are not literals (kernel, reference, make_inputs) are skipped."""
    tree = ast.parse(text, where)
    for node in tree.body:
        if (isinstance(node, ast.Assign) and any(getattr(t, "id", None) == "SPEC" for t in node.targets)
                and isinstance(node.value, ast.Call)):
            kw = {}
            for k in node.value.keywords:
                if k.arg in _SPEC_FIELDS:
                    kw[k.arg] = _literal(k.value)
            kw.setdefault("constexprs", {})
            kw.setdefault("signature", {})
            return KernelSpec(**kw)
    raise ValueError(f"{where}: no SPEC = KernelSpec(...) assignment")


_RECORDED = re.compile(r"out\[\s*'(\w+)'\s*\]\s*=\s*recorded\[")


def recorded_args(spec_text: str) -> list:
    """Arguments a spec's make_inputs takes from its recorded ``*_inputs.pt`` (``out['x'] =
    recorded['x']``) rather than from the seeded generator, in argument order."""
    return _RECORDED.findall(spec_text)


def read_recorded(path: str, workload: str, kernel_dir: str) -> dict:
    """The recorded inputs of one bundle kernel from a recorded-inputs file (``.npz`` written by
    tests/golden/extract_bundle.py: keys ``<workload>/<kernel dir>/<arg>``), as numpy arrays."""
    import numpy as np

    pre = f"{workload}/{kernel_dir}/"
    with np.load(path, allow_pickle=False) as z:
        return {k[len(pre):]: z[k] for k in z.files if k.startswith(pre)}


def load_kernel_dir(path: str) -> tuple:
    """(spec, triton source text) of one bundle kernel directory."""
    specs = sorted(f for f in os.listdir(path) if f.endswith("_spec.py"))
    if len(specs) != 1:
        raise ValueError(f"{path}: expected one *_spec.py, found {specs}")
    with open(os.path.join(path, specs[0])) as fh:
        text = fh.read()
    spec = parse_spec_text(text, specs[0])
    rec = recorded_args(text)
    if rec:
        spec.extra = dict(spec.extra or {}, recorded=rec)
    src = ""
    tri = specs[0][: -len("_spec.py")] + "_triton.py"
    if os.path.exists(os.path.join(path, tri)):
        with open(os.path.join(path, tri)) as fh:
            src = fh.read()
    return spec, src


def load_workload(path: str) -> Workload:
    with open(os.path.join(path, "manifest.json")) as fh:
        man = json.load(fh)
    suite = man.get("suite", "")
    keys = {k: man[k] for k in SUITE_KEYS.get(suite, ()) if k in man}
    w = Workload(name=man["workload"], suite=suite, keys=keys, path=path)
    seen = {}
    for launch in man["launches"]:
        d = launch["dir"]
        w.order.append(d)
        if d in seen:
            seen[d].launches += 1
            continue
        spec, src = load_kernel_dir(os.path.join(path, d))
        bk = BundleKernel(dir=d, spec=spec, source=src)
        seen[d] = bk
        w.kernels.append(bk)
    return w


def load_bundle(bundle_dir: str, suite: str | None = None, where=None) -> list:
    """Every workload under `bundle_dir` (optionally of one suite, and matching `where`, a dict of
    key -> value or a callable), sorted by name."""
    out = []
    for name in sorted(os.listdir(bundle_dir)):
        p = os.path.join(bundle_dir, name)
        if not os.path.isfile(os.path.join(p, "manifest.json")):
            continue
        with open(os.path.join(p, "manifest.json")) as fh:
            man = json.load(fh)
        if suite and man.get("suite") != suite:
            continue
        if isinstance(where, dict) and any(str(man.get(k)) != str(v) for k, v in where.items()):
            continue
        if callable(where) and not where(man):
            continue
        out.append(load_workload(p))
    return out


def read_manifests(path: str) -> dict:
    """A manifests file (``.json`` or ``.json.gz``): workload name -> {suite, keys, order, kernels},
    each kernel a manifest dict (``KernelSpec.manifest()`` plus ``extra.hints``, ``launches``,
    ``dir``) -- the bundle's facts without its directory tree."""
    opener = gzip.open if str(path).endswith(".gz") else open
    with opener(path, "rt") as fh:
        return json.load(fh)


def workloads_from_manifests(data: dict, suite: str | None = None, where=None) -> list:
    """The workloads of a manifests file as :class:`Workload` objects (the Triton source is absent;
    kernels that need index facts carry them as ``extra.hints``), filtered as :func:`load_bundle`."""
    out = []
    for name in sorted(data):
        w = data[name]
        if suite and w["suite"] != suite:
            continue
        if isinstance(where, dict) and any(str(w["keys"].get(k)) != str(v) for k, v in where.items()):
            continue
        if callable(where) and not where(dict(w["keys"], workload=name, suite=w["suite"])):
            continue
        wl = Workload(name=name, suite=w["suite"], keys=dict(w["keys"]), order=list(w["order"]),
                      ci=bool(w.get("ci", 1)))
        for man in w["kernels"]:
            wl.kernels.append(BundleKernel(dir=man["dir"], spec=spec_from_manifest(man), source="",
                                           launches=int(man.get("launches", 1))))
        out.append(wl)
    return out
