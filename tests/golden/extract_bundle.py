#!/usr/bin/env python3
"""Write the kernel manifests of every reference bundle workload as one gzipped JSON fixture.

Run in a container that has the reference checkout (default /root/reference).  It parses the
bundle's manifest.json and *_spec.py files with ptb_amd.bundle (ast, nothing imported or executed)
and stores per kernel only data: name, args (name, role, dtype, flat shape), grid, scalars,
constexprs, the launch count, the family that serves it (null when none does), the index facts
the HIP families otherwise read from the Triton source (``extra.hints``) and the arguments the
spec takes from its recorded inputs (``extra.recorded``); per workload, ``ci`` says whether its
suite's ``--ci`` times it (the gemm suite's cap reads the reference's measured Qwen3-30B-A3B
GEMM table, validation/gemm/tpu_v6e_qwen3moe_torchxla.csv, which is not at hand elsewhere).  The GPU tests and the validation runner
(``--manifests``) read these manifests where the bundle itself is absent.

The recorded inputs themselves (the MoE kernels' index tables, ``*_inputs.pt`` beside their specs,
loaded with ``torch.load(weights_only=True)``) go to ``recorded_inputs.npz`` as plain int arrays
keyed ``<workload>/<kernel dir>/<arg>``.
"""
import gzip
import json
import os
import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1] / "pytorchsim-triton-backend_amd"))

from ptb_amd import bundle, kernels, validation  # noqa: E402


def main(ref="/root/reference"):
    root = os.path.join(ref, "validation", "pytorchsim")
    capped = validation.read_capped(os.path.join(ref, "validation", validation.CAPPED_TABLE))
    out = {}
    recorded = {}
    for name in sorted(os.listdir(root)):
        if not os.path.isfile(os.path.join(root, name, "manifest.json")):
            continue
        w = bundle.load_workload(os.path.join(root, name))
        ks = []
        for bk in w.kernels:
            man = bk.spec.manifest()
            try:
                plan = kernels.resolve(bk.spec, bk.source)
            except kernels.UnsupportedKernel:
                plan = None
            man["extra"] = {"hints": kernels.kernel_hints(plan) if plan else {}}
            if (bk.spec.extra or {}).get("recorded"):
                man["extra"]["recorded"] = list(bk.spec.extra["recorded"])
                for arg, val in torch.load(_inputs_pt(root, name, bk.dir), weights_only=True).items():
                    recorded[f"{name}/{bk.dir}/{arg}"] = val.numpy()
            man["launches"] = bk.launches
            man["dir"] = bk.dir
            man["family"] = plan.family if plan else None
            ks.append(man)
        out[name] = {"suite": w.suite, "keys": w.keys, "order": w.order, "kernels": ks,
                     "ci": int(validation.under_ci_cap(w.suite, w.keys, capped))}
    path = HERE / "bundle_manifests.json.gz"
    # mtime 0 keeps the file byte-identical across runs
    with gzip.GzipFile(path, "wb", mtime=0) as fh:
        fh.write((json.dumps(out, indent=0, sort_keys=True) + "\n").encode())
    print(f"wrote {path} ({len(out)} workloads)")
    rpath = HERE / "recorded_inputs.npz"
    np.savez_compressed(rpath, **dict(sorted(recorded.items())))
    print(f"wrote {rpath} ({len(recorded)} arrays)")


def _inputs_pt(root, workload, kernel_dir):
    d = os.path.join(root, workload, kernel_dir)
    pts = [f for f in os.listdir(d) if f.endswith("_inputs.pt")]
    if len(pts) != 1:
        raise ValueError(f"{d}: expected one *_inputs.pt, found {pts}")
    return os.path.join(d, pts[0])


if __name__ == "__main__":
    main(*sys.argv[1:])
