#!/usr/bin/env python3
"""Write the kernel manifests of a few reference bundle workloads as JSON fixtures.

Run in a container that has the reference checkout (default /root/reference).  It parses the
bundle's manifest.json and *_spec.py files with ptb_amd.bundle (ast, nothing imported or executed)
and stores per kernel only data: name, args (name, role, dtype, flat shape), grid, scalars,
constexprs, the launch count, and the index facts the HIP families otherwise read from the Triton
source (``extra.hints``).  The GPU tests run these manifests through ptb_amd.launcher.
"""
import json
import os
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1] / "pytorchsim-triton-backend_amd"))

from ptb_amd import bundle, kernels  # noqa: E402

WORKLOADS = [
    "qwen3_8b_layer_prefill_2048x2048_bf16",
    "qwen3_8b_layer_prefill_512x512_bf16",
    "attention_prefill_32x8x4096_bf16",
    "attention_prefill_24x8x1024_bf16",
    "vector_softmax_2048x6144_bf16",
    "vector_softmax_1x8192_bf16",
    "vector_sum_1024x1024_bf16",
    "vector_max_1024x1024_bf16",
    "vector_add1_1024x1024_bf16",
    "gemm_1x768x768_bf16",
    "gemm_512x768x768_bf16",
    "gemm_4096x4096x4096_bf16",
    "qwen3_8b_layer_decode_1x4096_bf16",
    "qwen3_8b_layer_decode_1x128_bf16",
    "attention_decode_32x8x4096_bf16",
    "attention_decode_24x8x1024_bf16",
    "vector_slice_8x128_bf16",
]


def main(ref="/root/reference"):
    root = os.path.join(ref, "validation", "pytorchsim")
    out = {}
    for name in WORKLOADS:
        w = bundle.load_workload(os.path.join(root, name))
        ks = []
        for bk in w.kernels:
            plan = kernels.resolve(bk.spec, bk.source)
            man = bk.spec.manifest()
            man["extra"] = {"hints": kernels.kernel_hints(plan)}
            man["launches"] = bk.launches
            man["dir"] = bk.dir
            man["family"] = plan.family
            ks.append(man)
        out[name] = {"suite": w.suite, "keys": w.keys, "order": w.order, "kernels": ks}
    path = HERE / "bundle_manifests.json"
    path.write_text(json.dumps(out, indent=1) + "\n")
    print(f"wrote {path} ({len(out)} workloads)")


if __name__ == "__main__":
    main(*sys.argv[1:])
