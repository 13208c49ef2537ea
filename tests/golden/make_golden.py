#!/usr/bin/env python3
"""Write tests/golden/golden.safetensors: small seeded inputs, the oracle's outputs (a lock on the
oracle: any later change to its arithmetic shows up as a mismatch) and, beside them, the same
quantities from independent fp64 library computations (torch.nn.functional in float64), which
tests/test_oracle.py also compares.  Shapes follow the reference's own test cases
(tests/cases/workloads/{rmsnorm,softmax,swiglu,attention,qk_norm,rope}.py sizes, bf16 operands)."""
import math
import sys
from pathlib import Path

import torch
import torch.nn.functional as F
from safetensors.torch import save_file

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))

import oracle  # noqa: E402


def rnd(shape, seed, dtype=torch.bfloat16, std=1.0, mean=0.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * std + mean).to(dtype)


def main():
    t = {}
    x, w = rnd((32, 256), 0), rnd((256,), 1, torch.float32, 0.02, 1.0)
    t["rmsnorm.x"], t["rmsnorm.w"] = x, w
    t["rmsnorm.y"] = oracle.rmsnorm(x, w, 1e-6)
    t["rmsnorm.y64"] = F.rms_norm(x.double(), (256,), w.double(), 1e-6).to(torch.bfloat16)
    s = rnd((256, 64), 2)
    t["softmax.x"], t["softmax.y"] = s, oracle.softmax_rows(s)
    gu = rnd((16, 2 * 64), 3)
    t["silu.gu"], t["silu.y"] = gu, oracle.silu_mul(gu)
    rx, rw = rnd((16, 4, 128), 4), rnd((128,), 5)
    cos, sin = oracle.rope_tables(16, 128, 1.0e6)
    t["rope.x"], t["rope.w"], t["rope.cos"], t["rope.sin"] = rx, rw, cos, sin
    t["rope.y"] = oracle.qk_norm_rope(rx, rw, cos, sin, 1e-6)
    a, b, r = rnd((16, 64), 6, std=0.125), rnd((64, 32), 7, std=0.125), rnd((16, 32), 8)
    t["gemm.a"], t["gemm.b"], t["gemm.r"], t["gemm.c"] = a, b, r, oracle.gemm(a, b, r)
    fx = rnd((8, 128), 9)
    xq, sx = oracle.quant_rows_e4m3(fx)
    t["fp8.x"], t["fp8.xq"], t["fp8.sx"] = fx, xq.view(torch.uint8), sx
    q, k, v = rnd((4, 128, 128), 10), rnd((2, 128, 128), 11), rnd((2, 128, 128), 12)
    t["attn.q"], t["attn.k"], t["attn.v"] = q, k, v
    t["attn.o"] = oracle.flash_attention(q, k, v, 4, 2, True, 1 / math.sqrt(128), bq=128, bkv=128)
    kk, vv = k.double().repeat_interleave(2, 0), v.double().repeat_interleave(2, 0)
    t["attn.o64"] = F.scaled_dot_product_attention(q.double(), kk, vv, is_causal=True,
                                                   scale=1 / math.sqrt(128)).to(torch.bfloat16)
    save_file({k: v.contiguous() for k, v in t.items()}, str(HERE / "golden.safetensors"))
    print("wrote", HERE / "golden.safetensors", sum(v.numel() * v.element_size() for v in t.values()), "bytes")


if __name__ == "__main__":
    main()
