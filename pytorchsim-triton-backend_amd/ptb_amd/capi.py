"""The spec-driven C entry points (``ptb_<family>_args`` in include/ptb_amd.h) from Python.

A reference kernel is called by its generated driver with one memref descriptor per tensor in spec
order, its runtime scalars and the launch grid (reference: pytorchsim_triton_compiler/codegen/
wrapper.py:37-51, :126-277).  :func:`call_args` makes the same call on the GPU: device tensors in
spec order with their roles become ``ptb_tensor`` descriptors, and the family's integer and float
parameters and the grid go alongside.  :func:`plan_args` derives those parameters from a resolved
:class:`ptb_amd.kernels.Plan` and the kernel's program bound, so the launch hooks run the hot-path
families through these entries.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib

_DTYPE = {torch.bfloat16: _lib.PTB_DTYPE_BF16, torch.float32: _lib.PTB_DTYPE_F32, torch.int32: _lib.PTB_DTYPE_I32,
          torch.int64: _lib.PTB_DTYPE_I64, torch.float8_e4m3fn: _lib.PTB_DTYPE_E4M3, torch.uint8: _lib.PTB_DTYPE_E4M3}
ROLE = {"in": _lib.PTB_ROLE_IN, "out": _lib.PTB_ROLE_OUT, "inout": _lib.PTB_ROLE_INOUT}

# the families with a ptb_<family>_args entry, by the name kernels.resolve gives them
FAMILY_ENTRY = {"rmsnorm": "rmsnorm", "softmax": "softmax", "silu_mul": "silu_mul", "gemm": "gemm",
                "attention": "flash_attn", "attention_decode": "attn_decode", "qk_norm_rope": "qk_norm_rope",
                "transpose": "transpose_heads", "sumsq": "sumsq", "gemv": "gemv", "reduce": "reduce",
                "add_scalar": "add_scalar", "slice_add": "slice_add"}
_GEMV_MODE = {"plain": 0, "rms": 1, "silu": 2}


def descriptor(t: torch.Tensor, role: str = "in") -> _lib.PtbTensor:
    """A flat, contiguous tensor as the memref-style descriptor the C entries read."""
    if t.dtype not in _DTYPE:
        raise TypeError(f"no ptb dtype for {t.dtype}")
    if not t.is_contiguous():
        raise ValueError("descriptors describe contiguous tensors")
    p = t.data_ptr()
    return _lib.PtbTensor(p, p, 0, t.numel(), 1, _DTYPE[t.dtype], ROLE[role])


def call_args(family: str, tensors, roles, ints=(), floats=(), grid=(1, 1, 1), stream: int | None = None) -> None:
    """Run ``ptb_<family>_args`` over `tensors` (spec order) with `roles` ("in" / "out" / "inout")."""
    if len(tensors) != len(roles):
        raise ValueError("one role per tensor")
    n = len(tensors)
    descs = (_lib.PtbTensor * max(n, 1))(*[descriptor(t, r) for t, r in zip(tensors, roles)])
    iv = (ctypes.c_int64 * max(len(ints), 1))(*[int(v) for v in ints])
    fv = (ctypes.c_double * max(len(floats), 1))(*[float(v) for v in floats])
    g = tuple(int(v) for v in grid) + (1,) * (3 - len(tuple(grid)))
    gv = (ctypes.c_int32 * 3)(*g)
    if stream is None:
        dev = next((t.device for t in tensors if t.device.type == "cuda"), None)
        stream = torch.cuda.current_stream(dev).cuda_stream if dev is not None else 0
    _lib.call(f"ptb_{family}_args", descs, n, iv, len(ints), fv, len(floats), gv, stream)


def plan_args(plan, programs: int, block: int | None = None):
    """(entry, tensor names in the entry's order, ints, floats) for a resolved plan whose compiled
    kernel has `programs` programs along x (of `block` rows or elements each, its XBLOCK, for the
    row-block families when stated); None for a family without a spec-driven entry."""
    p, f = plan.params, plan.family
    if f not in FAMILY_ENTRY:
        return None
    e = FAMILY_ENTRY[f]
    blk = [int(block)] if block else []
    if f == "rmsnorm":
        return e, [p["x"], p["w"], p["y"]], [p["rows"], p["cols"], programs] + blk, [p["eps"]]
    if f == "softmax":
        return e, [p["x"], p["y"]], [p["rows"], p["cols"], programs] + blk, []
    if f == "silu_mul":
        return e, [p["x"], p["y"]], [p["rows"], p["inter"], programs] + blk, []
    if f == "gemm":
        names = ([p["residual"]] if p["residual"] else []) + [p["a"], p["b"], p["c"]]
        return e, names, [p["m"], p["n"], p["k"], programs], []
    if f == "attention":
        return (e, [p["q"], p["k"], p["v"], p["o"]],
                [p["batch"], p["hq"], p["hkv"], p["seq"], p["head_dim"], int(p["causal"])], [p["scale"]])
    if f == "attention_decode":
        return e, [p["q"], p["k"], p["v"], p["o"]], [p["nkv"], p["group"], p["seq"], p["head_dim"]], [p["scale"]]
    if f == "qk_norm_rope":
        return (e, [p["x"], p["w"], p["cos"], p["sin"], p["y"]], [p["tokens"], p["heads"], p["head_dim"], programs],
                [p["eps"]])
    if f == "transpose":
        return e, [p["x"], p["y"]], [p["d0"], p["d1"], p["inner"], programs], []
    if f == "sumsq":
        return e, [p["x"]] + ([p["y"]] if p["y"] else []) + [p["out"]], [p["n"], programs], []
    if f == "gemv":
        mode = p["mode"]
        if mode == "plain":
            names, extra, floats = [p["x"], p["w"], p["y"]], 0, []
        elif mode == "rms":
            names = [p["x"]] + ([p["add"]] if p["add"] else []) + [p["ss"], p["g"], p["w"], p["y"]]
            extra, floats = (1 if p["add"] else 0), [p["eps"]]
        else:
            res = [r for r in (p["res_a"], p["res_b"]) if r]
            names, extra, floats = [p["x"], p["w"]] + res + [p["y"]], len(res), []
        return e, names, [_GEMV_MODE[mode], p["k"], p["n"], extra, programs], floats
    if f == "reduce":
        op = _lib.PTB_REDUCE_SUM if p["op"] == "sum" else _lib.PTB_REDUCE_MAX
        return e, [p["x"], p["y"]], [p["n"], op, programs], []
    if f == "add_scalar":
        return e, [p["x"], p["y"]], [p["n"], programs] + blk, [p["s"]]
    if f == "slice_add":
        return e, [p["x"], p["y"]], [p["first"], p["count"], programs], [p["s"]]
    return None


def decode_workspace(nkv: int, group: int, seq: int, device) -> torch.Tensor | None:
    """The decode attention entry's workspace descriptor tensor (None when the cache needs none)."""
    need = _lib.load().ptb_attn_decode_workspace_bytes(nkv, group, seq)
    return torch.empty(need, dtype=torch.uint8, device=device) if need else None


def workspace_for(plan, device) -> torch.Tensor | None:
    """The trailing workspace descriptor tensor a family's entry takes for this plan (None if none)."""
    p, f, lib = plan.params, plan.family, _lib.load()
    if f == "attention_decode":
        return decode_workspace(p["nkv"], p["group"], p["seq"], device)
    if f == "gemv":
        need = lib.ptb_gemv_workspace_bytes(p["k"], p["n"])
    elif f == "reduce":
        need = lib.ptb_reduce_workspace_bytes(p["n"])
    else:
        return None
    return torch.empty(need, dtype=torch.uint8, device=device) if need else None
