"""Output comparison with the reference's verify semantics (tests/runtime/verify.py:28-69).

For every written argument: ``allclose(got, want, rtol, atol, equal_nan=True)`` in float, plus a
report of max_abs_err, max_rel_err (denominator max(|want|, 1e-12)), the worst index with both
values, and how many elements fall outside the tolerance.  bf16 / fp8 outputs are compared as the
float values their bits encode.  ``.raw`` files carry bf16 as uint16 bits and fp8 as uint8 bits.
"""
from __future__ import annotations

import numpy as np

from .contract import NP_DTYPE, KernelSpec

_BITS_AS = {"bfloat16": "bfloat16", "float8_e4m3fn": "float8_e4m3fn", "float8_e5m2": "float8_e5m2"}


def read_raw(path, arg) -> np.ndarray:
    """One argument's values from its .raw file, in the numpy carrier dtype."""
    data = np.fromfile(path, dtype=np.dtype(NP_DTYPE[arg.dtype]), count=arg.numel)
    if data.size != arg.numel:
        raise ValueError(f"{path}: read {data.size} elements, expected {arg.numel} "
                         f"(file truncated -- did the kernel write its output?)")
    return data.reshape(arg.shape)


def write_raw(path, arg, array) -> None:
    np.ascontiguousarray(array).astype(np.dtype(NP_DTYPE[arg.dtype]), copy=False).tofile(path)


def as_float(torch, value, dtype: str):
    """A float64 numpy view of a tensor/array whose elements are `dtype` (bit carriers decoded)."""
    if isinstance(value, np.ndarray):
        value = torch.from_numpy(np.ascontiguousarray(value))
    t = value.detach().cpu().contiguous()
    if dtype in _BITS_AS and t.dtype != getattr(torch, _BITS_AS[dtype]):
        t = t.view(getattr(torch, _BITS_AS[dtype]))
    return t.to(torch.float64).numpy()


def compare_arrays(name, got, want, rtol, atol, shape=None, dtype=""):
    """(ok, report lines) for one argument; got/want are float64 arrays of the same size."""
    g64 = np.asarray(got, dtype=np.float64).reshape(-1)
    w64 = np.asarray(want, dtype=np.float64).reshape(-1)
    if g64.size != w64.size:
        return False, [f"  {name:<10} FAIL  size {g64.size} != {w64.size}"]
    both_nan = np.isnan(g64) & np.isnan(w64)
    close = np.isclose(g64, w64, rtol=rtol, atol=atol, equal_nan=True)
    ok = bool(close.all())
    same = (g64 == w64) | both_nan
    diff = np.where(same, 0.0, np.abs(g64 - w64))
    diff = np.where(np.isnan(diff), np.inf, diff)
    rel = diff / np.maximum(np.abs(w64), 1e-12)
    lines = [f"  {name:<10} {'PASS' if ok else 'FAIL'}  shape={tuple(shape) if shape else (g64.size,)} dtype={dtype}",
             f"    max_abs_err = {diff.max() if diff.size else 0:.6g}   max_rel_err = {rel.max() if rel.size else 0:.6g}"
             f"   (rtol={rtol}, atol={atol})"]
    if not ok and diff.size:
        idx = int(np.argmax(diff))
        lines.append(f"    worst at flat index {idx}: got={g64[idx]!r}  want={w64[idx]!r}")
        lines.append(f"    {int((~close).sum())}/{diff.size} elements outside tolerance")
    return ok, lines


def compare(spec: KernelSpec, got: dict, want: dict, torch, rtol=None, atol=None):
    """(all_ok, lines) over the spec's written arguments; got/want map names to tensors or arrays."""
    rtol = spec.rtol if rtol is None else rtol
    atol = spec.atol if atol is None else atol
    all_ok, lines = True, []
    for arg in spec.outputs():
        if arg.name not in want:
            continue
        ok, ls = compare_arrays(arg.name, as_float(torch, got[arg.name], arg.dtype),
                                as_float(torch, want[arg.name], arg.dtype), rtol, atol, arg.shape, arg.dtype)
        all_ok &= ok
        lines += ls
    return all_ok, lines
