"""Tensor-level entry points of the mixture-of-experts kernels (``csrc/moe.hip`` and the grouped
mode of ``csrc/gemm_bf16.hip``), for the Qwen3-30B-A3B layer of the validation bundle.

As in :mod:`ptb_amd.ops`, torch only owns device memory and the current stream; every function
checks dtypes and sizes, then calls the HIP kernel.  Tensors are taken flat (any shape with the
stated number of elements); outputs are written in place into the tensors given.
"""
from __future__ import annotations

import torch

from . import _lib
from .ops import BF16, F32, _need, _stream

I32 = torch.int32
I64 = torch.int64
_CODE = {BF16: _lib.PTB_DTYPE_BF16, F32: _lib.PTB_DTYPE_F32, I32: _lib.PTB_DTYPE_I32, I64: _lib.PTB_DTYPE_I64}


def _numel(t: torch.Tensor, n: int, name: str) -> None:
    if t.numel() != n:
        raise ValueError(f"{name} has {t.numel()} elements, expected {n}")


def fill_zero(out: torch.Tensor) -> torch.Tensor:
    """out[:] = 0 (any dtype), by a fill kernel: safe inside a captured graph."""
    _need(out, "out", tuple(_CODE) + (torch.uint8,))
    _lib.call("ptb_fill_zero", out.data_ptr(), out.numel() * out.element_size(), _stream(out))
    return out


def cast_i64_i32(x: torch.Tensor, out: torch.Tensor) -> torch.Tensor:
    _need(x, "x", I64)
    _need(out, "out", I32)
    _numel(out, x.numel(), "out")
    _lib.call("ptb_cast_i64_i32", x.data_ptr(), out.data_ptr(), x.numel(), _stream(x))
    return out


def cumsum(x: torch.Tensor, out: torch.Tensor, out2: torch.Tensor | None = None) -> torch.Tensor:
    """Inclusive prefix sum of int32/int64 x into int32/int64 out (and the same values into out2);
    int32 results wrap as two's complement, as a cast before an int32 scan does."""
    _need(x, "x", (I32, I64))
    _need(out, "out", (I32, I64))
    _numel(out, x.numel(), "out")
    if out2 is not None:
        _need(out2, "out2", out.dtype)
        _numel(out2, x.numel(), "out2")
    _lib.call("ptb_cumsum_int", x.data_ptr(), _CODE[x.dtype], out.data_ptr(), 0 if out2 is None else out2.data_ptr(),
              _CODE[out.dtype], x.numel(), _stream(x))
    return out


def group_table(ends: torch.Tensor, nonempty: torch.Tensor, starts: torch.Tensor, rows: torch.Tensor) -> None:
    """From inclusive group ends: starts (exclusive ends), rows per group, and the running count
    of non-empty groups; all outputs int64."""
    _need(ends, "ends", (I32, I64))
    for t, nm in ((nonempty, "nonempty"), (starts, "starts"), (rows, "rows")):
        _need(t, nm, I64)
        _numel(t, ends.numel(), nm)
    _lib.call("ptb_moe_group_table", ends.data_ptr(), _CODE[ends.dtype], ends.numel(), nonempty.data_ptr(),
              starts.data_ptr(), rows.data_ptr(), _stream(ends))


def count_le(x: torch.Tensor, out: torch.Tensor) -> torch.Tensor:
    """out[i] = number of r with x[r] <= i (int32), i < out.numel()."""
    _need(x, "x", I64)
    _need(out, "out", I32)
    _lib.call("ptb_count_le", x.data_ptr(), x.numel(), out.data_ptr(), out.numel(), _stream(out))
    return out


def expert_count(ids: torch.Tensor, counts: torch.Tensor, cum: torch.Tensor, counts2: torch.Tensor | None = None):
    """counts[x] = #{s : ids[s] == x} over E = counts.numel() experts; cum[s, x] = #{s' <= s : ids[s'] == x}."""
    _need(ids, "ids", I64)
    _need(counts, "counts", I64)
    _need(cum, "cum", I64)
    e = counts.numel()
    _numel(cum, ids.numel() * e, "cum")
    if counts2 is not None:
        _need(counts2, "counts2", I64)
        _numel(counts2, e, "counts2")
    _lib.call("ptb_moe_expert_count", ids.data_ptr(), ids.numel(), e, counts.data_ptr(),
              0 if counts2 is None else counts2.data_ptr(), cum.data_ptr(), _stream(ids))


def rank_select(cum: torch.Tensor, ids: torch.Tensor, out: torch.Tensor) -> torch.Tensor:
    """out[s] = cum[s, ids[s]] (0 where ids[s] is not an expert index)."""
    _need(cum, "cum", I64)
    _need(ids, "ids", I64)
    _need(out, "out", I64)
    r = ids.numel()
    _numel(out, r, "out")
    if r == 0 or cum.numel() % r:
        raise ValueError("cum must hold E values per slot")
    _lib.call("ptb_moe_rank_select", cum.data_ptr(), ids.data_ptr(), r, cum.numel() // r, out.data_ptr(), _stream(out))
    return out


def sort_rows(x: torch.Tensor, values: torch.Tensor, indices: torch.Tensor, rows: int, descending: bool = False,
              workspace: torch.Tensor | None = None):
    """Stable sort of each of `rows` rows of x (int64 or fp32 keys): values in order and their
    original positions (int64); equal keys keep their original order."""
    _need(x, "x", (I64, F32))
    _need(values, "values", x.dtype)
    _need(indices, "indices", I64)
    if rows <= 0 or x.numel() % rows:
        raise ValueError("x must hold rows equal-length rows")
    e = x.numel() // rows
    _numel(values, x.numel(), "values")
    _numel(indices, x.numel(), "indices")
    need = _lib.load().ptb_sort_workspace_bytes(rows, e)
    if workspace is None:
        workspace = torch.empty(max(need, 16), dtype=torch.uint8, device=x.device)
    _lib.call("ptb_sort_rows", x.data_ptr(), _CODE[x.dtype], values.data_ptr(), indices.data_ptr(), rows, e,
              int(bool(descending)), workspace.data_ptr(), workspace.numel(), _stream(x))


def topk_rows(x: torch.Tensor, values: torch.Tensor, indices: torch.Tensor, e: int, k: int, largest: bool = True):
    """Per row of e fp32 values, the k largest (smallest) in order, ties to the lowest position."""
    _need(x, "x", F32)
    _need(values, "values", F32)
    _need(indices, "indices", I64)
    if e <= 0 or x.numel() % e:
        raise ValueError("x must hold rows of e values")
    rows = x.numel() // e
    _numel(values, rows * k, "values")
    _numel(indices, rows * k, "indices")
    _lib.call("ptb_topk_rows_f32", x.data_ptr(), rows, e, k, int(bool(largest)), values.data_ptr(), indices.data_ptr(),
              _stream(x))


def gather_rows(slot: torch.Tensor, x: torch.Tensor, out: torch.Tensor, k: int, cols: int) -> torch.Tensor:
    """out[s, :] = x[floor(slot[s] / k), :] (bf16 rows of `cols`), token index wrapped as Python
    indexing does; rows whose token is out of range are written as zeros."""
    _need(slot, "slot", I64)
    _need(x, "x", BF16)
    _need(out, "out", BF16)
    r = slot.numel()
    _numel(out, r * cols, "out")
    if x.numel() % cols:
        raise ValueError("x must hold rows of cols values")
    _lib.call("ptb_moe_gather_rows_bf16", slot.data_ptr(), r, k, x.data_ptr(), x.numel() // cols, cols, out.data_ptr(),
              _stream(out))
    return out


def combine(ids, ends, counts, rank, y, w, out, tokens: int, k: int, cols: int, wsum=None, h=None) -> torch.Tensor:
    """Each token's weighted sum of its k expert rows of y (see ptb_moe_combine_bf16): bf16 weights
    w, or fp32 w normalised by wsum; with h, out = (h + out) + sum in place."""
    for t, nm in ((ids, "ids"), (ends, "ends"), (counts, "counts"), (rank, "rank")):
        _need(t, nm, I64)
    _need(y, "y", BF16)
    _need(out, "out", BF16)
    _need(w, "w", (BF16, F32))
    if w.dtype == F32:
        if wsum is None:
            raise ValueError("fp32 weights need wsum")
        _need(wsum, "wsum", F32)
        _numel(wsum, tokens, "wsum")
    elif wsum is not None:
        raise ValueError("wsum goes with fp32 weights")
    if h is not None:
        _need(h, "h", BF16)
        _numel(h, tokens * cols, "h")
    _numel(ids, tokens * k, "ids")
    _numel(rank, tokens * k, "rank")
    _numel(w, tokens * k, "w")
    _numel(out, tokens * cols, "out")
    _numel(counts, ends.numel(), "counts")
    if y.numel() % cols:
        raise ValueError("y must hold rows of cols values")
    _lib.call("ptb_moe_combine_bf16", ids.data_ptr(), ends.data_ptr(), counts.data_ptr(), rank.data_ptr(), y.data_ptr(),
              y.numel() // cols, w.data_ptr(), _CODE[w.dtype], 0 if wsum is None else wsum.data_ptr(),
              0 if h is None else h.data_ptr(), out.data_ptr(), tokens, k, ends.numel(), cols, _stream(out))
    return out


def normalize_rows(x: torch.Tensor, out: torch.Tensor, k: int) -> torch.Tensor:
    """out[r, j] = bf16(x[r, j] / sum_j x[r, j]) for fp32 rows of k."""
    _need(x, "x", F32)
    _need(out, "out", BF16)
    _numel(out, x.numel(), "out")
    _lib.call("ptb_normalize_rows_f32", x.data_ptr(), x.numel() // k, k, out.data_ptr(), 0, _stream(x))
    return out


def row_sum(x: torch.Tensor, out: torch.Tensor) -> torch.Tensor:
    """out[r] = sum_j x[r, j] for fp32 rows (out.numel() rows)."""
    _need(x, "x", F32)
    _need(out, "out", F32)
    rows = out.numel()
    if rows == 0 or x.numel() % rows:
        raise ValueError("x must hold out.numel() equal rows")
    _lib.call("ptb_normalize_rows_f32", x.data_ptr(), rows, x.numel() // rows, 0, out.data_ptr(), _stream(x))
    return out


def add(a: torch.Tensor, b: torch.Tensor, out: torch.Tensor) -> torch.Tensor:
    for t, nm in ((a, "a"), (b, "b"), (out, "out")):
        _need(t, nm, BF16)
        _numel(t, a.numel(), nm)
    _lib.call("ptb_add_bf16", a.data_ptr(), b.data_ptr(), out.data_ptr(), a.numel(), _stream(a))
    return out


def rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, out: torch.Tensor, tokens: int) -> torch.Tensor:
    """Rotate-half RoPE of x [tokens, heads, 128] (bf16) with fp32 cos/sin [tokens, 128]."""
    _need(x, "x", BF16)
    _need(out, "out", BF16)
    _need(cos, "cos", F32)
    _need(sin, "sin", F32)
    _numel(cos, tokens * 128, "cos")
    _numel(sin, tokens * 128, "sin")
    _numel(out, x.numel(), "out")
    if tokens <= 0 or x.numel() % (tokens * 128):
        raise ValueError("x must be [tokens, heads, 128]")
    _lib.call("ptb_rope_bf16", x.data_ptr(), cos.data_ptr(), sin.data_ptr(), out.data_ptr(), tokens,
              x.numel() // (tokens * 128), 128, _stream(x))
    return out


def rmsnorm_add(x: torch.Tensor, a: torch.Tensor | None, w: torch.Tensor, out: torch.Tensor, eps: float = 1e-6):
    """out = bf16( (x + a) * rsqrt(mean((x + a)^2) + eps) * w ) per row of w.numel() (a may be None)."""
    _need(x, "x", BF16)
    _need(w, "w", BF16)
    _need(out, "out", BF16)
    cols = w.numel()
    if x.numel() % cols:
        raise ValueError("x must hold rows of w.numel()")
    if a is not None:
        _need(a, "a", BF16)
        _numel(a, x.numel(), "a")
    _numel(out, x.numel(), "out")
    _lib.call("ptb_rmsnorm_add_bf16", x.data_ptr(), 0 if a is None else a.data_ptr(), w.data_ptr(), out.data_ptr(),
              x.numel() // cols, cols, float(eps), _stream(x))
    return out


def rms_broadcast(x, a, ss, w, out, eps: float = 1e-6) -> torch.Tensor:
    """out[s, :] = bf16( (x + a) * rsqrt(ss / cols + eps) * w ) for every row s of out."""
    for t, nm in ((x, "x"), (a, "a"), (w, "w"), (out, "out")):
        _need(t, nm, BF16)
    _need(ss, "ss", F32)
    cols = x.numel()
    _numel(a, cols, "a")
    _numel(w, cols, "w")
    if out.numel() % cols:
        raise ValueError("out must hold rows of x.numel()")
    _lib.call("ptb_rms_broadcast_bf16", x.data_ptr(), a.data_ptr(), ss.data_ptr(), w.data_ptr(), out.data_ptr(),
              out.numel() // cols, cols, float(eps), _stream(x))
    return out


def grouped_gemm(a, b, group, start, rows, c, k: int, n: int, weight_stride: int, workspace=None,
                 gemv: bool = True) -> torch.Tensor:
    """For each program p: C[start[g] + i, :] = A[start[g] + i, :] @ B[g] (bf16, fp32 accumulation)
    for i < rows[g], g = group[p]; B[g] is row-major [k, n] at b + g * weight_stride.  With at most
    16 rows in A (and `gemv`), the split-K GEMV form (its workspace allocated here unless given)."""
    _need(a, "a", BF16)
    _need(b, "b", BF16)
    _need(c, "c", BF16)
    for t, nm in ((group, "group"), (start, "start"), (rows, "rows")):
        _need(t, nm, I32)
    _numel(rows, start.numel(), "rows")
    if a.numel() % k or c.numel() != (a.numel() // k) * n:
        raise ValueError("a must be [R, k] and c [R, n]")
    args = (a.data_ptr(), b.data_ptr(), group.data_ptr(), start.data_ptr(), rows.data_ptr(), c.data_ptr(),
            group.numel(), start.numel(), a.numel() // k, b.numel() // weight_stride, k, n, weight_stride)
    need = _lib.load().ptb_grouped_gemm_workspace_bytes(group.numel(), a.numel() // k, k, n) if gemv else 0
    if need:
        if workspace is None:
            workspace = torch.empty(need, dtype=torch.uint8, device=a.device)
        _lib.call("ptb_grouped_gemm_bf16_ws", *args, workspace.data_ptr(),
                  workspace.numel() * workspace.element_size(), _stream(a))
    else:
        _lib.call("ptb_grouped_gemm_bf16", *args, _stream(a))
    return c
