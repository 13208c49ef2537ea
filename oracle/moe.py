"""torch-CPU restatement of the Qwen3-30B-A3B (MoE) layer's kernels (test infrastructure only).

Paths are relative to ``validation/pytorchsim/`` of the reference; ``LOP_<op>`` stands for
``layer_op_<op>_1024x0_bf16`` and ``LL`` for ``layer_layer_prefill_1024x1024_bf16`` (the other
token counts differ only in their sizes).  Integer results are exact; floating point is fp32 with
one bf16 rounding where the reference stores bf16.  Where the reference's kernel would stop on a
device_assert (an index outside its table), these functions return zeros for that element, as the
HIP kernels do.
"""
from __future__ import annotations

import torch

BF16 = torch.bfloat16
F32 = torch.float32
I32 = torch.int32
I64 = torch.int64

__all__ = [
    "fill_zero", "cast_i64_i32", "cumsum_int", "group_table", "count_le", "expert_count", "rank_select",
    "sort_rows", "topk_rows", "gather_rows", "combine", "normalize_rows", "row_sum", "add_bf16", "rope",
    "rmsnorm_add", "rms_broadcast", "grouped_mm",
]


def fill_zero(n: int, dtype=I64) -> torch.Tensor:
    """LOP_gmm_gate_up/00_..._fused_new_zeros_q6uym5lr_triton.py: out[0] = 0 (int64)."""
    return torch.zeros(n, dtype=dtype)


def cast_i64_i32(x: torch.Tensor) -> torch.Tensor:
    """LOP_gmm_gate_up/04_..._fused__to_copy_oeoxw6br_triton.py: int64 -> int32 (two's-complement wrap)."""
    return x.to(I32)


def cumsum_int(x: torch.Tensor, out_dtype=I64) -> torch.Tensor:
    """LOP_gmm_gate_up/01_..._fused_cumsum_6fi3sv3v (int32 scan), LOP_combine/01_..._fused_cumsum_qi2bfo64
    (int64 scan), LL/08_..._fused__to_copy_cumsum_ggousx36 (cast to int32, then an int32 scan):
    the inclusive prefix sum in the output's width (int32 wraps)."""
    return torch.cumsum(x.to(out_dtype), 0, dtype=out_dtype)


def group_table(ends: torch.Tensor):
    """LOP_gmm_gate_up/02_..._fused__to_copy_cat_cumsum_gt_new_zeros_slice_sub_gnib2ocx_triton.py:
    starts[i] = ends[i-1] (0 for i = 0) (:37-50), rows = ends - starts (:51), nonempty = inclusive
    count of rows > 0 (:52-57).  Returns (nonempty, starts, rows), all int64."""
    e = ends.to(I64)
    starts = torch.cat([torch.zeros(1, dtype=I64), e[:-1]])
    rows = e - starts
    return torch.cumsum((rows > 0).to(I64), 0), starts, rows


def count_le(x: torch.Tensor, m: int) -> torch.Tensor:
    """LOP_gmm_gate_up/03_..._fused__to_copy_arange_le_sum_unsqueeze_j72wougd_triton.py: out[i] =
    sum_r (x[r] <= i), i < m, as int32 (:27-35)."""
    i = torch.arange(m, dtype=I64)
    return (x.to(I64)[None, :] <= i[:, None]).sum(1).to(I32)


def expert_count(ids: torch.Tensor, e: int):
    """LOP_combine/00_..._fused__to_copy_arange_cumsum_eq_sum_unsqueeze_view_dmnbvm2a_triton.py:
    counts[x] = sum_r (ids[r] == x) (:35-40, :53-54) and cum[r, x] = inclusive scan over r of
    (ids[r] == x) (:41-50), stored at x + E*r.  Returns (counts [E], cum [R*E]), int64."""
    onehot = (ids.to(I64)[:, None] == torch.arange(e, dtype=I64)[None, :]).to(I64)
    return onehot.sum(0), torch.cumsum(onehot, 0).reshape(-1)


def rank_select(cum: torch.Tensor, ids: torch.Tensor, e: int) -> torch.Tensor:
    """LOP_combine/02_..._fused__to_copy_arange_eq_mul_sum_unsqueeze_view_dmbn5ao4_triton.py:
    out[s] = sum_j cum[s, j] * (ids[s] == j) = cum[s, ids[s]] (0 when ids[s] is not in [0, E))."""
    c = cum.reshape(-1, e)
    idx = ids.to(I64)
    ok = (idx >= 0) & (idx < e)
    got = c.gather(1, idx.clamp(0, e - 1)[:, None])[:, 0]
    return torch.where(ok, got, torch.zeros_like(got))


def _sort_keys(x: torch.Tensor, descending: bool) -> torch.Tensor:
    """LOP_dispatch/00__sort_kernel/_sort_kernel_triton.py:11-20: the int64 key of each element."""
    if x.dtype == F32:
        b = x.view(torch.int32).clone()
        b = torch.where(x != x, torch.full_like(b, 0x7FC00000), b)
        b = torch.where(x == 0, torch.zeros_like(b), b)
        b = b ^ ((b >> 31) & 0x7FFFFFFF)
        k = b.to(I64)
    else:
        k = x.to(I64)
    return ~k if descending else k


def sort_rows(x: torch.Tensor, rows: int, descending: bool = False):
    """LOP_dispatch/00__sort_kernel/_sort_kernel_triton.py:4-49: per row, the bitonic network orders
    (key, original position) pairs (the tie rule :38-40), so the result is the stable sort by key;
    values come back through the inverse key map (:41-47).  Returns (values, indices int64)."""
    xr = x.reshape(rows, -1)
    keys = _sort_keys(xr, descending)
    sk, order = torch.sort(keys, dim=1, stable=True)
    if descending:
        sk = ~sk
    if x.dtype == F32:
        b = sk.to(I32)
        b = b ^ ((b >> 31) & 0x7FFFFFFF)
        vals = b.view(F32)
    else:
        vals = sk
    return vals.reshape(-1), order.to(I64).reshape(-1)


def topk_rows(x: torch.Tensor, e: int, k: int, largest: bool = True):
    """LOP_router_post/01__topk_kernel/_topk_kernel_triton.py:4-28, round by round: columns past
    the row and taken columns hold the spent value, -inf (+inf for the smallest, :10-14); each of
    the k rounds takes the row's max (min, :18-21), the lowest column holding it (:22), records
    both (:23-24) and marks that column spent (:25).  A column that holds the spent value itself is
    therefore never reported by its own index: once only spent values remain, every further round
    reports (spent, column 0), column 0 then holding the spent value.  Equal values (-0 == +0
    included) go by lower column.  A NaN, which the reference's comparisons leave to its backend,
    is ranked below every number and above the spent value, NaNs among themselves by column
    (parity unpinned for NaN); a taken element is reported with its own value (for +-0 the
    reference reports the max's zero, whose sign is the backend's).  Returns (values [rows*k]
    fp32, indices [rows*k] int64)."""
    xr = x.reshape(-1, e).float()
    rows = xr.shape[0]
    spent = float("-inf") if largest else float("inf")
    # the rounds run on fp64 keys, larger first: NaN sits below every fp32 number, above -inf
    key = (xr if largest else -xr).double()
    key = torch.where(torch.isnan(xr), torch.full_like(key, -1.7e308), key)
    cols = torch.arange(e).expand(rows, e)
    r = torch.arange(rows)
    vals = torch.empty(rows, k, dtype=F32)
    idxs = torch.empty(rows, k, dtype=I64)
    for n in range(k):
        best = key.max(dim=1).values
        at = torch.where(key == best[:, None], cols, e).min(dim=1).values
        vals[:, n] = torch.where(best == float("-inf"), torch.full((rows,), spent), xr[r, at])
        idxs[:, n] = at
        key[r, at] = float("-inf")
    return vals.reshape(-1).contiguous(), idxs.reshape(-1).contiguous()


def gather_rows(slot: torch.Tensor, x: torch.Tensor, k: int, cols: int) -> torch.Tensor:
    """LOP_dispatch/01_..._fused_floor_divide_index_select_guslzqr3_triton.py:17-42: out[s, c] =
    x[floor(slot[s] / k), c] (Python floor division :21-35; negative token indices wrap :36-38)."""
    xr = x.reshape(-1, cols)
    t = xr.shape[0]
    src = torch.div(slot.to(I64), k, rounding_mode="floor")
    src = torch.where(src < 0, src + t, src)
    ok = (src >= 0) & (src < t)
    out = xr[src.clamp(0, max(t - 1, 0))]
    out[~ok] = 0
    return out.reshape(-1)


def combine(ids, ends, counts, rank, y, w, tokens: int, k: int, cols: int, wsum=None, h=None, io=None):
    """Slot s = t*k + j of expert id = ids[s] (wrapped into [0, E)) sits at row ends[id] - counts[id]
    + rank[s] - 1 of y (wrapped into [0, rows)).  LOP_combine/03_..._jskr7oe3_triton.py:25-54: out =
    bf16(sum_j y[row] * float(w[s])) with bf16 w; LL/27_..._pjwo6jhr_triton.py:26-63: io =
    bf16((h + io) + sum_j y[row] * (w[s] / wsum[t])) with fp32 w.  fp32 throughout."""
    e = ends.numel()
    yr = y.reshape(-1, cols).float()
    ny = yr.shape[0]
    idv = ids.to(I64).reshape(tokens, k)
    idw = torch.where(idv < 0, idv + e, idv)
    ok = (idw >= 0) & (idw < e)
    idc = idw.clamp(0, e - 1)
    row = ends.to(I64)[idc] - counts.to(I64)[idc] + rank.to(I64).reshape(tokens, k) - 1
    row = torch.where(row < 0, row + ny, row)
    ok = ok & (row >= 0) & (row < ny)
    if wsum is not None:
        wt = w.float().reshape(tokens, k) / wsum.float()[:, None]
    else:
        wt = w.float().reshape(tokens, k)
    acc = torch.zeros(tokens, cols, dtype=F32)
    rowc = row.clamp(0, ny - 1)
    for j in range(k):
        acc = acc + yr[rowc[:, j]] * wt[:, j:j + 1]
    if h is not None:
        acc = (h.float().reshape(tokens, cols) + io.float().reshape(tokens, cols)) + acc
    acc[~ok.all(1)] = 0
    return acc.to(BF16).reshape(-1)


def normalize_rows(x: torch.Tensor, k: int) -> torch.Tensor:
    """LOP_router_post/02_..._fused__to_copy_div_sum_d4c5sb6k_triton.py: bf16(x / sum_j x) per row of k."""
    xr = x.float().reshape(-1, k)
    return (xr / xr.sum(1, keepdim=True)).to(BF16).reshape(-1)


def row_sum(x: torch.Tensor, rows: int) -> torch.Tensor:
    """LL/22_..._fused_sum_kon7yqsn_triton.py: fp32 row sums of [rows, k]."""
    return x.float().reshape(rows, -1).sum(1)


def add_bf16(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """LOP_residual/00_..._fused_add_dfgomnnn_triton.py: bf16(float(a) + float(b))."""
    return (a.float() + b.float()).to(BF16)


def rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, tokens: int) -> torch.Tensor:
    """LOP_rope_q/00_..._fused__to_copy_add_cat_mul_neg_slice_unsqueeze_4de5dxfe_triton.py:17-47:
    x [T, H, 128]: out = x*cos[t] + cat(-x[64:], x[:64])*sin[t], fp32, one bf16 store."""
    xr = x.float().reshape(tokens, -1, 128)
    c = cos.float().reshape(tokens, 1, 128)
    s = sin.float().reshape(tokens, 1, 128)
    rot = torch.cat([-xr[..., 64:], xr[..., :64]], dim=-1)
    return (xr * c + rot * s).to(BF16).reshape(-1)


def rmsnorm_add(x: torch.Tensor, a, w: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """LL/18_..._fused__to_copy_add_mean_mul_pow_rsqrt_p5e5f5kj_triton.py: v = x + a in fp32 (no
    rounding), y = bf16(v * rsqrt(sum(v^2)/C + eps) * w) per row of C = w.numel()."""
    c = w.numel()
    v = x.float().reshape(-1, c)
    if a is not None:
        v = v + a.float().reshape(-1, c)
    r = torch.rsqrt((v * v).sum(1, keepdim=True) / float(c) + eps)
    return ((v * r) * w.float()).to(BF16).reshape(-1)


def rms_broadcast(x, a, ss, w, rows: int, eps: float = 1e-6) -> torch.Tensor:
    """layer_layer_decode_1x1024_bf16/19_..._wkrpkilh_triton.py:17-60 (one token): out[s, c] =
    bf16(((x + a) * rsqrt(ss / C + eps)) * w) for each of the token's rows s."""
    c = x.numel()
    r = torch.rsqrt(ss.float().reshape(()) / float(c) + eps)
    v = ((x.float() + a.float()) * r) * w.float()
    return v.to(BF16).repeat(rows)


def grouped_mm(a, b, group, start, rows, k: int, n: int, weight_stride: int, c=None) -> torch.Tensor:
    """LOP_gmm_gate_up/05__grouped_mm_kernel/_grouped_mm_kernel_triton.py:4-46: for each program p,
    g = group[p]: C[start[g] + i] = bf16(A[start[g] + i] @ B[g]) for i < rows[g] (the dot in fp32;
    here in fp64, rounded once to fp32).  Rows no program covers keep c's values."""
    ar = a.reshape(-1, k)
    out = (c.clone() if c is not None else torch.zeros(ar.shape[0] * n, dtype=BF16)).reshape(-1, n)
    nw = b.numel() // weight_stride
    for p in range(group.numel()):
        g = int(group[p])
        if g < 0 or g >= start.numel():
            continue
        s0, nr = int(start[g]), int(rows[g])
        if nr <= 0 or s0 < 0 or s0 + nr > ar.shape[0] or g >= nw:
            continue
        bg = b[g * weight_stride: g * weight_stride + k * n].reshape(k, n)
        out[s0:s0 + nr] = (ar[s0:s0 + nr].double() @ bg.double()).to(F32).to(BF16)
    return out.reshape(-1)
