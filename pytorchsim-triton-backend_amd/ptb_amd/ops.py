"""Tensor-level entry points over the C ABI.

PyTorch is used only as the owner of device memory and of the current HIP stream: each function
checks device, dtype, shape and contiguity, allocates its outputs (unless ``out=`` is given) and
calls the HIP kernel through :mod:`ptb_amd._lib` with raw pointers.  No function has a CPU or
PyTorch-compute fallback.
"""
from __future__ import annotations

import math

import torch

from . import _lib

BF16 = torch.bfloat16
F32 = torch.float32
E4M3 = torch.float8_e4m3fn


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _need(t: torch.Tensor, name: str, dtypes, ndim: int | None = None) -> None:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor")
    if t.device.type != "cuda":
        raise ValueError(f"{name} must live on the GPU (got {t.device})")
    if t.dtype not in (dtypes if isinstance(dtypes, tuple) else (dtypes,)):
        raise TypeError(f"{name} has dtype {t.dtype}, expected {dtypes}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    if ndim is not None and t.dim() != ndim:
        raise ValueError(f"{name} must be {ndim}-D, got shape {tuple(t.shape)}")


def _out(out, shape, dtype, like: torch.Tensor, name="out") -> torch.Tensor:
    if out is None:
        return torch.empty(shape, dtype=dtype, device=like.device)
    _need(out, name, dtype)
    if tuple(out.shape) != tuple(shape):
        raise ValueError(f"{name} has shape {tuple(out.shape)}, expected {tuple(shape)}")
    return out


def rmsnorm(x: torch.Tensor, w: torch.Tensor, eps: float = 1e-6, out=None) -> torch.Tensor:
    """y = bf16(x * rsqrt(mean(x^2) + eps) * w) over the last dim of a 2-D bf16 x; for an fp32 x (and
    fp32 w) the same in fp32 throughout, y fp32."""
    if isinstance(x, torch.Tensor) and x.dtype == F32:
        _need(x, "x", F32, 2)
        _need(w, "w", F32, 1)
        rows, cols = x.shape
        if w.numel() != cols:
            raise ValueError(f"w has {w.numel()} elements, x rows have {cols}")
        y = _out(out, (rows, cols), F32, x)
        _lib.call("ptb_rmsnorm_f32", x.data_ptr(), w.data_ptr(), y.data_ptr(), rows, cols, float(eps), _stream(x))
        return y
    _need(x, "x", BF16, 2)
    _need(w, "w", (BF16, F32), 1)
    rows, cols = x.shape
    if w.numel() != cols:
        raise ValueError(f"w has {w.numel()} elements, x rows have {cols}")
    y = _out(out, (rows, cols), BF16, x)
    wd = _lib.PTB_DTYPE_F32 if w.dtype == F32 else _lib.PTB_DTYPE_BF16
    _lib.call("ptb_rmsnorm_bf16", x.data_ptr(), w.data_ptr(), wd, y.data_ptr(), rows, cols, float(eps), _stream(x))
    return y


def col_rms(x: torch.Tensor, eps: float = 1e-5, out=None) -> torch.Tensor:
    """c[j] = rsqrt(mean_i x[i, j]^2 + eps) over the rows of a 2-D fp32 x (the column arm of the
    reference's fp32 RMSNorm case)."""
    _need(x, "x", F32, 2)
    rows, cols = x.shape
    c = _out(out, (cols,), F32, x)
    _lib.call("ptb_col_rms_f32", x.data_ptr(), c.data_ptr(), rows, cols, float(eps), _stream(x))
    return c


def softmax_rows(x: torch.Tensor, out=None, out_dtype=BF16) -> torch.Tensor:
    """Row softmax of bf16 rows; the result in bf16 (one rounding) or, with out_dtype fp32, unrounded.
    fp32 rows give fp32 probabilities."""
    if isinstance(x, torch.Tensor) and x.dtype == F32:
        _need(x, "x", F32, 2)
        y = _out(out, tuple(x.shape), F32, x)
        _lib.call("ptb_softmax_rows_f32", x.data_ptr(), y.data_ptr(), x.shape[0], x.shape[1], _stream(x))
        return y
    _need(x, "x", BF16, 2)
    if out_dtype not in (BF16, F32):
        raise TypeError(f"softmax_rows writes bf16 or fp32, not {out_dtype}")
    y = _out(out, tuple(x.shape), out_dtype, x)
    fn = "ptb_softmax_rows_bf16_f32" if out_dtype == F32 else "ptb_softmax_rows_bf16"
    _lib.call(fn, x.data_ptr(), y.data_ptr(), x.shape[0], x.shape[1], _stream(x))
    return y


def silu_mul(gate_up: torch.Tensor, out=None) -> torch.Tensor:
    """[T, 2I] (gate | up) -> [T, I]: silu(gate) * up, in bf16 (one rounding) or, for fp32 input, fp32."""
    dt = F32 if isinstance(gate_up, torch.Tensor) and gate_up.dtype == F32 else BF16
    _need(gate_up, "gate_up", dt, 2)
    rows, two_i = gate_up.shape
    if two_i % 2:
        raise ValueError("gate_up's last dim must be even (gate | up)")
    y = _out(out, (rows, two_i // 2), dt, gate_up)
    fn = "ptb_silu_mul_f32" if dt == F32 else "ptb_silu_mul_bf16"
    _lib.call(fn, gate_up.data_ptr(), y.data_ptr(), rows, two_i // 2, _stream(gate_up))
    return y


def swiglu_f32(x: torch.Tensor, wg: torch.Tensor, wu: torch.Tensor, out=None) -> torch.Tensor:
    """o = silu(x @ wg) * (x @ wu) for fp32 x [M, K], wg / wu [K, N], fp32 accumulation."""
    _need(x, "x", F32, 2)
    _need(wg, "wg", F32, 2)
    _need(wu, "wu", F32, 2)
    m, k = x.shape
    if wg.shape[0] != k or tuple(wu.shape) != tuple(wg.shape):
        raise ValueError("wg and wu must both be [K, N] for x [M, K]")
    n = wg.shape[1]
    o = _out(out, (m, n), F32, x)
    _lib.call("ptb_swiglu_f32", x.data_ptr(), wg.data_ptr(), wu.data_ptr(), o.data_ptr(), m, n, k, _stream(x))
    return o


def _row_ld(x: torch.Tensor, name: str):
    """A bf16 [A, B, D] tensor whose [B, D] rows are each contiguous (a column slice of a wider
    [A, L] matrix is one): None when x is contiguous, else the elements between consecutive rows."""
    if not isinstance(x, torch.Tensor) or x.is_contiguous():
        _need(x, name, BF16, 3)
        return None
    if x.device.type != "cuda" or x.dtype != BF16 or x.dim() != 3:
        raise ValueError(f"{name} must be a 3-D bf16 GPU tensor")
    a, b, d = x.shape
    if x.stride(2) != 1 or x.stride(1) != d or x.stride(0) < b * d:
        raise ValueError(f"{name} must have contiguous [B, D] rows (strides (ld, D, 1)), got {x.stride()}")
    return x.stride(0)


def transpose_heads(x: torch.Tensor, out=None) -> torch.Tensor:
    """[A, B, D] -> [B, A, D] (exact).  x may be a column slice of a wider matrix (rows ld apart)."""
    ld = _row_ld(x, "x")
    a, b, d = x.shape
    y = _out(out, (b, a, d), BF16, x)
    if ld is None:
        _lib.call("ptb_transpose_heads_bf16", x.data_ptr(), y.data_ptr(), a, b, d, _stream(x))
    else:
        _lib.call("ptb_transpose_heads_ld_bf16", x.data_ptr(), ld, y.data_ptr(), a, b, d, _stream(x))
    return y


def qk_norm_rope(x: torch.Tensor, w: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, eps: float = 1e-6,
                 out=None) -> torch.Tensor:
    """x [T, H, D] -> per-head RMSNorm(w) + rotate-half RoPE -> [H, T, D].  x may be a column slice
    of a wider matrix (token rows ld apart), as the q or k part of a fused q|k|v projection."""
    ld = _row_ld(x, "x")
    _need(w, "w", BF16, 1)
    _need(cos, "cos", F32, 2)
    _need(sin, "sin", F32, 2)
    t, h, d = x.shape
    if w.numel() != d or tuple(cos.shape) != (t, d) or tuple(sin.shape) != (t, d):
        raise ValueError("w must be [D] and cos/sin [T, D]")
    y = _out(out, (h, t, d), BF16, x)
    if ld is None:
        _lib.call("ptb_qk_norm_rope_bf16", x.data_ptr(), w.data_ptr(), cos.data_ptr(), sin.data_ptr(),
                  y.data_ptr(), t, h, d, float(eps), _stream(x))
    else:
        _lib.call("ptb_qk_norm_rope_ld_bf16", x.data_ptr(), ld, w.data_ptr(), cos.data_ptr(), sin.data_ptr(),
                  y.data_ptr(), t, h, d, float(eps), _stream(x))
    return y


def reduce(x: torch.Tensor, op: str = "sum", out=None, workspace=None) -> torch.Tensor:
    """Whole-tensor sum or max of a bf16 or fp32 tensor, as one fp32 value (shape [1])."""
    _need(x, "x", (BF16, F32))
    code = {"sum": _lib.PTB_REDUCE_SUM, "max": _lib.PTB_REDUCE_MAX}[op]
    y = _out(out, (1,), F32, x)
    need = _lib.load().ptb_reduce_workspace_bytes(x.numel())
    if workspace is None:
        workspace = torch.empty(need, dtype=torch.uint8, device=x.device)
    fn = "ptb_reduce_f32" if x.dtype == F32 else "ptb_reduce_bf16"
    _lib.call(fn, x.data_ptr(), y.data_ptr(), x.numel(), code, workspace.data_ptr(),
              workspace.numel() * workspace.element_size(), _stream(x))
    return y


def add_scalar(x: torch.Tensor, s: float, out=None) -> torch.Tensor:
    _need(x, "x", BF16)
    y = _out(out, tuple(x.shape), BF16, x)
    _lib.call("ptb_add_scalar_bf16", x.data_ptr(), y.data_ptr(), x.numel(), float(s), _stream(x))
    return y


def slice_add(x: torch.Tensor, first: int, count: int, s: float, out=None) -> torch.Tensor:
    """out[i] = float(x.flat[first + i]) + s (fp32), i < count."""
    _need(x, "x", BF16)
    if first < 0 or count < 0 or first + count > x.numel():
        raise ValueError(f"slice [{first}, {first + count}) is outside the {x.numel()} elements")
    y = _out(out, (count,), F32, x)
    _lib.call("ptb_slice_add_bf16", x.data_ptr(), y.data_ptr(), first, count, float(s), _stream(x))
    return y


def gemm(a: torch.Tensor, b: torch.Tensor, residual: torch.Tensor | None = None, out=None,
         workspace: torch.Tensor | None = None, split_k: bool = True) -> torch.Tensor:
    """C = A[M,K] @ B[K,N] (+ residual[M,N]), bf16 operands, fp32 accumulation, bf16 C.  Shapes whose
    output tiles would leave most CUs idle run split-K over a workspace (given, or allocated here);
    split_k=False forces the single-pass kernel."""
    _need(a, "a", BF16, 2)
    _need(b, "b", BF16, 2)
    m, k = a.shape
    k2, n = b.shape
    if k != k2:
        raise ValueError(f"inner dims differ: a is {tuple(a.shape)}, b is {tuple(b.shape)}")
    rp = 0
    if residual is not None:
        _need(residual, "residual", BF16, 2)
        if tuple(residual.shape) != (m, n):
            raise ValueError("residual must be [M, N]")
        rp = residual.data_ptr()
    c = _out(out, (m, n), BF16, a)
    need = _lib.load().ptb_gemm_bf16_workspace_bytes(m, n, k) if split_k else 0
    if need:
        if workspace is None:
            workspace = torch.empty(need, dtype=torch.uint8, device=a.device)
        _lib.call("ptb_gemm_bf16_ws", a.data_ptr(), b.data_ptr(), rp, c.data_ptr(), m, n, k, workspace.data_ptr(),
                  workspace.numel() * workspace.element_size(), _stream(a))
    else:
        _lib.call("ptb_gemm_bf16", a.data_ptr(), b.data_ptr(), rp, c.data_ptr(), m, n, k, _stream(a))
    return c


def gemm_swiglu(a: torch.Tensor, b: torch.Tensor, out=None) -> torch.Tensor:
    """C[M, I] = silu(bf16(A @ B[:, :I])) * bf16(A @ B[:, I:]) for B [K, 2I]: the gate_up GEMM and the
    SwiGLU gate in one kernel, equal bit for bit to ``silu_mul(gemm(a, b))``."""
    _need(a, "a", BF16, 2)
    _need(b, "b", BF16, 2)
    m, k = a.shape
    k2, n = b.shape
    if k != k2 or n % 2:
        raise ValueError(f"a is {tuple(a.shape)}, b is {tuple(b.shape)}: need B [K, 2I]")
    c = _out(out, (m, n // 2), BF16, a)
    _lib.call("ptb_gemm_swiglu_bf16", a.data_ptr(), b.data_ptr(), c.data_ptr(), m, n // 2, k, _stream(a))
    return c


def quant_rows_e4m3(x: torch.Tensor):
    """Per-row dynamic e4m3 quantisation: (xq [R,C] float8_e4m3fn, scale [R] fp32)."""
    _need(x, "x", BF16, 2)
    rows, cols = x.shape
    xq = torch.empty((rows, cols), dtype=E4M3, device=x.device)
    sc = torch.empty((rows,), dtype=F32, device=x.device)
    _lib.call("ptb_quant_rows_e4m3", x.data_ptr(), xq.data_ptr(), sc.data_ptr(), rows, cols, _stream(x))
    return xq, sc


def quant_weight_e4m3(w: torch.Tensor):
    """Per-output-channel e4m3 quantisation of fp32 W[K,N]: (wq_t [N,K] float8_e4m3fn, scale [N] fp32)."""
    _need(w, "w", F32, 2)
    k, n = w.shape
    wq = torch.empty((n, k), dtype=E4M3, device=w.device)
    sc = torch.empty((n,), dtype=F32, device=w.device)
    _lib.call("ptb_quant_weight_e4m3", w.data_ptr(), wq.data_ptr(), sc.data_ptr(), k, n, _stream(w))
    return wq, sc


def gemm_fp8(aq: torch.Tensor, sa: torch.Tensor, wq_t: torch.Tensor, sw: torch.Tensor, out=None) -> torch.Tensor:
    """C = bf16((Aq[M,K] @ Wt[N,K]^T) * sa[M] * sw[N]) with e4m3 operands and fp32 accumulation."""
    _need(aq, "aq", E4M3, 2)
    _need(wq_t, "wq_t", E4M3, 2)
    _need(sa, "sa", F32, 1)
    _need(sw, "sw", F32, 1)
    m, k = aq.shape
    n, k2 = wq_t.shape
    if k != k2 or sa.numel() != m or sw.numel() != n:
        raise ValueError("shapes: aq [M,K], sa [M], wq_t [N,K], sw [N]")
    c = _out(out, (m, n), BF16, aq)
    _lib.call("ptb_gemm_fp8_scaled", aq.data_ptr(), sa.data_ptr(), wq_t.data_ptr(), sw.data_ptr(), c.data_ptr(),
              m, n, k, _stream(aq))
    return c


def fp8_linear(x: torch.Tensor, wq_t: torch.Tensor, sw: torch.Tensor, out=None) -> torch.Tensor:
    """Per-token dynamic quantisation of x, then the fp8 GEMM (BASELINE config 4's path)."""
    xq, sx = quant_rows_e4m3(x)
    return gemm_fp8(xq, sx, wq_t, sw, out=out)


def default_scale(head_dim: int) -> float:
    return 1.0 / math.sqrt(head_dim)


def flash_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, hq: int, hkv: int, causal: bool = True,
                    scale: float | None = None, out=None, tokens_out: bool = False) -> torch.Tensor:
    """Flash-attention forward over head-major q [B*hq, S, D], k/v [B*hkv, S, D] -> o like q, or with
    `tokens_out` o [B, S, hq, D] (token-major, no separate head transpose)."""
    for t, name in ((q, "q"), (k, "k"), (v, "v")):
        _need(t, name, BF16, 3)
    bhq, s, d = q.shape
    if hq <= 0 or hkv <= 0 or hq % hkv or bhq % hq:
        raise ValueError(f"bad head counts hq={hq}, hkv={hkv} for q of shape {tuple(q.shape)}")
    batch = bhq // hq
    if tuple(k.shape) != (batch * hkv, s, d) or tuple(v.shape) != (batch * hkv, s, d):
        raise ValueError("k and v must be [B*hkv, S, D] matching q")
    o = _out(out, (batch, s, hq, d) if tokens_out else tuple(q.shape), BF16, q)
    sc = default_scale(d) if scale is None else float(scale)
    _lib.call("ptb_flash_attn_fwd_tokens_bf16" if tokens_out else "ptb_flash_attn_fwd_bf16", q.data_ptr(),
              k.data_ptr(), v.data_ptr(), o.data_ptr(), batch, hq, hkv, s, d, sc, 1 if causal else 0, _stream(q))
    return o


def flash_attention_qkv(qkv: torch.Tensor, k: torch.Tensor, qnorm_w: torch.Tensor, cos: torch.Tensor,
                        sin: torch.Tensor, hq: int, hkv: int, eps: float, causal: bool = True,
                        scale: float | None = None, out=None) -> torch.Tensor:
    """Attention over a fused projection output: qkv [B*S, ld] bf16 holds q | k | v per token
    (row stride ld >= (hq + 2*hkv)*128), k the normalised, rotated keys [B*hkv, S, 128]; the queries
    are normalised (qnorm_w, eps) and rotated (cos/sin [S, 128] fp32) in the kernel and v read in
    place.  Returns o [B, S, hq, 128] token-major, bit for bit qk_norm_rope(q) + transpose_heads(v) +
    flash_attention(tokens_out=True)."""
    _need(k, "k", BF16, 3)
    _need(qnorm_w, "qnorm_w", BF16, 1)
    _need(cos, "cos", F32, 2)
    _need(sin, "sin", F32, 2)
    if qkv.dtype != BF16 or qkv.dim() != 2 or qkv.stride(1) != 1:
        raise ValueError("qkv must be a row-major [B*S, ld] bf16 matrix (rows may be a strided view)")
    bhkv, s, d = k.shape
    if hq <= 0 or hkv <= 0 or hq % hkv or bhkv % hkv:
        raise ValueError(f"bad head counts hq={hq}, hkv={hkv} for k of shape {tuple(k.shape)}")
    batch = bhkv // hkv
    ld = qkv.stride(0)
    if qkv.shape[0] != batch * s or qkv.shape[1] < (hq + 2 * hkv) * d:
        raise ValueError(f"qkv must be [B*S, >= (hq + 2*hkv)*{d}], got {tuple(qkv.shape)}")
    if tuple(cos.shape) != (s, d) or tuple(sin.shape) != (s, d) or qnorm_w.numel() != d:
        raise ValueError("cos/sin must be [S, head_dim] and qnorm_w [head_dim]")
    o = _out(out, (batch, s, hq, d), BF16, qkv)
    sc = default_scale(d) if scale is None else float(scale)
    _lib.call("ptb_flash_attn_fwd_qkv_bf16", qkv.data_ptr(), ld, k.data_ptr(), qnorm_w.data_ptr(), cos.data_ptr(),
              sin.data_ptr(), float(eps), o.data_ptr(), batch, hq, hkv, s, d, sc, 1 if causal else 0, _stream(qkv))
    return o


# ---- single-token (decode) path -------------------------------------------------------------------

def sumsq(x: torch.Tensor, y: torch.Tensor | None = None, out=None) -> torch.Tensor:
    """sum((x + y)^2) (or sum(x^2)) over all elements of bf16 vectors, as one fp32 value (shape [1])."""
    _need(x, "x", BF16)
    if y is not None:
        _need(y, "y", BF16)
        if y.numel() != x.numel():
            raise ValueError("x and y must have the same number of elements")
    r = _out(out, (1,), F32, x)
    _lib.call("ptb_sumsq_bf16", x.data_ptr(), y.data_ptr() if y is not None else None, r.data_ptr(), x.numel(),
              _stream(x))
    return r


def _gemv_args(xk: int, w: torch.Tensor, out, like: torch.Tensor, workspace):
    _need(w, "w", BF16, 2)
    k, n = w.shape
    if xk != k:
        raise ValueError(f"the vector has {xk} elements, W has {k} rows")
    y = _out(out, (n,), BF16, like)
    need = _lib.load().ptb_gemv_workspace_bytes(k, n)
    if workspace is None:
        workspace = torch.empty(max(need, 4), dtype=torch.uint8, device=like.device)
    return k, n, y, workspace, workspace.numel() * workspace.element_size()


def gemv(x: torch.Tensor, w: torch.Tensor, out=None, workspace=None) -> torch.Tensor:
    """y[n] = bf16(sum_k x[k] W[k,n]), W [K,N] bf16, fp32 accumulation."""
    _need(x, "x", BF16)
    k, n, y, ws, wsb = _gemv_args(x.numel(), w, out, x, workspace)
    _lib.call("ptb_gemv_bf16", x.data_ptr(), w.data_ptr(), y.data_ptr(), k, n, ws.data_ptr(), wsb, _stream(x))
    return y


def gemv_rmsnorm(x: torch.Tensor, ss: torch.Tensor, g: torch.Tensor, w: torch.Tensor, add: torch.Tensor | None = None,
                 eps: float = 1e-6, out=None, workspace=None) -> torch.Tensor:
    """y = bf16( (((x + add) * rsqrt(ss/K + eps)) * g) @ W ), the normalised vector kept in fp32.
    ss=None: the kernel forms sum((x + add)^2) itself (no separate sumsq launch)."""
    _need(x, "x", BF16)
    if ss is not None:
        _need(ss, "ss", F32)
    _need(g, "g", BF16)
    if add is not None:
        _need(add, "add", BF16)
        if add.numel() != x.numel():
            raise ValueError("add must match x")
    if g.numel() != x.numel():
        raise ValueError("g must match x")
    k, n, y, ws, wsb = _gemv_args(x.numel(), w, out, x, workspace)
    _lib.call("ptb_gemv_rmsnorm_bf16", x.data_ptr(), add.data_ptr() if add is not None else None,
              ss.data_ptr() if ss is not None else None,
              g.data_ptr(), float(eps), w.data_ptr(), y.data_ptr(), k, n, ws.data_ptr(), wsb, _stream(x))
    return y


def gemv_rmsnorm_parts(x: torch.Tensor, ss: torch.Tensor | None, g: torch.Tensor, w: torch.Tensor,
                       add: torch.Tensor | None = None, eps: float = 1e-6, parts=None) -> torch.Tensor:
    """gemv_rmsnorm's partial pass alone: returns its fp32 partials (a uint8 tensor of
    ptb_gemv_workspace_bytes(K, N) bytes, `parts` if given), to be finished by :func:`gemv_silu_parts`."""
    _need(x, "x", BF16)
    if ss is not None:
        _need(ss, "ss", F32)
    _need(g, "g", BF16)
    _need(w, "w", BF16, 2)
    if add is not None:
        _need(add, "add", BF16)
        if add.numel() != x.numel():
            raise ValueError("add must match x")
    k, n = w.shape
    if x.numel() != k or g.numel() != k:
        raise ValueError(f"x and g must hold {k} values")
    need = _lib.load().ptb_gemv_workspace_bytes(k, n)
    if parts is None:
        parts = torch.empty(max(need, 4), dtype=torch.uint8, device=x.device)
    _lib.call("ptb_gemv_rmsnorm_parts_bf16", x.data_ptr(), add.data_ptr() if add is not None else None,
              ss.data_ptr() if ss is not None else None, g.data_ptr(), float(eps), w.data_ptr(), parts.data_ptr(),
              k, n, parts.numel() * parts.element_size(), _stream(x))
    return parts


def gemv_silu_parts(gate_up_parts: torch.Tensor, gate_up_k: int, w: torch.Tensor, res_a: torch.Tensor | None = None,
                    res_b: torch.Tensor | None = None, out=None, workspace=None) -> torch.Tensor:
    """:func:`gemv_silu` over the gate|up vector that :func:`gemv_rmsnorm_parts` left as partials (its
    W was [gate_up_k, 2K]); bit for bit gemv_rmsnorm followed by gemv_silu, one launch fewer."""
    if not isinstance(gate_up_parts, torch.Tensor) or gate_up_parts.device.type != "cuda":
        raise ValueError("gate_up_parts must be a GPU tensor")
    for t, name in ((res_a, "res_a"), (res_b, "res_b")):
        if t is not None:
            _need(t, name, BF16)
    if res_b is not None and res_a is None:
        raise ValueError("res_b needs res_a")
    _need(w, "w", BF16, 2)
    k, n, y, ws, wsb = _gemv_args(w.shape[0], w, out, gate_up_parts, workspace)
    if gate_up_parts.numel() * gate_up_parts.element_size() < _lib.load().ptb_gemv_workspace_bytes(gate_up_k, 2 * k):
        raise ValueError("gate_up_parts is smaller than the producing GEMV's partials")
    for t, name in ((res_a, "res_a"), (res_b, "res_b")):
        if t is not None and t.numel() != n:
            raise ValueError(f"{name} must have {n} elements")
    _lib.call("ptb_gemv_silu_parts_bf16", gate_up_parts.data_ptr(), int(gate_up_k), w.data_ptr(),
              res_a.data_ptr() if res_a is not None else None, res_b.data_ptr() if res_b is not None else None,
              y.data_ptr(), k, n, ws.data_ptr(), wsb, _stream(gate_up_parts))
    return y


def gemv_silu(gate_up: torch.Tensor, w: torch.Tensor, res_a: torch.Tensor | None = None,
              res_b: torch.Tensor | None = None, out=None, workspace=None) -> torch.Tensor:
    """y = bf16( (silu(g) * u) @ W + (res_a + res_b) ), gate_up = g | u (2K values)."""
    _need(gate_up, "gate_up", BF16)
    if gate_up.numel() % 2:
        raise ValueError("gate_up must hold gate and up halves")
    for t, name in ((res_a, "res_a"), (res_b, "res_b")):
        if t is not None:
            _need(t, name, BF16)
    if res_b is not None and res_a is None:
        raise ValueError("res_b needs res_a")
    k, n, y, ws, wsb = _gemv_args(gate_up.numel() // 2, w, out, gate_up, workspace)
    for t, name in ((res_a, "res_a"), (res_b, "res_b")):
        if t is not None and t.numel() != n:
            raise ValueError(f"{name} must have {n} elements")
    _lib.call("ptb_gemv_silu_bf16", gate_up.data_ptr(), w.data_ptr(),
              res_a.data_ptr() if res_a is not None else None, res_b.data_ptr() if res_b is not None else None,
              y.data_ptr(), k, n, ws.data_ptr(), wsb, _stream(gate_up))
    return y


def attention_decode(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float | None = None, out=None,
                     workspace=None, qnorm=None) -> torch.Tensor:
    """One-token attention over a KV cache: q [NKV, G, D], k/v [NKV, S, D] bf16 -> o [NKV, G, D].
    `workspace`: ``ptb_attn_decode_workspace_bytes`` bytes (none for a cache of at most 256 keys,
    which is a single pass).  `qnorm` = (w [D] bf16, cos [D] fp32, sin [D] fp32, eps): q is then the
    raw projection, normalized and rotated in the kernel's prologue exactly as :func:`qk_norm_rope`
    would (one launch instead of two)."""
    _need(q, "q", BF16, 3)
    _need(k, "k", BF16, 3)
    _need(v, "v", BF16, 3)
    nkv, g, d = q.shape
    if k.shape[0] != nkv or k.shape[2] != d or tuple(v.shape) != tuple(k.shape):
        raise ValueError("k and v must be [NKV, S, D] matching q")
    s = k.shape[1]
    o = _out(out, (nkv, g, d), BF16, q)
    need = _lib.load().ptb_attn_decode_workspace_bytes(nkv, g, s)
    if workspace is None and need:
        workspace = torch.empty(need, dtype=torch.uint8, device=q.device)
    sc = default_scale(d) if scale is None else float(scale)
    wsp = workspace.data_ptr() if workspace is not None else None
    wsb = workspace.numel() * workspace.element_size() if workspace is not None else 0
    if qnorm is None:
        _lib.call("ptb_attn_decode_bf16", q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), nkv, g, s, d, sc,
                  wsp, wsb, _stream(q))
        return o
    w, cos, sin, eps = qnorm
    _need(w, "qnorm w", BF16, 1)
    _need(cos, "cos", F32)
    _need(sin, "sin", F32)
    if w.numel() != d or cos.numel() != d or sin.numel() != d:
        raise ValueError("qnorm w, cos and sin must hold D elements")
    _lib.call("ptb_attn_decode_qnorm_rope_bf16", q.data_ptr(), w.data_ptr(), cos.data_ptr(), sin.data_ptr(),
              float(eps), k.data_ptr(), v.data_ptr(), o.data_ptr(), nkv, g, s, d, sc, wsp, wsb, _stream(q))
    return o
