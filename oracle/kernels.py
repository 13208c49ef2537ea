"""torch-CPU restatement of the reference kernels on the hot path (test infrastructure only).

All inputs/outputs are CPU tensors.  bf16 values are rounded exactly where the reference kernel
stores to a bf16 pointer (Triton's store casts fp32 -> bf16 with round-to-nearest-even); every
intermediate is fp32 as the reference computes it, unless a docstring says otherwise.
Reference paths are relative to the reference repository root; ``L2048`` stands for
``validation/pytorchsim/qwen3_8b_layer_prefill_2048x2048_bf16`` and ``D4096`` for
``validation/pytorchsim/qwen3_8b_layer_decode_1x4096_bf16`` (the other decode lengths differ only
in S).
"""
from __future__ import annotations

import math

import torch

BF16 = torch.bfloat16
F32 = torch.float32
E4M3 = torch.float8_e4m3fn

__all__ = [
    "rmsnorm", "softmax_rows", "silu_mul", "transpose_heads", "qk_norm_rope", "reduce_sum", "reduce_max",
    "add_scalar", "gemm", "quant_rows_e4m3", "quant_weight_e4m3", "gemm_fp8", "flash_attention",
    "rope_tables", "qwen3_layer", "E4M3_MAX",
    "slice_add", "sumsq", "gemv", "gemv_rmsnorm", "gemv_silu", "attention_decode", "qwen3_decode_layer",
    "rmsnorm_f32", "col_rms_f32", "silu_mul_f32", "swiglu_f32",
]

E4M3_MAX = 448.0


def rmsnorm(x: torch.Tensor, w: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """L2048/00_..._gwdq6qer_triton.py:17-60: per row, s = sum(x^2) in fp32 (:24-42), then
    y = (x * rsqrt(s / cols + eps)) * w (:44-59), stored to bf16 once (:60).  w may be bf16
    (the bundle kernel) or fp32."""
    xf = x.float()
    s = (xf * xf).sum(dim=-1, keepdim=True)
    r = torch.rsqrt(s / float(x.shape[-1]) + eps)
    return ((xf * r) * w.float()).to(BF16)


def rmsnorm_f32(x: torch.Tensor, w: torch.Tensor, eps: float = 1e-5) -> torch.Tensor:
    """tests/cases/workloads/rmsnorm.py:44-54, the row arm of the fp32 case: ms = sum(x*x) / N (:51),
    y = x * rsqrt(ms + EPS) (:52), o = y * w (:54); everything fp32, nothing rounded below it."""
    xf = x.float()
    ms = (xf * xf).sum(dim=-1, keepdim=True) / float(x.shape[-1])
    return (xf * torch.rsqrt(ms + eps)) * w.float()


def col_rms_f32(x: torch.Tensor, eps: float = 1e-5) -> torch.Tensor:
    """tests/cases/workloads/rmsnorm.py:56-57, the column arm: rsqrt(sum_i x[i,j]^2 / rows + EPS)."""
    xf = x.float()
    return torch.rsqrt((xf * xf).sum(dim=0) / float(x.shape[0]) + eps)


def silu_mul_f32(gu: torch.Tensor) -> torch.Tensor:
    """The elementwise half of tests/cases/workloads/swiglu.py (:61-62): gate / (1 + exp(-gate)) * up
    in fp32, gate | up side by side as in the bf16 kernel's [T, 2I] layout."""
    inter = gu.shape[-1] // 2
    g = gu[..., :inter].float()
    u = gu[..., inter:].float()
    return (g / (1.0 + torch.exp(-g))) * u


def swiglu_f32(x: torch.Tensor, wg: torch.Tensor, wu: torch.Tensor) -> torch.Tensor:
    """tests/cases/workloads/swiglu.py:44-62: gate = x @ wg and up = x @ wu with fp32 accumulation
    (:52-58; the products are summed in fp64 and rounded once to fp32, the exact value every fp32
    order approximates), then gate / (1 + exp(-gate)) * up in fp32 (:61-62)."""
    g = (x.double() @ wg.double()).float()
    u = (x.double() @ wu.double()).float()
    return (g / (1.0 + torch.exp(-g))) * u


def softmax_rows(x: torch.Tensor, out_dtype=BF16) -> torch.Tensor:
    """vector_softmax_2048x6144_bf16/00_..._sa7wwqqf_triton.py:17-68: NaN-propagating row max
    (tl.maximum(..., PropagateNan.ALL), :30-33), sum of exp(x - max) (:35-47), exp(x - max) / sum
    stored as bf16 (:49-68).  out_dtype fp32: the MoE router's softmax, stored unrounded
    (layer_layer_decode_1x1024_bf16/16_..._qslpdpud_triton.py:31-45; its max2 does not propagate NaN,
    which only differs for rows holding a NaN)."""
    xf = x.float()
    m = torch.amax(xf, dim=-1, keepdim=True)  # amax propagates NaN
    e = torch.exp(xf - m)
    return (e / e.sum(dim=-1, keepdim=True)).to(out_dtype)


def silu_mul(gu: torch.Tensor) -> torch.Tensor:
    """L2048/10_..._ktzl5s2h_triton.py:17-36: g = gu[:, :I], u = gu[:, I:] (:26-27),
    (g / (exp(-g) + 1)) * u in fp32 (:28-35), one bf16 store (:36)."""
    inter = gu.shape[-1] // 2
    g = gu[..., :inter].float()
    u = gu[..., inter:].float()
    return ((g / (torch.exp(-g) + 1.0)) * u).to(BF16)


def transpose_heads(x: torch.Tensor) -> torch.Tensor:
    """L2048/05_..._ff5nvvqz_triton.py:17-27 ([T,H,D] -> [H,T,D]) and L2048/07_..._ei42assc_triton.py
    :17-27 ([H,T,D] -> [T,H,D]): pure permutation of the first two dims."""
    return x.permute(1, 0, 2).contiguous()


def qk_norm_rope(x: torch.Tensor, w: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
                 eps: float = 1e-6) -> torch.Tensor:
    """L2048/02_..._mmis7ufj_triton.py:17-98 (and 04_..._ll67ghqi for 8 heads).  x [T,H,D]:
    s = sum(x^2) over D (:37-41), r = rsqrt(s/D + eps) (:50-53), a = (x*r)*w (:54-57); rotate-half:
    element d < D/2 takes -((x[d+D/2]*r)*w[d+D/2]) (:49-71), element d >= D/2 takes
    (x[d-D/2]*r)*w[d-D/2] (:72-87); out = a*cos[t,d] + rot*sin[t,d] (:88-96), no intermediate bf16
    rounding, stored head-major [H,T,D] as bf16 (:98)."""
    t, h, d = x.shape
    half = d // 2
    xf = x.float()
    s = (xf * xf).sum(dim=-1, keepdim=True)
    r = torch.rsqrt(s / float(d) + eps)
    a = (xf * r) * w.float()
    rot = torch.cat([-a[..., half:], a[..., :half]], dim=-1)
    out = a * cos.float()[:, None, :] + rot * sin.float()[:, None, :]
    return out.to(BF16).permute(1, 0, 2).contiguous()


def reduce_sum(x: torch.Tensor) -> torch.Tensor:
    """vector_sum_<R>x<C>_bf16/00_..._2y6fwkvp_triton.py: fp32 sum of all elements.  Restated as the
    correctly rounded sum (fp64 accumulation, one rounding to fp32); the kernel's fp32 partial sums
    differ from it by the accumulation error only."""
    return x.double().sum().to(F32).reshape(1)


def reduce_max(x: torch.Tensor) -> torch.Tensor:
    """vector_max_<R>x<C>_bf16/00_..._q47252w4_triton.py: NaN-propagating max as fp32."""
    return torch.amax(x.float().reshape(-1)).reshape(1)


def add_scalar(x: torch.Tensor, s: float = 1.0) -> torch.Tensor:
    """vector_add1_<R>x<C>_bf16/00_..._du5rd5jd_triton.py: bf16(float(x) + 1.0)."""
    return (x.float() + s).to(BF16)


def slice_add(x: torch.Tensor, first: int = 0, count: int = 1, s: float = 1.0) -> torch.Tensor:
    """vector_slice_<R>x<C>_bf16/00_..._slnyinbt_triton.py:17-27: fp32 out = float(x[0]) + 1.0 (:22-27),
    generalised to a run of `count` elements from `first`."""
    return x.reshape(-1)[first:first + count].float() + s


def gemm(a: torch.Tensor, b: torch.Tensor, residual: torch.Tensor | None = None) -> torch.Tensor:
    """L2048/01_..._fused_mm_ckb6aiys_triton.py:18-97 (tl.dot with fp32 accumulation, ALLOW_TF32
    False, :69-85; bf16 store :97) and the residual epilogues L2048/08_..._utuycvlm_triton.py:96-99 /
    11_..._fjjozd2g_triton.py:48-51 (acc + float(R), one bf16 store).  The sum is taken in fp64 and
    rounded once to fp32, i.e. the exact value every fp32 accumulation order approximates."""
    acc = (a.double() @ b.double()).to(F32)
    if residual is not None:
        acc = acc + residual.float()
    return acc.to(BF16)


def quant_rows_e4m3(x: torch.Tensor):
    """Per-token dynamic e4m3 quantisation: scale = absmax(row)/448 (1 for an
    all-zero row), q = e4m3fn(x / scale) with torch's round-to-nearest-even cast, which is the
    fp32 -> fp8 conversion tests/cases/mechanism/ops/ops_fp8_e4m3_dot.py:41-44 uses."""
    xf = x.float()
    amax = xf.abs().amax(dim=-1)
    sc = torch.where(amax > 0, amax / E4M3_MAX, torch.ones_like(amax))
    return (xf / sc[:, None]).to(E4M3), sc


def quant_weight_e4m3(w: torch.Tensor):
    """Per-output-channel quantisation of W[K,N]: scale[n] = absmax(W[:, n])/448, packed transposed
    wq_t[n, k] = e4m3fn(W[k, n] / scale[n])."""
    wf = w.float()
    amax = wf.abs().amax(dim=0)
    sc = torch.where(amax > 0, amax / E4M3_MAX, torch.ones_like(amax))
    return (wf / sc[None, :]).to(E4M3).t().contiguous(), sc


def gemm_fp8(aq: torch.Tensor, sa: torch.Tensor, wq_t: torch.Tensor, sw: torch.Tensor) -> torch.Tensor:
    """e4m3 dot with fp32 accumulation (ops_fp8_e4m3_dot.py:41-44) and the per-token x per-channel
    scale epilogue of tests/cases/workloads/int8_dequant_matmul.py:59-69: bf16((acc * sa) * sw).
    The dot is summed in fp64 (products of e4m3 values are exact) and rounded once to fp32."""
    acc = (aq.double() @ wq_t.double().t()).to(F32)
    return ((acc * sa.float()[:, None]) * sw.float()[None, :]).to(BF16)


def flash_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, hq: int, hkv: int, causal: bool = True,
                    scale: float | None = None, bq: int = 1024, bkv: int = 1024) -> torch.Tensor:
    """attention_prefill_32x8x4096_bf16/00__prefill_kernel/_prefill_kernel_triton.py:4-44.
    Layout [B*H, S, D].  Program pid = (b, h) reads kv head b*hkv + h // (hq/hkv) (:7-10).  Per Q
    block of bq rows: m = -1e30, l = 0, acc = 0 (:15-17); unmasked KV blocks below the block's
    start (:18-30), then the diagonal block with keys > query set to -1e30 (:31-42).  qk =
    (q @ k^T) * scale in fp32; p = exp(qk - m_new) in fp32; l sums the fp32 p; P is rounded to
    bf16 before P @ V (:29, :41); output acc / l stored as bf16 (:43-44)."""
    bh, s, d = q.shape
    if scale is None:
        scale = 1.0 / math.sqrt(d)
    g = hq // hkv
    bq = min(bq, s)
    bkv = min(bkv, s)
    if causal and bq != bkv:
        raise ValueError("the reference's causal schedule needs bq == bkv")
    if s % bq or s % bkv:
        raise ValueError("S must be a multiple of the block sizes")
    out = torch.empty_like(q)
    for pid in range(bh):
        b, h = divmod(pid, hq)
        kvh = b * hkv + h // g
        Q, K, V = q[pid].float(), k[kvh].float(), v[kvh]
        for qb in range(s // bq):
            rm = torch.arange(qb * bq, (qb + 1) * bq)
            qq = Q[rm]
            m_i = torch.full((bq,), -1.0e30)
            l_i = torch.zeros(bq)
            acc = torch.zeros(bq, d)
            blocks = [(st, False) for st in range(0, qb * bq if causal else s, bkv)]
            if causal:
                blocks.append((qb * bq, True))
            for st, diag in blocks:
                n = torch.arange(st, st + bkv)
                qk = (qq @ K[n].t()) * scale
                if diag:
                    qk = torch.where(rm[:, None] >= n[None, :], qk, torch.tensor(-1.0e30))
                m_new = torch.maximum(m_i, qk.amax(dim=1))
                alpha = torch.exp(m_i - m_new)
                p = torch.exp(qk - m_new[:, None])
                l_i = l_i * alpha + p.sum(dim=1)
                acc = acc * alpha[:, None] + p.to(BF16).float() @ V[n].float()
                m_i = m_new
            out[pid, rm] = (acc / l_i[:, None]).to(BF16)
    return out


def rope_tables(tokens: int, head_dim: int = 128, theta: float = 1.0e6):
    """cos/sin [T, D] fp32 for rotate-half RoPE: angle[t, i] = t / theta^(2i/D), duplicated over
    the two halves (the fp32 cos/sin inputs of L2048/02 and 04)."""
    inv = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.float64) / head_dim))
    ang = torch.arange(tokens, dtype=torch.float64)[:, None] * inv[None, :]
    emb = torch.cat([ang, ang], dim=-1)
    return emb.cos().to(F32), emb.sin().to(F32)


def qwen3_layer(x: torch.Tensor, wts: dict, cos: torch.Tensor, sin: torch.Tensor, hq: int = 32, hkv: int = 8,
                head_dim: int = 128, eps: float = 1e-6, bq: int = 1024, gemm_fn=None) -> torch.Tensor:
    """The Qwen3-8B decoder layer as L2048/manifest.json's 14 launches compose it (data flow read
    from the kernels' index arithmetic): K00 rmsnorm -> K01/K03/K03 q/k/v projections -> K02/K04
    q/k norm + RoPE + head transpose -> K05 v transpose -> K06 causal GQA attention -> K07
    transpose back -> K08 o-projection + residual -> K00 rmsnorm -> K09 gate_up -> K10 silu_mul ->
    K11 down projection + residual.  gemm_fn(a, b, residual=None) replaces the fp64-summed gemm
    (the CPU baseline times the layer with the reference's fp32 matmul golden)."""
    gemm = gemm_fn or globals()["gemm"]
    t = x.shape[0]
    xn = rmsnorm(x, wts["w_in"], eps)
    q = gemm(xn, wts["wq"])
    k = gemm(xn, wts["wk"])
    v = gemm(xn, wts["wv"])
    qh = qk_norm_rope(q.view(t, hq, head_dim), wts["w_qn"], cos, sin, eps)
    kh = qk_norm_rope(k.view(t, hkv, head_dim), wts["w_kn"], cos, sin, eps)
    vh = transpose_heads(v.view(t, hkv, head_dim))
    oh = flash_attention(qh, kh, vh, hq, hkv, True, 1.0 / math.sqrt(head_dim), bq=bq, bkv=bq)
    o = transpose_heads(oh).view(t, hq * head_dim)
    h = gemm(o, wts["wo"], residual=x)
    hn = rmsnorm(h, wts["w_post"], eps)
    gu = gemm(hn, wts["wgu"])
    a = silu_mul(gu)
    return gemm(a, wts["wd"], residual=h)


# ---- single-token (decode) path ---------------------------------------------------------------

def sumsq(x: torch.Tensor, y: torch.Tensor | None = None) -> torch.Tensor:
    """D4096/00_..._3iwn5auz_triton.py:17-41: sum of float(x)^2 over the vector, fp32 (:34-41);
    D4096/05_..._tcz6sl32_triton.py:17-43: the same over float(x) + float(a), the sum kept in fp32
    (:34-38).  Returns shape [1]."""
    v = x.float().reshape(-1)
    if y is not None:
        v = v + y.float().reshape(-1)
    return (v * v).sum().reshape(1)


def gemv(x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """D4096/04_..._vumxrjnr_triton.py:17-42: y[n] = bf16(sum_k float(x[k]) * float(W[k, n]))
    with W [K, N] row-major (in_ptr1 + x0 + N*r0, :36), fp32 accumulation (:35-42)."""
    return (x.float().reshape(1, -1) @ w.float()).reshape(-1).to(BF16)


def gemv_rmsnorm(x: torch.Tensor, ss: torch.Tensor, g: torch.Tensor, w: torch.Tensor,
                 add: torch.Tensor | None = None, eps: float = 1e-6) -> torch.Tensor:
    """D4096/01_..._ddfn4f75_triton.py:17-55 (add None): r = rsqrt(ss/K + eps) (:41-45),
    xp = (float(x) * r) * float(g) (:46-49), y = bf16(sum_k xp[k] W[k, n]) (:50-55), no bf16
    rounding of xp.  D4096/06_..._5gopcdje_triton.py:17-57: the same with float(x) + float(a)
    summed in fp32 first (:41-42)."""
    k = w.shape[0]
    v = x.float().reshape(-1)
    if add is not None:
        v = v + add.float().reshape(-1)
    r = torch.rsqrt(ss.float().reshape(()) / float(k) + eps)
    xp = (v * r) * g.float().reshape(-1)
    return (xp.reshape(1, -1) @ w.float()).reshape(-1).to(BF16)


def gemv_silu(gu: torch.Tensor, w: torch.Tensor, res_a: torch.Tensor | None = None,
              res_b: torch.Tensor | None = None) -> torch.Tensor:
    """D4096/07_..._3d4ocw7y_triton.py:17-56: g = gu[:K], u = gu[K:] (:35-36); xp = (g / (exp(-g) + 1))
    * u in fp32 (:38-46); acc = sum_k xp[k] W[k, n] (:47-51); y = bf16(acc + (float(res_a) +
    float(res_b))) (:52-56)."""
    k = w.shape[0]
    gf = gu.float().reshape(-1)
    g, u = gf[:k], gf[k:2 * k]
    xp = (g / (torch.exp(-g) + 1.0)) * u
    acc = (xp.reshape(1, -1) @ w.float()).reshape(-1)
    if res_a is not None:
        r = res_a.float().reshape(-1)
        if res_b is not None:
            r = r + res_b.float().reshape(-1)
        acc = acc + r
    return acc.to(BF16)


def attention_decode(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float | None = None,
                     bkv: int | None = None) -> torch.Tensor:
    """attention_decode_32x8x4096_bf16/00__decode_kernel/_decode_kernel_triton.py:4-29.  q [NKV, G, D]
    (program pid = kv head reads q rows pid*G .. +G, :7-13), k/v [NKV, S, D].  Per block of bkv
    keys (the spec's BKV; every bundle spec has BKV = S): qk = (q @ k^T) * scale in fp32 (:21),
    m_new = max(m, rowmax) with m from -1e30 (:14, :22), alpha = exp(m - m_new), p = exp(qk - m_new)
    (:23-24), l = l*alpha + sum(p) (:25), acc = acc*alpha + bf16(p) @ v (:26); o = bf16(acc / l) (:28-29)."""
    nkv, g, d = q.shape
    s = k.shape[1]
    if scale is None:
        scale = 1.0 / math.sqrt(d)
    bkv = s if bkv is None else min(bkv, s)
    out = torch.empty_like(q)
    for h in range(nkv):
        qq = q[h].float()
        m_i = torch.full((g,), -1.0e30)
        l_i = torch.zeros(g)
        acc = torch.zeros(g, d)
        for st in range(0, s, bkv):
            kk = k[h, st:st + bkv].float()
            vv = v[h, st:st + bkv].float()
            qk = (qq @ kk.t()) * scale
            m_new = torch.maximum(m_i, qk.amax(dim=1))
            alpha = torch.exp(m_i - m_new)
            p = torch.exp(qk - m_new[:, None])
            l_i = l_i * alpha + p.sum(dim=1)
            acc = acc * alpha[:, None] + p.to(BF16).float() @ vv
            m_i = m_new
        out[h] = (acc / l_i[:, None]).to(BF16)
    return out


def qwen3_decode_layer(x: torch.Tensor, wts: dict, kcache: torch.Tensor, vcache: torch.Tensor,
                       cos: torch.Tensor, sin: torch.Tensor, hq: int = 32, hkv: int = 8, head_dim: int = 128,
                       eps: float = 1e-6) -> torch.Tensor:
    """D4096/manifest.json's 8 launches for one token over a KV cache [hkv, S, D] (data flow read
    from the kernels' index arithmetic): K00 ss = sum x^2 -> K01 q = (x*r*w_in) Wq -> K02 q-norm +
    RoPE (cos/sin of the token's position, [D]) -> K03 decode attention -> K04 a = o Wo ->
    K05 ss2 = sum (x+a)^2 -> K06 gu = ((x+a)*r2*w_post) Wgu -> K07 y = (silu(g)*u) Wd + (x + a)."""
    ss = sumsq(x)
    q = gemv_rmsnorm(x, ss, wts["w_in"], wts["wq"], eps=eps)
    qh = qk_norm_rope(q.view(1, hq, head_dim), wts["w_qn"], cos.reshape(1, head_dim), sin.reshape(1, head_dim), eps)
    o = attention_decode(qh.view(hkv, hq // hkv, head_dim), kcache, vcache, 1.0 / math.sqrt(head_dim))
    a = gemv(o.reshape(-1), wts["wo"])
    ss2 = sumsq(x, a)
    gu = gemv_rmsnorm(x, ss2, wts["w_post"], wts["wgu"], add=a, eps=eps)
    return gemv_silu(gu, wts["wd"], x, a)
