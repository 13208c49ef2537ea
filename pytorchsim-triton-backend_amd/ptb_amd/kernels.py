"""Map a reference kernel (its spec or manifest, plus the Triton source when at hand) to the HIP
kernel family that executes it, and run it over flat device tensors.

The reference compiles each Inductor-generated Triton kernel to its own ELF; here every kernel of
the hot path is one of a few hand-written HIP families, chosen from what the spec states:

  attention   ``_prefill_kernel`` with constexprs HQ, G, S, D, CAUSAL, SCALE
              (attention_prefill_*/00__prefill_kernel/_prefill_kernel_triton.py:4-44)
  gemm        args arg_A, arg_B, out_ptr0 (+ a leading in_ptr0 residual): the ``mm`` and RESIDENT
              templates (qwen3_8b_layer_prefill_*/01, 03, 08, 09, 11; gemm_<M>x<K>x<N>_bf16)
  rmsnorm     x, w, out with a mean/rsqrt reduction over w's length (.../00_..._gwdq6qer)
  qk_norm_rope x, w[D], cos, sin (fp32), out head-major (.../02, 04)
  transpose   one bf16 in, one bf16 out, an affine permutation of [A, B, D] -> [B, A, D]
              (.../05, 07), read from the kernel's index expressions
  silu_mul    in [T, 2I] -> out [T, I] (.../10); I from the kernel's index expressions
  softmax     ``softmax`` kernels with scalars xnumel (rows), r0_numel (cols) (vector_softmax_*)
  reduce      whole-tensor ``sum`` / ``max`` into one fp32 (vector_sum_*, vector_max_*)
  add_scalar  ``fused_add``: bf16(x + c) (vector_add1_*)
  slice_add   fp32 out[i] = x[first + i] + c (vector_slice_*)
  attention_decode ``_decode_kernel`` with constexprs HKV, G, S, D (attention_decode_*/00,
              qwen3_8b_layer_decode_*/03)
  sumsq       sum of squares of one bf16 vector (or of the sum of two) into one fp32
              (qwen3_8b_layer_decode_*/00, 05)
  gemv        out[N] = sum_k xp[k] * W[k, N] with W [K, N] row-major: plain (decode 04 and the M = 1
              ``mm`` template), with an RMSNorm prologue over a precomputed sum of squares (decode
              01, 06), or with a silu(g)*u prologue and a residual sum epilogue (decode 07)

The Qwen3-30B-A3B (MoE) layer's kernels (layer_op_* and layer_layer_*), identified by name
fragment, argument roles, dtypes and sizes (no source needed):

  fill_zero, cast, cumsum, group_table, count_le   the expert-table bookkeeping around the grouped
              GEMM (``new_zeros``, ``_to_copy``, ``cumsum``, ``cat_cumsum_gt_new_zeros_slice_sub``,
              ``arange_..._le_sum``)
  expert_count, rank_select   per-expert slot counts with each slot's running rank
              (``arange_cumsum_eq_sum``, ``arange_eq_mul_sum``)
  sort, topk  ``_sort_kernel`` (stable, int64 or fp32 keys) and ``_topk_kernel``
  gather_rows, rms_broadcast   token rows laid out slot by slot (``floor_divide_index_select``; the
              single-token form fused with the RMSNorm)
  combine     the weighted sum of each token's expert rows (``index_select_mul_sub_sum``), with
              bf16 weights, or fp32 weights over their sum plus the residual
  normalize_rows, row_sum, add, rope, rmsnorm_add   router weights over their sum, their row sums,
              the residual add, RoPE without the norm, and add + RMSNorm
  grouped_mm  ``_grouped_mm_kernel``

Anything else raises :class:`UnsupportedKernel` -- there is no fallback execution.
"""
from __future__ import annotations

import math
import re
from dataclasses import dataclass, field

from .contract import KernelSpec


class UnsupportedKernel(ValueError):
    pass


@dataclass
class Plan:
    family: str
    params: dict = field(default_factory=dict)


# ---------------------------------------------------------------- Triton source helpers
_DECOMP = re.compile(r"^\s*(x\d+)\s*=\s*(.+?)\s*$", re.M)


def _index_terms(expr: str) -> dict:
    """'x0 + 128*x2 + 1024*x1' -> {'x0': 1, 'x2': 128, 'x1': 1024} (affine, positive strides)."""
    out = {}
    for term in expr.replace(" ", "").split("+"):
        if not term:
            continue
        m = re.fullmatch(r"(?:(\d+)\*)?\(?([a-z]\w*)\)?(?:\*(\d+))?", term)
        if not m:
            m2 = re.fullmatch(r"\(?(\d+)\)?", term)
            if m2:
                out["const"] = out.get("const", 0) + int(m2.group(1))
                continue
            raise UnsupportedKernel(f"index term {term!r} is not affine")
        coef = int(m.group(1) or m.group(3) or 1)
        out[m.group(2)] = out.get(m.group(2), 0) + coef
    return out


def _decomposition(src: str) -> dict:
    """x-variable definitions of a pointwise Inductor kernel: name -> (divisor, modulus or None)."""
    out = {}
    for name, rhs in _DECOMP.findall(src):
        r = rhs.replace(" ", "")
        m = re.fullmatch(r"\(*xindex(?://(\d+))?\)*(?:%(\d+))?\)*", r)
        if m:
            out[name] = (int(m.group(1) or 1), int(m.group(2)) if m.group(2) else None)
    return out


def _load_index(src: str, ptr: str) -> str:
    m = re.search(r"tl\.load\(\s*" + re.escape(ptr) + r"\s*\+\s*\((.*?)\)\s*,", src)
    if not m:
        raise UnsupportedKernel(f"no affine load of {ptr} in the kernel source")
    return m.group(1)


def _permutation_from_source(src: str, numel: int):
    """For a [A, B, D] -> [B, A, D] copy kernel: (A, B, D) from its index expressions."""
    dec = _decomposition(src)
    terms = _index_terms(_load_index(src, "in_ptr0"))
    # output dims from the decomposition: innermost x (divisor 1, modulus D), middle (divisor D,
    # modulus n1), outer (divisor D*n1)
    inner = [v for v, (d, mod) in dec.items() if d == 1 and mod]
    if len(inner) != 1:
        raise UnsupportedKernel("cannot find the innermost index of the copy kernel")
    xi = inner[0]
    d = dec[xi][1]
    mid = [v for v, (dv, mod) in dec.items() if dv == d and mod]
    outer = [v for v, (dv, mod) in dec.items() if dv > d and mod is None]
    if len(mid) != 1 or len(outer) != 1:
        raise UnsupportedKernel("copy kernel is not a 3-D permutation")
    xm, xo = mid[0], outer[0]
    n_mid = dec[xm][1]
    n_out = numel // (d * n_mid)
    # input strides: inner must be 1; y[o, m, i] = x[...]; the transpose family needs x = [m][o][i]
    if terms.get(xi) != 1 or terms.get(xo) != d or terms.get(xm) != d * n_out or terms.get("const"):
        raise UnsupportedKernel(f"copy kernel's input strides {terms} are not a head transpose")
    return n_mid, n_out, d   # x is [n_mid, n_out, d], y is [n_out, n_mid, d]


def _row_length_from_source(src: str) -> int:
    """silu_mul: the gate row length I from 'x0 = (xindex % I)'."""
    for _, (dv, mod) in _decomposition(src).items():
        if dv == 1 and mod:
            return mod
    raise UnsupportedKernel("cannot read the gate width from the silu_mul kernel")


def _float_constant(src: str, default: float) -> float:
    m = re.search(r"tl\.full\(\[1\],\s*([-0-9.e]+),\s*tl\.float32\)", src or "")
    return float(m.group(1)) if m else default


# ---------------------------------------------------------------- resolution
def _names(spec):
    return [a.name for a in spec.args]


def _gemv_plan(spec: KernelSpec, source: str | None) -> Plan | None:
    """The decode layer's matrix-vector kernels, recognised by their operands: one bf16 output of N
    values, a bf16 weight of K*N values read row-major (``in_ptrW + (x0 + N*r0_1)``, checked when
    the source is at hand) and the vector operands beside it."""
    pure = [a for a in spec.args if a.role == "in"]
    outs = spec.outputs()
    if len(outs) != 1 or outs[0].dtype != "bfloat16" or len(pure) < 2:
        return None
    y = outs[0]
    n = y.numel
    w = max(pure, key=lambda a: a.numel)
    if w.dtype != "bfloat16" or n == 0 or w.numel % n or w.numel == n:
        return None
    k = w.numel // n
    rest = [a for a in pure if a is not w]
    name = spec.name
    scal = [a for a in rest if a.dtype == "float32" and a.numel == 1]
    vecs = [a for a in rest if a.dtype == "bfloat16" and a.numel == k]
    plan = None
    if "silu" in name:
        gu = [a for a in rest if a.dtype == "bfloat16" and a.numel == 2 * k]
        res = [a for a in rest if a.dtype == "bfloat16" and a.numel == n]
        if len(gu) == 1 and len(res) <= 2 and len(rest) == 1 + len(res):
            plan = Plan("gemv", dict(mode="silu", k=k, n=n, x=gu[0].name, w=w.name, y=y.name,
                                     res_a=res[0].name if res else None, res_b=res[1].name if len(res) > 1 else None))
    elif "rsqrt" in name and len(scal) == 1 and len(rest) == len(vecs) + 1 and len(vecs) in (2, 3):
        # argument order: x (, a) before the sum of squares, the norm weight after it
        ss = scal[0]
        before = [a for a in vecs if rest.index(a) < rest.index(ss)]
        after = [a for a in vecs if rest.index(a) > rest.index(ss)]
        if len(after) == 1 and len(before) in (1, 2):
            plan = Plan("gemv", dict(mode="rms", k=k, n=n, x=before[0].name,
                                     add=before[1].name if len(before) == 2 else None, ss=ss.name,
                                     g=after[0].name, eps=1e-6, w=w.name, y=y.name))
    elif len(rest) == 1 and len(vecs) == 1:
        plan = Plan("gemv", dict(mode="plain", k=k, n=n, x=vecs[0].name, w=w.name, y=y.name))
    if plan is not None and source:
        terms = _index_terms(_load_index(source, w.name))
        if terms != {"x0": 1, "r0_1": n}:
            raise UnsupportedKernel(f"{name}: W is read as {terms}, not row-major [K, N]")
    return plan


_I64, _I32, _F32, _BF16 = "int64", "int32", "float32", "bfloat16"


def _moe_plan(spec: KernelSpec, name: str, sizes) -> Plan | None:
    """The MoE layer's kernels; None when `spec` is not one of them."""
    ce = spec.constexprs or {}
    pure = [a for a in spec.args if a.role == "in"]
    outs = [a for a in spec.args if a.role in ("out", "inout")]
    n_grid = 1
    for g in spec.grid:
        n_grid *= int(g)

    def need(ok: bool, why: str):
        if not ok:
            raise UnsupportedKernel(f"{name}: {why}")

    if name == "_sort_kernel":
        x, v, i = spec.arg("x_ptr"), spec.arg("v_ptr"), spec.arg("i_ptr")
        rows = n_grid
        need(x.dtype in (_I64, _F32) and v.dtype == x.dtype and i.dtype == _I64, "sort keys int64 or fp32")
        need(bool(ce.get("FLOAT", False)) == (x.dtype == _F32), "FLOAT constexpr and key dtype disagree")
        need(x.numel % rows == 0 and v.numel == x.numel == i.numel, "sort rows do not divide the keys")
        return Plan("sort", dict(rows=rows, e=x.numel // rows, descending=bool(ce.get("DESCENDING", False)),
                                 x=x.name, v=v.name, i=i.name))
    if name == "_topk_kernel":
        x, v, i = spec.arg("x_ptr"), spec.arg("v_ptr"), spec.arg("i_ptr")
        e, k = int(ce["E"]), int(ce["K"])
        need(x.dtype == _F32 and v.dtype == _F32 and i.dtype == _I64, "top-k over fp32")
        need(x.numel % e == 0 and v.numel == i.numel == (x.numel // e) * k, "top-k sizes")
        return Plan("topk", dict(e=e, k=k, largest=bool(ce.get("LARGEST", True)), x=x.name, v=v.name, i=i.name))
    if name == "_grouped_mm_kernel":
        a, b, c = spec.arg("a_ptr"), spec.arg("b_ptr"), spec.arg("c_ptr")
        k, n = int(ce["K"]), int(ce["N"])
        sbg, sbk, sbn = int(ce["sbg"]), int(ce["sbk"]), int(ce["sbn"])
        need(sbn == 1 and sbk == n, "grouped weights are not row-major [K, N]")
        need(int(ce.get("BN", n)) * int(spec.grid[1] if len(spec.grid) > 1 else 1) >= n, "column tiles short of N")
        need(a.dtype == b.dtype == c.dtype == _BF16 and a.numel % k == 0 and c.numel == a.numel // k * n,
             "grouped GEMM operand sizes")
        return Plan("grouped_mm", dict(k=k, n=n, stride=sbg, a_rows=a.numel // k, nprog=spec.arg("group_ptr").numel,
                                       nweights=b.numel // sbg, a=a.name, b=b.name, group="group_ptr",
                                       start="start_ptr", rows="rows_ptr", c=c.name))
    if not name.startswith("pytorchsim_triton_compiler_fused"):
        return None
    if "new_zeros" in name and not pure and len(outs) == 1 and "cumsum" not in name:
        return Plan("fill_zero", dict(y=outs[0].name))
    if "cumsum_eq_sum" in name:
        need(len(pure) == 1 and pure[0].dtype == _I64 and all(o.dtype == _I64 for o in outs), "expert histogram")
        r = pure[0].numel
        small = [o for o in outs if any(q.numel == o.numel * r for q in outs if q is not o)]
        big = [o for o in outs if o not in small]
        need(len(big) == 1 and 1 <= len(small) <= 2, "expert histogram outputs")
        e = small[0].numel
        return Plan("expert_count", dict(r=r, e=e, ids=pure[0].name, counts=small[0].name,
                                         counts2=small[1].name if len(small) == 2 else None, cum=big[0].name))
    if "eq_mul_sum" in name:
        need(len(pure) == 2 and len(outs) == 1 and all(a.dtype == _I64 for a in pure + outs), "rank select")
        cum, ids = sorted(pure, key=lambda a: -a.numel)
        need(cum.numel % ids.numel == 0 and outs[0].numel == ids.numel, "rank select sizes")
        return Plan("rank_select", dict(r=ids.numel, e=cum.numel // ids.numel, cum=cum.name, ids=ids.name,
                                        y=outs[0].name))
    if "cat_cumsum_gt_new_zeros_slice_sub" in name:
        need(len(pure) == 1 and len(outs) == 3 and pure[0].dtype in (_I32, _I64)
             and all(o.dtype == _I64 and o.numel == pure[0].numel for o in outs), "group table")
        return Plan("group_table", dict(n=pure[0].numel, ends=pure[0].name, nonempty=outs[0].name,
                                        starts=outs[1].name, rows=outs[2].name))
    if "cumsum" in name:
        need(len(pure) == 1 and 1 <= len(outs) <= 2 and pure[0].dtype in (_I32, _I64)
             and all(o.dtype == outs[0].dtype and o.dtype in (_I32, _I64) and o.numel == pure[0].numel for o in outs),
             "integer scan")
        return Plan("cumsum", dict(n=pure[0].numel, x=pure[0].name, y=outs[0].name,
                                   y2=outs[1].name if len(outs) == 2 else None))
    if "_le_" in name and len(pure) == 1 and len(outs) == 1 and pure[0].dtype == _I64 and outs[0].dtype == _I32:
        return Plan("count_le", dict(n=pure[0].numel, m=outs[0].numel, x=pure[0].name, y=outs[0].name))
    if (len(pure) == 1 and len(outs) == 1 and pure[0].dtype == _I64 and outs[0].dtype == _I32
            and pure[0].numel == outs[0].numel):
        return Plan("cast", dict(n=pure[0].numel, x=pure[0].name, y=outs[0].name))
    if "floor_divide_index_select" in name and "rsqrt" in name:
        slot, x, a, ss, w = pure
        need(len(outs) == 1 and slot.dtype == _I64 and ss.dtype == _F32 and ss.numel == 1
             and x.dtype == a.dtype == w.dtype == outs[0].dtype == _BF16 and x.numel == a.numel == w.numel
             and outs[0].numel == slot.numel * x.numel, "single-token dispatch with RMSNorm")
        return Plan("rms_broadcast", dict(rows=slot.numel, cols=x.numel, eps=1e-6, x=x.name, a=a.name, ss=ss.name,
                                          w=w.name, y=outs[0].name))
    if "floor_divide_index_select" in name:
        need(len(pure) == 2 and len(outs) == 1, "dispatch gather args")
        slot, x = pure
        r = slot.numel
        need(slot.dtype == _I64 and x.dtype == outs[0].dtype == _BF16 and outs[0].numel % r == 0, "dispatch gather")
        cols = outs[0].numel // r
        t = x.numel // cols
        need(t > 0 and x.numel == t * cols and r % t == 0, "dispatch gather sizes")
        return Plan("gather_rows", dict(r=r, t=t, k=r // t, cols=cols, slot=slot.name, x=x.name, y=outs[0].name))
    if "index_select_mul_sub_sum" in name:
        io = [a for a in spec.args if a.role == "inout"]
        if io:   # (h + io) + sum_j y * (w / wsum)
            need(len(pure) == 8, "combine with residual args")
            ids, ends, counts, rank, y, w, wsum, h = pure
            tokens, cols = wsum.numel, h.numel // wsum.numel
            out = io[0]
            need(w.dtype == wsum.dtype == _F32 and h.dtype == out.dtype == _BF16, "combine with residual dtypes")
        else:
            need(len(pure) == 6 and len(outs) == 1, "combine args")
            ids, ends, counts, rank, y, w = pure
            out, wsum, h = outs[0], None, None
            need(w.dtype == _BF16 and out.dtype == _BF16, "combine dtypes")
            cols = y.numel // ids.numel
            tokens = out.numel // cols
        k = ids.numel // tokens if tokens else 0
        need(tokens > 0 and k > 0 and ids.numel == tokens * k and out.numel == tokens * cols and y.numel % cols == 0
             and all(a.dtype == _I64 for a in (ids, ends, counts, rank)) and y.dtype == _BF16, "combine sizes")
        return Plan("combine", dict(tokens=tokens, k=k, cols=cols, ids=ids.name, ends=ends.name, counts=counts.name,
                                    rank=rank.name, y=y.name, w=w.name, wsum=wsum.name if wsum else None,
                                    h=h.name if h else None, out=out.name))
    if "div_sum" in name and len(pure) == 1 and len(outs) == 1:
        k = sizes("r0_numel")
        need(bool(k) and pure[0].dtype == _F32 and outs[0].dtype == _BF16 and pure[0].numel == outs[0].numel
             and pure[0].numel % k == 0, "router weight normalisation")
        return Plan("normalize_rows", dict(k=k, n=pure[0].numel, x=pure[0].name, y=outs[0].name))
    if ("_sum_" in name or name.endswith("sum") or "fused_sum" in name) and len(pure) == 1 and len(outs) == 1 \
            and pure[0].dtype == outs[0].dtype == _F32 and outs[0].numel > 1 and pure[0].numel % outs[0].numel == 0:
        return Plan("row_sum", dict(rows=outs[0].numel, n=pure[0].numel, x=pure[0].name, y=outs[0].name))
    if "fused_add_" in name and len(pure) == 2 and len(outs) == 1 and \
            all(a.dtype == _BF16 and a.numel == outs[0].numel for a in pure + outs):
        return Plan("add", dict(n=outs[0].numel, a=pure[0].name, b=pure[1].name, y=outs[0].name))
    if "cat_mul_neg_slice" in name and "rsqrt" not in name and len(pure) == 3 and len(outs) == 1:
        x, cs, sn = pure
        tokens = cs.numel // 128
        need(x.dtype == outs[0].dtype == _BF16 and cs.dtype == sn.dtype == _F32 and cs.numel == sn.numel == tokens * 128
             and tokens > 0 and x.numel % (tokens * 128) == 0 and outs[0].numel == x.numel, "RoPE sizes")
        return Plan("rope", dict(tokens=tokens, n=x.numel, x=x.name, cos=cs.name, sin=sn.name, y=outs[0].name))
    if ("rsqrt" in name and "mean" in name and "_mm_" not in name and len(pure) == 3 and len(outs) == 1
            and pure[0].numel == pure[1].numel == outs[0].numel and pure[2].numel < pure[0].numel
            and all(a.dtype == _BF16 for a in pure + outs)):
        x, a, w = pure
        need(x.numel % w.numel == 0, "add + RMSNorm rows")
        return Plan("rmsnorm_add", dict(rows=x.numel // w.numel, cols=w.numel, eps=1e-6, x=x.name, a=a.name, w=w.name,
                                        y=outs[0].name))
    return None


def resolve(spec: KernelSpec, source: str | None = None) -> Plan:
    """The HIP family and its parameters for one reference kernel."""
    names = _names(spec)
    ce = spec.constexprs or {}
    sv = spec.scalar_values
    # index facts a manifest may carry instead of the Triton source (see kernel_hints)
    hints = (spec.extra or {}).get("hints", {})
    name = spec.name
    if {"HKV", "G", "S", "D"} <= set(ce) and "decode" in name:
        if len(spec.args) != 4:
            raise UnsupportedKernel(f"{name}: decode attention takes q, k, v, o")
        hkv, g, s, d = int(ce["HKV"]), int(ce["G"]), int(ce["S"]), int(ce["D"])
        q = spec.args[0]
        nkv = q.numel // (g * d)
        if nkv * g * d != q.numel or spec.args[1].numel != nkv * s * d:
            raise UnsupportedKernel(f"{name}: q/k sizes do not match HKV={hkv}, G={g}, S={s}, D={d}")
        return Plan("attention_decode", dict(nkv=nkv, group=g, seq=s, head_dim=d,
                                             scale=float(ce.get("SCALE", 1.0 / math.sqrt(d))),
                                             q=names[0], k=names[1], v=names[2], o=names[3]))
    if {"HQ", "G", "S", "D"} <= set(ce):
        q = spec.args[0]
        hq, g, s, d = int(ce["HQ"]), int(ce["G"]), int(ce["S"]), int(ce["D"])
        if "decode" in name:
            raise UnsupportedKernel(f"{name}: decode attention with these constexprs is not on the HIP path")
        if len(spec.args) != 4:
            raise UnsupportedKernel(f"{name}: attention takes q, k, v, o")
        return Plan("attention", dict(batch=q.numel // (hq * s * d), hq=hq, hkv=hq // g, seq=s, head_dim=d,
                                      causal=bool(ce.get("CAUSAL", True)),
                                      scale=float(ce.get("SCALE", 1.0 / math.sqrt(d))),
                                      q=names[0], k=names[1], v=names[2], o=names[3]))
    if "arg_A" in names and "arg_B" in names:
        a, b = spec.arg("arg_A"), spec.arg("arg_B")
        outs = spec.outputs()
        if len(outs) != 1:
            raise UnsupportedKernel(f"{name}: a GEMM with {len(outs)} outputs")
        c = outs[0]
        m2 = a.numel * c.numel / b.numel
        m = int(round(math.sqrt(m2)))
        if m <= 0 or m * m != int(round(m2)):
            raise UnsupportedKernel(f"{name}: operand sizes {a.numel}, {b.numel}, {c.numel} are not a GEMM")
        k, n = a.numel // m, c.numel // m
        resid = [x for x in spec.inputs() if x.name not in ("arg_A", "arg_B")]
        return Plan("gemm", dict(m=m, k=k, n=n, residual=resid[0].name if resid else None, a="arg_A", b="arg_B",
                                 c=c.name))
    ins, outs = spec.inputs(), spec.outputs()

    def sizes(key):  # a size the kernel pins as a runtime scalar or as a constexpr
        v = sv.get(key, ce.get(key))
        return int(v) if v is not None else None

    moe_plan = _moe_plan(spec, name, sizes)
    if moe_plan is not None:
        return moe_plan

    if "softmax" in name and len(ins) == 1 and len(outs) == 1:
        cols = sizes("r0_numel")
        if not cols or ins[0].numel % cols:
            raise UnsupportedKernel(f"{name}: softmax needs its row length r0_numel")
        if ins[0].dtype != "bfloat16" or outs[0].dtype not in ("bfloat16", "float32"):
            raise UnsupportedKernel(f"{name}: softmax reads bf16 and writes bf16 or fp32")
        return Plan("softmax", dict(rows=ins[0].numel // cols, cols=cols, x=ins[0].name, y=outs[0].name,
                                    out_f32=outs[0].dtype == "float32"))
    if "_mm_" in name and len(ins) == 2 and len(outs) == 1 and sizes("r0_numel") and sizes("xnumel"):
        # the M = 1 template: out[n] = sum_k in0[k] * in1[k * N + n] (gemm_1x<K>x<N>_bf16)
        k, n = sizes("r0_numel"), sizes("xnumel")
        a, b = ins
        if source:
            terms = _index_terms(_load_index(source, b.name))
            if terms != {"x0": 1, "r0_1": n}:
                raise UnsupportedKernel(f"{name}: the M = 1 template reads B as {terms}, not row-major [K, N]")
        if a.numel == k and b.numel == k * n and outs[0].numel == n:
            return Plan("gemv", dict(mode="plain", k=k, n=n, x=a.name, w=b.name, y=outs[0].name))
    pure = [a for a in spec.args if a.role == "in"]
    if ("pow" in name and "mean" in name and "mm" not in name and "rsqrt" not in name and len(outs) == 1
            and outs[0].numel == 1 and outs[0].dtype == "float32" and 1 <= len(pure) <= 2
            and all(a.dtype == "bfloat16" and a.numel == pure[0].numel for a in pure)):
        return Plan("sumsq", dict(n=pure[0].numel, x=pure[0].name, y=pure[1].name if len(pure) == 2 else None,
                                  out=outs[0].name))
    gv = _gemv_plan(spec, source)
    if gv is not None:
        return gv
    if len(ins) == 1 and len(outs) == 1 and outs[0].dtype == "float32" and "slice" in name:
        # out[i] = float(x[first + i]) + c: the load offset and the constant from the source
        first = int(hints.get("first", 0))
        if source:
            m = re.search(r"tl\.load\(\s*" + re.escape(ins[0].name) + r"\s*\+\s*\(\s*(\d+)\s*\)\s*\)", source)
            if not m:
                raise UnsupportedKernel(f"{name}: the slice kernel does not load one fixed element")
            first = int(m.group(1))
        return Plan("slice_add", dict(first=first, count=outs[0].numel, s=_float_constant(source, 1.0), x=ins[0].name,
                                      y=outs[0].name))
    if (len(ins) == 1 and len(outs) == 1 and outs[0].numel == 1 and outs[0].dtype == "float32"
            and ins[0].dtype in ("bfloat16", "float32")):
        if "_sum_" in name or name.endswith("sum"):
            return Plan("reduce", dict(op="sum", n=ins[0].numel, x=ins[0].name, y=outs[0].name,
                                       in_f32=ins[0].dtype == "float32"))
        if "_max_" in name or name.endswith("max"):
            return Plan("reduce", dict(op="max", n=ins[0].numel, x=ins[0].name, y=outs[0].name,
                                       in_f32=ins[0].dtype == "float32"))
    if "rsqrt" in name and "mean" in name:
        if len(ins) == 2 and len(outs) == 1:
            x, w = ins
            return Plan("rmsnorm", dict(rows=x.numel // w.numel, cols=w.numel, eps=1e-6, x=x.name, w=w.name,
                                        y=outs[0].name))
        if len(pure) == 4 and len(outs) == 1:
            x, w, cs, sn = pure
            d = w.numel
            t = cs.numel // d
            return Plan("qk_norm_rope", dict(tokens=t, heads=x.numel // (t * d), head_dim=d, eps=1e-6, x=x.name,
                                             w=w.name, cos=cs.name, sin=sn.name, y=outs[0].name))
    if len(ins) == 1 and len(outs) == 1 and ins[0].dtype == outs[0].dtype == "bfloat16":
        x, y = ins[0], outs[0]
        if "silu" in name and x.numel == 2 * y.numel:
            if "inter" in hints:
                inter = int(hints["inter"])
            elif source:
                inter = _row_length_from_source(source)
            else:
                raise UnsupportedKernel(f"{name}: silu_mul needs the kernel source (or an 'inter' hint)")
            return Plan("silu_mul", dict(rows=y.numel // inter, inter=inter, x=x.name, y=y.name))
        if "transpose" in name and x.numel == y.numel:
            if {"d0", "d1", "inner"} <= set(hints):
                d0, d1, inner = int(hints["d0"]), int(hints["d1"]), int(hints["inner"])
            elif source:
                d0, d1, inner = _permutation_from_source(source, x.numel)
            else:
                raise UnsupportedKernel(f"{name}: a transpose needs the kernel source (or d0/d1/inner hints)")
            if d0 * d1 * inner != x.numel:
                raise UnsupportedKernel(f"{name}: transpose dims {d0}x{d1}x{inner} do not cover {x.numel} elements")
            return Plan("transpose", dict(d0=d0, d1=d1, inner=inner, x=x.name, y=y.name))
        if "fused_add" in name and x.numel == y.numel:
            return Plan("add_scalar", dict(s=_float_constant(source, 1.0), n=x.numel, x=x.name, y=y.name))
    raise UnsupportedKernel(f"{name}: no HIP kernel family matches this kernel")


def kernel_hints(plan: Plan) -> dict:
    """The index facts of a plan that :func:`resolve` otherwise reads from the Triton source, for a
    manifest to carry under ``extra["hints"]`` when the source does not travel with it."""
    if plan.family == "transpose":
        return {k: plan.params[k] for k in ("d0", "d1", "inner")}
    if plan.family == "silu_mul":
        return {"inter": plan.params["inter"]}
    if plan.family == "slice_add":
        return {"first": plan.params["first"]}
    return {}


# ---------------------------------------------------------------- execution
def run(plan: Plan, tensors: dict) -> None:
    """Launch `plan` on the current stream over flat device tensors keyed by argument name."""
    from . import ops

    p, t = plan.params, tensors
    f = plan.family
    if f == "gemm":
        m, k, n = p["m"], p["k"], p["n"]
        r = t[p["residual"]].view(m, n) if p["residual"] else None
        ops.gemm(t[p["a"]].view(m, k), t[p["b"]].view(k, n), r, out=t[p["c"]].view(m, n))
    elif f == "attention":
        bh, s, d = p["batch"] * p["hq"], p["seq"], p["head_dim"]
        q, k, v, o = t[p["q"]], t[p["k"]], t[p["v"]], t[p["o"]]
        kv = p["batch"] * p["hkv"]
        ops.flash_attention(q.view(bh, s, d), k.view(kv, s, d), v.view(kv, s, d), p["hq"], p["hkv"], p["causal"],
                            p["scale"], out=o.view(bh, s, d))
    elif f == "rmsnorm":
        ops.rmsnorm(t[p["x"]].view(p["rows"], p["cols"]), t[p["w"]], p["eps"], out=t[p["y"]].view(p["rows"], p["cols"]))
    elif f == "qk_norm_rope":
        tk, h, d = p["tokens"], p["heads"], p["head_dim"]
        ops.qk_norm_rope(t[p["x"]].view(tk, h, d), t[p["w"]], t[p["cos"]].view(tk, d), t[p["sin"]].view(tk, d),
                         p["eps"], out=t[p["y"]].view(h, tk, d))
    elif f == "transpose":
        ops.transpose_heads(t[p["x"]].view(p["d0"], p["d1"], p["inner"]), out=t[p["y"]].view(p["d1"], p["d0"], p["inner"]))
    elif f == "silu_mul":
        ops.silu_mul(t[p["x"]].view(p["rows"], 2 * p["inter"]), out=t[p["y"]].view(p["rows"], p["inter"]))
    elif f == "softmax":
        ops.softmax_rows(t[p["x"]].view(p["rows"], p["cols"]), out=t[p["y"]].view(p["rows"], p["cols"]),
                         out_dtype=ops.F32 if p["out_f32"] else ops.BF16)
    elif f == "reduce":
        ops.reduce(t[p["x"]], p["op"], out=t[p["y"]])
    elif f == "add_scalar":
        ops.add_scalar(t[p["x"]], p["s"], out=t[p["y"]])
    elif f == "slice_add":
        ops.slice_add(t[p["x"]], p["first"], p["count"], p["s"], out=t[p["y"]])
    elif f == "attention_decode":
        nkv, g, s, d = p["nkv"], p["group"], p["seq"], p["head_dim"]
        ops.attention_decode(t[p["q"]].view(nkv, g, d), t[p["k"]].view(nkv, s, d), t[p["v"]].view(nkv, s, d),
                             p["scale"], out=t[p["o"]].view(nkv, g, d))
    elif f == "sumsq":
        ops.sumsq(t[p["x"]], t[p["y"]] if p["y"] else None, out=t[p["out"]])
    elif f == "gemv":
        k, n = p["k"], p["n"]
        w, y = t[p["w"]].view(k, n), t[p["y"]]
        if p["mode"] == "plain":
            ops.gemv(t[p["x"]], w, out=y)
        elif p["mode"] == "rms":
            ops.gemv_rmsnorm(t[p["x"]], t[p["ss"]], t[p["g"]], w, add=t[p["add"]] if p["add"] else None,
                             eps=p["eps"], out=y)
        else:
            ops.gemv_silu(t[p["x"]], w, t[p["res_a"]] if p["res_a"] else None,
                          t[p["res_b"]] if p["res_b"] else None, out=y)
    elif f in _MOE_FAMILIES:
        _run_moe(plan, t)
    else:
        raise UnsupportedKernel(f"unknown family {f}")


_MOE_FAMILIES = {"fill_zero", "cast", "cumsum", "group_table", "count_le", "expert_count", "rank_select", "sort",
                 "topk", "gather_rows", "rms_broadcast", "combine", "normalize_rows", "row_sum", "add", "rope",
                 "rmsnorm_add", "grouped_mm"}


def _run_moe(plan: Plan, t: dict) -> None:
    from . import moe

    p, f = plan.params, plan.family
    if f == "fill_zero":
        moe.fill_zero(t[p["y"]])
    elif f == "cast":
        moe.cast_i64_i32(t[p["x"]], t[p["y"]])
    elif f == "cumsum":
        moe.cumsum(t[p["x"]], t[p["y"]], t[p["y2"]] if p["y2"] else None)
    elif f == "group_table":
        moe.group_table(t[p["ends"]], t[p["nonempty"]], t[p["starts"]], t[p["rows"]])
    elif f == "count_le":
        moe.count_le(t[p["x"]], t[p["y"]])
    elif f == "expert_count":
        moe.expert_count(t[p["ids"]], t[p["counts"]], t[p["cum"]], t[p["counts2"]] if p["counts2"] else None)
    elif f == "rank_select":
        moe.rank_select(t[p["cum"]], t[p["ids"]], t[p["y"]])
    elif f == "sort":
        moe.sort_rows(t[p["x"]], t[p["v"]], t[p["i"]], p["rows"], p["descending"])
    elif f == "topk":
        moe.topk_rows(t[p["x"]], t[p["v"]], t[p["i"]], p["e"], p["k"], p["largest"])
    elif f == "gather_rows":
        moe.gather_rows(t[p["slot"]], t[p["x"]], t[p["y"]], p["k"], p["cols"])
    elif f == "rms_broadcast":
        moe.rms_broadcast(t[p["x"]], t[p["a"]], t[p["ss"]], t[p["w"]], t[p["y"]], p["eps"])
    elif f == "combine":
        moe.combine(t[p["ids"]], t[p["ends"]], t[p["counts"]], t[p["rank"]], t[p["y"]], t[p["w"]], t[p["out"]],
                    p["tokens"], p["k"], p["cols"], wsum=t[p["wsum"]] if p["wsum"] else None,
                    h=t[p["h"]] if p["h"] else None)
    elif f == "normalize_rows":
        moe.normalize_rows(t[p["x"]], t[p["y"]], p["k"])
    elif f == "row_sum":
        moe.row_sum(t[p["x"]], t[p["y"]])
    elif f == "add":
        moe.add(t[p["a"]], t[p["b"]], t[p["y"]])
    elif f == "rope":
        moe.rope(t[p["x"]], t[p["cos"]], t[p["sin"]], t[p["y"]], p["tokens"])
    elif f == "rmsnorm_add":
        moe.rmsnorm_add(t[p["x"]], t[p["a"]], t[p["w"]], t[p["y"]], p["eps"])
    elif f == "grouped_mm":
        moe.grouped_gemm(t[p["a"]], t[p["b"]], t[p["group"]], t[p["start"]], t[p["rows"]], t[p["c"]], p["k"], p["n"],
                         p["stride"])


def launch(spec: KernelSpec, tensors: dict, source: str | None = None) -> Plan:
    """Resolve and run one kernel; returns the plan it ran."""
    plan = resolve(spec, source)
    run(plan, tensors)
    return plan


def work_of(plan: Plan) -> tuple:
    """(flops, algorithmic HBM bytes) of one launch -- each operand read once, each output written
    once; flop conventions as the reference's reports use them (2MNK per GEMM, 4*H*D*S(S+1)/2 for
    causal attention, validation/attention/emit_report.py:295; vector ops by element,
    validation/vector/emit_report.py:20-39)."""
    p, f = plan.params, plan.family
    if f == "gemm":
        m, k, n = p["m"], p["k"], p["n"]
        return 2.0 * m * n * k, 2.0 * (m * k + k * n + m * n * (2 if p["residual"] else 1))
    if f == "attention":
        h, d, s = p["batch"] * p["hq"], p["head_dim"], p["seq"]
        pairs = s * (s + 1) / 2 if p["causal"] else s * s
        return 4.0 * h * d * pairs, 2.0 * d * s * (2 * h + 2 * p["batch"] * p["hkv"])
    if f == "rmsnorm":
        r, c = p["rows"], p["cols"]
        return 4.0 * r * c, 2.0 * (2 * r * c + c)
    if f == "qk_norm_rope":
        n = p["tokens"] * p["heads"] * p["head_dim"]
        return 10.0 * n, 4.0 * n + 8.0 * p["tokens"] * p["head_dim"]
    if f == "transpose":
        n = p["d0"] * p["d1"] * p["inner"]
        return 0.0, 4.0 * n
    if f == "silu_mul":
        n = p["rows"] * p["inter"]
        return 5.0 * n, 6.0 * n
    if f == "softmax":
        n = p["rows"] * p["cols"]
        return 5.0 * n, (6.0 if p.get("out_f32") else 4.0) * n
    if f == "reduce":
        return float(p["n"]), (4.0 if p.get("in_f32") else 2.0) * p["n"] + 4.0
    if f == "add_scalar":
        return float(p["n"]), 4.0 * p["n"]
    if f == "slice_add":
        return float(p["count"]), 6.0 * p["count"]
    if f == "attention_decode":
        rows, s, d = p["nkv"] * p["group"], p["seq"], p["head_dim"]
        return 4.0 * rows * d * s, 2.0 * (2 * p["nkv"] * s * d + 2 * rows * d)
    if f == "sumsq":
        return (3.0 if p["y"] else 2.0) * p["n"], (4.0 if p["y"] else 2.0) * p["n"] + 4.0
    if f == "gemv":
        k, n = p["k"], p["n"]
        xk = 2 * k if p["mode"] == "silu" else k
        extra = {"plain": 0, "rms": 2 * k + 4 + (2 * k if p.get("add") else 0),
                 "silu": 2 * n * ((1 if p.get("res_a") else 0) + (1 if p.get("res_b") else 0))}[p["mode"]]
        return 2.0 * k * n, 2.0 * (k * n + xk + n) + extra
    # the MoE kernels: bytes each must move (index tables at their width), flops where they compute
    if f == "grouped_mm":   # every row of A through one weight; each program's weight read once
        r, k, n = p["a_rows"], p["k"], p["n"]
        return 2.0 * r * k * n, 2.0 * (r * k + r * n + min(p["nprog"], p["nweights"]) * k * n)
    if f in ("fill_zero", "cast", "cumsum", "count_le"):
        n = p.get("n", p.get("m", 1))
        return float(n), 12.0 * n
    if f == "group_table":
        return float(p["n"]), 32.0 * p["n"]
    if f == "expert_count":
        return float(p["r"] * p["e"]), 8.0 * (p["r"] + p["r"] * p["e"] + p["e"])
    if f == "rank_select":
        return float(p["r"]), 24.0 * p["r"]
    if f == "sort":
        n = p["rows"] * p["e"]
        return n * max(1.0, math.log2(max(p["e"], 2))), 24.0 * n
    if f == "topk":
        return float(p["k"]) * p["e"] * 2, 4.0 * p["e"] + 12.0 * p["k"]
    if f == "gather_rows":
        return 0.0, 2.0 * 2 * p["r"] * p["cols"] + 8.0 * p["r"]
    if f == "rms_broadcast":
        return 4.0 * p["rows"] * p["cols"], 2.0 * (3 * p["cols"] + p["rows"] * p["cols"]) + 4.0
    if f == "combine":
        tk, c = p["tokens"] * p["k"], p["cols"]
        res = 3 if p["h"] else 1
        return 2.0 * tk * c, 2.0 * (tk * c + res * p["tokens"] * c) + 32.0 * tk
    if f == "normalize_rows":
        return 2.0 * p["n"], 6.0 * p["n"]
    if f == "row_sum":
        return float(p["n"]), 4.0 * (p["n"] + p["rows"])
    if f == "add":
        return float(p["n"]), 6.0 * p["n"]
    if f == "rope":
        return 3.0 * p["n"], 4.0 * p["n"] + 8.0 * 128 * p["tokens"]
    if f == "rmsnorm_add":
        n = p["rows"] * p["cols"]
        return 5.0 * n, 6.0 * n + 2.0 * p["cols"]
    raise UnsupportedKernel(f"unknown family {f}")
