"""Parity of the MoE kernels (csrc/moe.hip, the grouped mode of csrc/gemm_bf16.hip) with the oracle's
restatements of the Qwen3-30B-A3B layer kernels (layer_op_* / layer_layer_*): integer and index
work bit-exact; bf16 outputs rtol 2e-2 with the absolute floor at 2e-2 of the output's mean
magnitude; fp32 sums within 1e-6 of the sum of |terms|."""
import pytest
import torch

import oracle
from helpers import assert_close, bits_equal
from ptb_amd import moe

pytestmark = pytest.mark.gpu

DEV = "cuda"
I64, I32, F32, BF16 = torch.int64, torch.int32, torch.float32, torch.bfloat16


def gen(seed):
    return torch.Generator().manual_seed(seed)


def close_scaled(got, want, what):
    scale = float(want.float().abs().mean()) + 1e-6
    assert_close(got, want, 2e-2, 2e-2 * max(scale, 1e-3), what)


def test_fill_cast_cumsum_table_count():
    z = torch.full((13,), 7, dtype=I64, device=DEV)
    assert moe.fill_zero(z).cpu().tolist() == [0] * 13
    zb = torch.ones(7, dtype=BF16, device=DEV)
    assert moe.fill_zero(zb).cpu().float().tolist() == [0.0] * 7
    x = torch.randint(-2 ** 40, 2 ** 40, (129,), generator=gen(0), dtype=I64)
    y = torch.empty(129, dtype=I32, device=DEV)
    assert torch.equal(moe.cast_i64_i32(x.to(DEV), y).cpu(), oracle.cast_i64_i32(x))
    for n, idt, odt in ((128, I32, I32), (128, I64, I64), (128, I64, I32), (5000, I64, I64), (1, I32, I64)):
        v = torch.randint(-100, 1000, (n,), generator=gen(n), dtype=idt)
        o, o2 = torch.empty(n, dtype=odt, device=DEV), torch.empty(n, dtype=odt, device=DEV)
        moe.cumsum(v.to(DEV), o, o2)
        want = oracle.cumsum_int(v, odt)
        assert torch.equal(o.cpu(), want) and torch.equal(o2.cpu(), want), (n, idt, odt)
    big = torch.full((6,), 2 ** 31 - 1, dtype=I64)
    o = torch.empty(6, dtype=I32, device=DEV)
    assert torch.equal(moe.cumsum(big.to(DEV), o).cpu(), oracle.cumsum_int(big, I32))     # int32 wrap
    counts = torch.randint(0, 3, (128,), generator=gen(1), dtype=I64)
    ends = torch.cumsum(counts, 0).to(I32)
    outs = [torch.empty(128, dtype=I64, device=DEV) for _ in range(3)]
    moe.group_table(ends.to(DEV), *outs)
    for got, want in zip(outs, oracle.group_table(ends)):
        assert torch.equal(got.cpu(), want)
    ne = oracle.group_table(ends)[0]
    for m in (128, 8, 300):
        c = torch.empty(m, dtype=I32, device=DEV)
        assert torch.equal(moe.count_le(ne.to(DEV), c).cpu(), oracle.count_le(ne, m)), m


@pytest.mark.parametrize("r,e,lo,hi", [(8192, 128, 0, 128), (32768, 128, 0, 128), (8, 128, 0, 128),
                                       (1000, 16, -3, 20), (64, 1024, 0, 1024), (65, 1, 0, 2)])
def test_expert_count_and_rank(r, e, lo, hi):
    ids = torch.randint(lo, hi, (r,), generator=gen(r + e), dtype=I64)
    counts, cum = torch.empty(e, dtype=I64, device=DEV), torch.empty(r * e, dtype=I64, device=DEV)
    counts2 = torch.empty(e, dtype=I64, device=DEV)
    idd = ids.to(DEV)
    moe.expert_count(idd, counts, cum, counts2)
    wc, wcum = oracle.expert_count(ids, e)
    assert torch.equal(counts.cpu(), wc) and torch.equal(counts2.cpu(), wc) and torch.equal(cum.cpu(), wcum)
    rank = torch.empty(r, dtype=I64, device=DEV)
    assert torch.equal(moe.rank_select(cum, idd, rank).cpu(), oracle.rank_select(wcum, ids, e))


@pytest.mark.parametrize("rows,e,kind,desc", [(1, 8192, "int", False), (1, 8, "int", False), (1, 32768, "int", False),
                                              (3, 12345, "int", False), (2, 1000, "float", True), (1, 20000, "float", False),
                                              (4, 4096, "float", True), (1, 1, "int", False), (5, 256, "float", False),
                                              (3, 200, "int", True), (2, 257, "int", False), (7, 63, "float", True)])
def test_sort_rows(rows, e, kind, desc):
    """The rank sort (rows of at most 256 keys), one bitonic workgroup (up to 8192), chunks plus merge
    passes beyond; ties, signed zeros, NaN and infinities keep the reference's order."""
    g = gen(rows * 7 + e)
    if kind == "int":
        x = torch.randint(0, 128, (rows * e,), generator=g, dtype=I64)          # many ties: stability matters
    else:
        x = torch.randn(rows * e, generator=g)
        x[::97] = 0.0
        x[5::211] = -0.0
        x[7::499] = float("nan")
        x[11::307] = float("inf")
    v = torch.empty_like(x, device=DEV)
    i = torch.empty(rows * e, dtype=I64, device=DEV)
    moe.sort_rows(x.to(DEV), v, i, rows, desc)
    wv, wi = oracle.sort_rows(x, rows, desc)
    assert torch.equal(i.cpu(), wi)
    assert bits_equal(v.cpu(), wv) if kind == "float" else torch.equal(v.cpu(), wv)


@pytest.mark.parametrize("rows,e,k,largest", [(1024, 128, 8, True), (1, 128, 8, True), (4096, 128, 8, True),
                                              (100, 1000, 5, False), (7, 64, 64, True), (3, 100, 65, True),
                                              (5, 33, 8, False), (2, 300, 16, True), (9, 1024, 64, False)])
def test_topk_rows(rows, e, k, largest):
    """Rows in registers with wave-argmax rounds (k <= 64, 1 to 16 values a lane, ragged e) and the
    LDS rank kernel (k = 65)."""
    x = torch.randn(rows * e, generator=gen(rows + k))
    x[3::17] = x[::17][: x[3::17].numel()]     # repeated values: ties by lowest position
    v, i = torch.empty(rows * k, device=DEV), torch.empty(rows * k, dtype=I64, device=DEV)
    moe.topk_rows(x.to(DEV), v, i, e, k, largest)
    wv, wi = oracle.topk_rows(x, e, k, largest)
    assert torch.equal(v.cpu(), wv) and torch.equal(i.cpu(), wi)


@pytest.mark.parametrize("e,k", [(64, 8), (100, 40), (300, 65), (1000, 100)])
@pytest.mark.parametrize("largest", [True, False])
def test_topk_rows_nan_and_signed_zero(e, k, largest):
    """Rows holding NaNs (of either sign) and both zeros: both kernels (k <= 64 in registers, k > 64
    through the LDS ranks) take the numbers first in value order, equal values (-0 == +0 included) by
    lower position, then the NaNs by position -- the oracle's order -- and return the elements' own
    values; a row of fewer than k elements other than the spent value ends in the reference's
    (spent, 0) rounds."""
    rows = 6
    x = torch.randn(rows * e, generator=gen(e + k)).view(rows, e)
    x[0, 5] = float("nan")
    x[0, 2] = -float("nan")
    x[1, :] = float("nan")                       # all NaN: positions in order
    x[2, 7], x[2, 3], x[2, 11] = 0.0, -0.0, 0.0
    x[3, ::3] = float("nan")
    x[4, :] = 0.0
    x[4, 1::2] = -0.0
    # mostly the spent value (-inf for the largest, +inf for the smallest), a few numbers and the
    # opposite infinity: fewer than k elements to take, then the reference's (spent, 0) tail
    spent = float("-inf") if largest else float("inf")
    x[5, :] = spent
    x[5, 3::17] = torch.randn(x[5, 3::17].numel(), generator=gen(k))
    x[5, 5::37] = -spent
    x = x.reshape(-1)
    v, i = torch.empty(rows * k, device=DEV), torch.empty(rows * k, dtype=I64, device=DEV)
    moe.topk_rows(x.to(DEV), v, i, e, k, largest)
    wv, wi = oracle.topk_rows(x, e, k, largest)
    assert torch.equal(i.cpu(), wi)
    got, want = v.cpu(), wv
    both_nan = torch.isnan(got) & torch.isnan(want)
    assert torch.equal(torch.isnan(got), torch.isnan(want))
    assert torch.equal(got[~both_nan].view(torch.int32), want[~both_nan].view(torch.int32))   # -0 stays -0


@pytest.mark.parametrize("t,k,c", [(1024, 8, 2048), (1, 8, 2048), (37, 3, 64)])
def test_gather_rows(t, k, c):
    r = t * k
    x = torch.randn(t * c, generator=gen(t)).to(BF16)
    slot = torch.randint(-r - 3, r + 3, (r,), generator=gen(t + 1), dtype=I64)    # negatives wrap, some miss
    out = torch.empty(r * c, dtype=BF16, device=DEV)
    moe.gather_rows(slot.to(DEV), x.to(DEV), out, k, c)
    assert bits_equal(out.cpu(), oracle.gather_rows(slot, x, k, c))


def _routing(t, e, k, seed, skew=False):
    g = gen(seed)
    logits = torch.randn(t, e, generator=g)
    if skew:   # most tokens prefer the first few experts: ragged groups, some empty
        logits[:, :4] += 3.0
    probs = oracle.softmax_rows(logits.to(BF16), F32)
    return oracle.topk_rows(probs.reshape(-1), e, k, True)


@pytest.mark.parametrize("t,c,residual", [(1024, 2048, False), (1024, 2048, True), (1, 2048, True), (33, 256, False)])
def test_combine(t, c, residual):
    e, k = 128, 8
    tv, ti = _routing(t, e, k, t + c)
    counts, cum = oracle.expert_count(ti, e)
    ends = oracle.cumsum_int(counts, I64)
    rank = oracle.rank_select(cum, ti, e)
    y = torch.randn(t * k * c, generator=gen(3)).to(BF16)
    if residual:
        wsum = oracle.row_sum(tv, t)
        h = torch.randn(t * c, generator=gen(4)).to(BF16)
        io = torch.randn(t * c, generator=gen(5)).to(BF16)
        want = oracle.combine(ti, ends, counts, rank, y, tv, t, k, c, wsum=wsum, h=h, io=io)
        out = io.to(DEV)
        moe.combine(ti.to(DEV), ends.to(DEV), counts.to(DEV), rank.to(DEV), y.to(DEV), tv.to(DEV), out, t, k, c,
                    wsum=wsum.to(DEV), h=h.to(DEV))
    else:
        w = tv.to(BF16)
        want = oracle.combine(ti, ends, counts, rank, y, w, t, k, c)
        out = torch.empty(t * c, dtype=BF16, device=DEV)
        moe.combine(ti.to(DEV), ends.to(DEV), counts.to(DEV), rank.to(DEV), y.to(DEV), w.to(DEV), out, t, k, c)
    close_scaled(out.cpu(), want, f"combine {t}x{c} residual={residual}")


def test_small_row_ops():
    x = torch.rand(1024 * 8, generator=gen(6)) + 0.05
    nb = torch.empty(1024 * 8, dtype=BF16, device=DEV)
    assert_close(moe.normalize_rows(x.to(DEV), nb, 8).cpu(), oracle.normalize_rows(x, 8), 2e-2, 1e-3, "normalize")
    rs = torch.empty(1024, device=DEV)
    got = moe.row_sum(x.to(DEV), rs).cpu()
    assert (got - oracle.row_sum(x, 1024)).abs().max() <= 1e-6 * 8
    for n in (2097152, 1000003, 3):
        a, b = torch.randn(n, generator=gen(n)).to(BF16), torch.randn(n, generator=gen(n + 1)).to(BF16)
        o = torch.empty(n, dtype=BF16, device=DEV)
        assert bits_equal(moe.add(a.to(DEV), b.to(DEV), o).cpu(), oracle.add_bf16(a, b))


@pytest.mark.parametrize("t,h", [(1024, 32), (1024, 4), (1, 32), (5, 3)])
def test_rope(t, h):
    x = torch.randn(t * h * 128, generator=gen(t + h)).to(BF16)
    cos_t, sin_t = oracle.rope_tables(t, 128, 1.0e6)
    out = torch.empty_like(x, device=DEV)
    moe.rope(x.to(DEV), cos_t.reshape(-1).to(DEV), sin_t.reshape(-1).to(DEV), out, t)
    close_scaled(out.cpu(), oracle.rope(x, cos_t.reshape(-1), sin_t.reshape(-1), t), f"rope {t}x{h}")


@pytest.mark.parametrize("rows,cols", [(1024, 2048), (1, 2048), (33, 136)])
def test_rmsnorm_add_and_broadcast(rows, cols):
    x = torch.randn(rows * cols, generator=gen(rows)).to(BF16)
    a = torch.randn(rows * cols, generator=gen(rows + 1)).to(BF16)
    w = (torch.randn(cols, generator=gen(2)) * 0.02 + 1).to(BF16)
    out = torch.empty(rows * cols, dtype=BF16, device=DEV)
    moe.rmsnorm_add(x.to(DEV), a.to(DEV), w.to(DEV), out)
    close_scaled(out.cpu(), oracle.rmsnorm_add(x, a, w), "rmsnorm_add")
    moe.rmsnorm_add(x.to(DEV), None, w.to(DEV), out)
    close_scaled(out.cpu(), oracle.rmsnorm_add(x, None, w), "rmsnorm (no add)")
    v = x[:cols].float() + a[:cols].float()
    ss = (v * v).sum().reshape(1)
    bc = torch.empty(8 * cols, dtype=BF16, device=DEV)
    moe.rms_broadcast(x[:cols].to(DEV), a[:cols].to(DEV), ss.to(DEV), w.to(DEV), bc)
    close_scaled(bc.cpu(), oracle.rms_broadcast(x[:cols], a[:cols], ss, w, 8), "rms_broadcast")


def _tables(ti, e):
    """The grouped GEMM's launch tables the layer builds: group ends, (starts, rows) with an empty
    129th entry, and program -> non-empty group (the rest pointing at the empty entry)."""
    counts, _ = oracle.expert_count(ti, e)
    ends = oracle.cumsum_int(counts, I32)
    nonempty, starts, rows = oracle.group_table(ends)
    starts = torch.cat([starts, torch.zeros(1, dtype=I64)]).to(I32)
    rows = torch.cat([rows, torch.zeros(1, dtype=I64)]).to(I32)
    group = oracle.count_le(nonempty, e)
    return group, starts, rows


@pytest.mark.parametrize("t,k_dim,n,skew", [(1024, 2048, 1536, False), (1024, 768, 2048, True), (1, 2048, 1536, False),
                                            (200, 512, 256, True), (1, 768, 2048, False), (2, 2048, 1536, True),
                                            (2, 128, 520, False)])
def test_grouped_gemm(t, k_dim, n, skew):
    """MFMA tiles for many rows; at most 16 rows (t <= 2 with top-8) the split-K GEMV form, with
    one row a group at decode and ragged groups of up to 2 rows when skewed."""
    e, k = 128, 8
    _, ti = _routing(t, e, k, t + n, skew)
    group, starts, rows = _tables(ti, e)
    r = t * k
    a = (torch.randn(r * k_dim, generator=gen(7)) / 8).to(BF16)
    b = (torch.randn(e * k_dim * n, generator=gen(8)) / 32).to(BF16)
    c0 = torch.randn(r * n, generator=gen(9)).to(BF16)
    c = c0.to(DEV)
    moe.grouped_gemm(a.to(DEV), b.to(DEV), group.to(DEV), starts.to(DEV), rows.to(DEV), c, k_dim, n, k_dim * n)
    want = oracle.grouped_mm(a, b, group, starts, rows, k_dim, n, k_dim * n, c=c0)
    close_scaled(c.cpu(), want, f"grouped gemm {t}x{k_dim}x{n} skew={skew}")


def test_grouped_gemm_skips_tables_outside_a():
    """Programs whose table entry points outside A or B count as empty; C stays as it was."""
    k_dim, n = 128, 64
    a = torch.randn(64 * k_dim, generator=gen(10)).to(BF16)
    b = torch.randn(2 * k_dim * n, generator=gen(11)).to(BF16)
    group = torch.tensor([0, 1, 2, 5, -1], dtype=I32)
    starts = torch.tensor([0, 60, 10, 0], dtype=I32)
    rows = torch.tensor([16, 8, 4, 0], dtype=I32)          # group 1 runs past A's 64 rows; group 2 has no weight
    c0 = torch.randn(64 * n, generator=gen(12)).to(BF16)
    c = c0.to(DEV)
    moe.grouped_gemm(a.to(DEV), b.to(DEV), group.to(DEV), starts.to(DEV), rows.to(DEV), c, k_dim, n, k_dim * n)
    want = c0.clone().reshape(64, n)
    want[:16] = (a.reshape(64, k_dim)[:16].double() @ b.reshape(2, k_dim, n)[0].double()).to(F32).to(BF16)
    close_scaled(c.cpu(), want.reshape(-1), "grouped gemm with bad tables")
    assert torch.equal(c.cpu().reshape(64, n)[16:], c0.reshape(64, n)[16:])


@pytest.mark.parametrize("gemv", [True, False])
def test_grouped_gemm_few_rows_tables(gemv):
    """Sixteen rows of A (the GEMV form when allowed): a group of 6 rows (two passes of 4 over the
    weight slice), a group listed by two programs, entries past A's rows, past the weights and
    negative, and rows no program covers keep C's values; both forms give the same result."""
    k_dim, n = 256, 136
    a = torch.randn(16 * k_dim, generator=gen(20)).to(BF16)
    b = (torch.randn(3 * k_dim * n, generator=gen(21)) / 8).to(BF16)
    group = torch.tensor([0, 1, 1, 2, 3, -1, 4], dtype=I32)
    starts = torch.tensor([0, 6, 14, 9, 0], dtype=I32)
    rows = torch.tensor([6, 3, 3, 2, 0], dtype=I32)   # group 2 runs past row 16; group 3 has no weight
    c0 = torch.randn(16 * n, generator=gen(22)).to(BF16)
    c = c0.to(DEV)
    moe.grouped_gemm(a.to(DEV), b.to(DEV), group.to(DEV), starts.to(DEV), rows.to(DEV), c, k_dim, n, k_dim * n,
                     gemv=gemv)
    want = oracle.grouped_mm(a, b, group, starts, rows, k_dim, n, k_dim * n, c=c0)
    close_scaled(c.cpu(), want, f"grouped gemm few rows gemv={gemv}")
    assert torch.equal(c.cpu().reshape(16, n)[9:], c0.reshape(16, n)[9:])


def test_moe_layer_chain_matches_the_oracle():
    """Router -> dispatch -> gate_up grouped GEMM -> silu -> down grouped GEMM -> combine at the
    bundle's Qwen3-30B-A3B sizes (hidden 2048, 128 experts, top 8, expert width 768), all on the GPU
    through moe.*, against the oracle chain on the same inputs."""
    t, c, e, k, inter = 64, 2048, 128, 8, 768
    x = torch.randn(t * c, generator=gen(13)).to(BF16)
    logits = torch.randn(t * e, generator=gen(14)).to(BF16)
    wgu = (torch.randn(e * c * 2 * inter, generator=gen(15)) / 45).to(BF16)
    wd = (torch.randn(e * inter * c, generator=gen(16)) / 28).to(BF16)
    h = torch.randn(t * c, generator=gen(17)).to(BF16)
    d = {n: v.to(DEV) for n, v in dict(x=x, logits=logits, wgu=wgu, wd=wd, h=h).items()}
    from ptb_amd import ops

    probs = ops.softmax_rows(d["logits"].view(t, e), out_dtype=F32).reshape(-1)
    tv, ti = torch.empty(t * k, device=DEV), torch.empty(t * k, dtype=I64, device=DEV)
    moe.topk_rows(probs, tv, ti, e, k, True)
    wsum = moe.row_sum(tv, torch.empty(t, device=DEV))
    sv, order = torch.empty(t * k, dtype=I64, device=DEV), torch.empty(t * k, dtype=I64, device=DEV)
    moe.sort_rows(ti, sv, order, 1)
    xs = moe.gather_rows(order, d["x"], torch.empty(t * k * c, dtype=BF16, device=DEV), k, c)
    counts, cum = torch.empty(e, dtype=I64, device=DEV), torch.empty(t * k * e, dtype=I64, device=DEV)
    moe.expert_count(ti, counts, cum)
    ends = moe.cumsum(counts, torch.empty(e, dtype=I32, device=DEV))
    ne, st, rw = (torch.empty(e, dtype=I64, device=DEV) for _ in range(3))
    moe.group_table(ends, ne, st, rw)
    starts = torch.cat([st, torch.zeros(1, dtype=I64, device=DEV)]).to(I32)
    rows = torch.cat([rw, torch.zeros(1, dtype=I64, device=DEV)]).to(I32)
    group = moe.count_le(ne, torch.empty(e, dtype=I32, device=DEV))
    gu = torch.empty(t * k * 2 * inter, dtype=BF16, device=DEV)
    moe.grouped_gemm(xs, d["wgu"], group, starts, rows, gu, c, 2 * inter, c * 2 * inter)
    act = ops.silu_mul(gu.view(t * k, 2 * inter)).reshape(-1)
    y = torch.empty(t * k * c, dtype=BF16, device=DEV)
    moe.grouped_gemm(act, d["wd"], group, starts, rows, y, inter, c, inter * c)
    rank = moe.rank_select(cum, ti, torch.empty(t * k, dtype=I64, device=DEV))
    io = torch.zeros(t * c, dtype=BF16, device=DEV)
    moe.combine(ti, ends.to(I64), counts, rank, y, tv, io, t, k, c, wsum=wsum, h=d["h"])
    got = io.cpu()

    # the oracle chain on the same inputs, step by step
    p_o = oracle.softmax_rows(logits.view(t, e), F32).reshape(-1)
    tv_o, ti_o = oracle.topk_rows(p_o, e, k, True)
    assert torch.equal(ti.cpu(), ti_o)
    wsum_o = oracle.row_sum(tv_o, t)
    _, order_o = oracle.sort_rows(ti_o, 1)
    xs_o = oracle.gather_rows(order_o, x, k, c)
    counts_o, cum_o = oracle.expert_count(ti_o, e)
    group_o, starts_o, rows_o = _tables(ti_o, e)
    gu_o = oracle.grouped_mm(xs_o, wgu, group_o, starts_o, rows_o, c, 2 * inter, c * 2 * inter)
    act_o = oracle.silu_mul(gu_o.view(t * k, 2 * inter)).reshape(-1)
    y_o = oracle.grouped_mm(act_o, wd, group_o, starts_o, rows_o, inter, c, inter * c)
    ends_o = oracle.cumsum_int(counts_o, I64)
    rank_o = oracle.rank_select(cum_o, ti_o, e)
    want = oracle.combine(ti_o, ends_o, counts_o, rank_o, y_o, tv_o, t, k, c, wsum=wsum_o, h=h,
                          io=torch.zeros(t * c, dtype=BF16))
    close_scaled(got, want, "moe layer chain")


def test_grouped_gemm_repeated_groups_fill_the_grid():
    """The MFMA form with large groups listed by several programs: repeats take no tiles, so the
    later programs' rows are still computed (without that, 3 programs over 2 groups of 512 rows
    need 12 row tiles where the grid has ceil(1024 / 128) + 3 = 11)."""
    k_dim, n, a_rows = 256, 512, 1024
    a = (torch.randn(a_rows * k_dim, generator=gen(30)) / 8).to(BF16)
    b = (torch.randn(2 * k_dim * n, generator=gen(31)) / 16).to(BF16)
    group = torch.tensor([0, 0, 1, 0], dtype=I32)
    starts = torch.tensor([0, 512], dtype=I32)
    rows = torch.tensor([512, 512], dtype=I32)
    c0 = torch.randn(a_rows * n, generator=gen(32)).to(BF16)
    c = c0.to(DEV)
    moe.grouped_gemm(a.to(DEV), b.to(DEV), group.to(DEV), starts.to(DEV), rows.to(DEV), c, k_dim, n, k_dim * n,
                     gemv=False)
    want = oracle.grouped_mm(a, b, group, starts, rows, k_dim, n, k_dim * n, c=c0)
    close_scaled(c.cpu(), want, "grouped gemm, repeated groups")
