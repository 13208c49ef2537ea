"""Pins for the MoE oracle (oracle/moe.py): library routines and brute-force loops on the same
inputs, and the routing invariant that dispatch -> experts -> combine reproduces the dense mixture.
Each check is chosen so a plausible slip (an off-by-one rank, a swapped ends/counts, a floor that
truncates, an unstable tie) fails it."""
import math

import pytest
import torch

import oracle

I64, I32, F32, BF16 = torch.int64, torch.int32, torch.float32, torch.bfloat16


def gen(seed):
    return torch.Generator().manual_seed(seed)


def test_cumsum_and_int32_wrap():
    x = torch.randint(-50, 50, (128,), generator=gen(0), dtype=I64)
    want, run = [], 0
    for v in x.tolist():
        run += v
        want.append(run)
    assert oracle.cumsum_int(x, I64).tolist() == want
    big = torch.full((4,), 2 ** 31 - 1, dtype=I64)          # wraps in int32 as a cast-then-scan does
    got = oracle.cumsum_int(big, I32).tolist()
    assert got == [((v + 2 ** 31) % 2 ** 32) - 2 ** 31 for v in [(2 ** 31 - 1) * (i + 1) for i in range(4)]]


def test_group_table_by_hand():
    ends = torch.tensor([3, 3, 7, 7, 8], dtype=I32)
    nonempty, starts, rows = oracle.group_table(ends)
    assert starts.tolist() == [0, 3, 3, 7, 7]
    assert rows.tolist() == [3, 0, 4, 0, 1]
    assert nonempty.tolist() == [1, 1, 2, 2, 3]


def test_count_le_is_a_searchsorted():
    x = torch.sort(torch.randint(0, 40, (64,), generator=gen(1), dtype=I64)).values
    got = oracle.count_le(x, 50)
    want = torch.searchsorted(x, torch.arange(50, dtype=I64), right=True).to(I32)
    assert torch.equal(got, want)
    xu = torch.randint(-5, 60, (33,), generator=gen(2), dtype=I64)          # unsorted: brute force
    assert oracle.count_le(xu, 70).tolist() == [sum(1 for v in xu.tolist() if v <= i) for i in range(70)]


def test_expert_count_and_rank_against_loops():
    e = 16
    ids = torch.randint(-2, e + 2, (200,), generator=gen(3), dtype=I64)     # some ids outside [0, E)
    counts, cum = oracle.expert_count(ids, e)
    assert counts.tolist() == [sum(1 for v in ids.tolist() if v == x) for x in range(e)]
    c = cum.reshape(200, e)
    seen = [0] * e
    for s, v in enumerate(ids.tolist()):
        if 0 <= v < e:
            seen[v] += 1
        assert c[s].tolist() == seen
    rank = oracle.rank_select(cum, ids, e)
    for s, v in enumerate(ids.tolist()):
        want = c[s, v].item() if 0 <= v < e else 0
        assert rank[s].item() == want
    # every valid slot's rank is in 1..count of its expert and ranks within an expert are 1..count
    for x in range(e):
        r = sorted(rank[ids == x].tolist())
        assert r == list(range(1, counts[x].item() + 1))


def _brute_sort(vals, descending):
    """Stable order by value with NaN above +inf and -0 equal to +0; descending puts larger values
    first, equal values still in position order."""
    def key(v):
        if math.isnan(v):
            return (2, 0.0)
        return (1, 0.0 if v == 0 else v)
    if descending:
        return sorted(range(len(vals)), key=lambda i: ((-key(vals[i])[0], -key(vals[i])[1]), i))
    return sorted(range(len(vals)), key=lambda i: (key(vals[i]), i))


@pytest.mark.parametrize("descending", [False, True])
def test_sort_is_the_stable_sort(descending):
    x = torch.randint(-5, 5, (3, 40), generator=gen(4), dtype=I64)
    vals, idx = oracle.sort_rows(x.reshape(-1), 3, descending)
    tv, ti = torch.sort(x, dim=1, stable=True, descending=descending)
    assert torch.equal(vals.reshape(3, 40), tv) and torch.equal(idx.reshape(3, 40), ti)
    f = torch.tensor([1.5, -0.0, 0.0, float("nan"), -2.0, float("inf"), 0.0, -float("inf"), 1.5, float("nan")])
    fv, fi = oracle.sort_rows(f, 1, descending)
    assert fi.tolist() == _brute_sort(f.tolist(), descending)
    # -0 comes back as +0 and every NaN as the one canonical NaN, as the key map does
    assert all(not (v == 0 and math.copysign(1, v) < 0) for v in fv.tolist())


def test_topk_against_library_and_ties():
    x = torch.randn(12, 128, generator=gen(5))
    v, i = oracle.topk_rows(x.reshape(-1), 128, 8, True)
    tv, ti = torch.topk(x, 8, dim=1, largest=True, sorted=True)
    assert torch.equal(v.reshape(12, 8), tv) and torch.equal(i.reshape(12, 8), ti)
    v, i = oracle.topk_rows(x.reshape(-1), 128, 8, False)
    tv, ti = torch.topk(x, 8, dim=1, largest=False, sorted=True)
    assert torch.equal(v.reshape(12, 8), tv) and torch.equal(i.reshape(12, 8), ti)
    t = torch.tensor([[1.0, 3.0, 3.0, 2.0, 3.0]])
    v, i = oracle.topk_rows(t.reshape(-1), 5, 4, True)
    assert v.tolist() == [3.0, 3.0, 3.0, 2.0] and i.tolist() == [1, 2, 4, 3]    # ties: lowest position first


def test_topk_spent_values_follow_the_reference_rounds():
    """Rows holding the spent value itself (-inf for the largest, +inf for the smallest): worked
    by hand through _topk_kernel_triton.py:17-25, a round that finds only spent values left
    reports (spent, column 0) however often it runs, and a spent value is never reported by its
    own column."""
    inf = float("inf")
    v, i = oracle.topk_rows(torch.tensor([1.0, -inf, 2.0, -inf]), 4, 4, True)
    assert v.tolist() == [2.0, 1.0, -inf, -inf] and i.tolist() == [2, 0, 0, 0]
    v, i = oracle.topk_rows(torch.tensor([1.0, inf, 2.0, inf]), 4, 4, False)
    assert v.tolist() == [1.0, 2.0, inf, inf] and i.tolist() == [0, 2, 0, 0]
    v, i = oracle.topk_rows(torch.tensor([-inf, 5.0, -inf]), 3, 3, True)
    assert v.tolist() == [5.0, -inf, -inf] and i.tolist() == [1, 0, 0]
    # the opposite infinity is an ordinary value
    v, i = oracle.topk_rows(torch.tensor([inf, 1.0, inf]), 3, 3, True)
    assert v.tolist() == [inf, inf, 1.0] and i.tolist() == [0, 2, 1]
    # random rows with spent values sprinkled in: the rounds before the spent tail are torch.topk
    # over the other values (stable: lower column first), the tail is (spent, 0)
    x = torch.randn(40, 50, generator=gen(9))
    x[torch.rand(40, 50, generator=gen(10)) < 0.5] = -inf
    v, i = oracle.topk_rows(x.reshape(-1), 50, 30, True)
    v, i = v.reshape(40, 30), i.reshape(40, 30)
    for r in range(40):
        live = torch.nonzero(x[r] > -inf).flatten()
        n = min(30, live.numel())
        order = live[torch.sort(x[r, live], descending=True, stable=True).indices][:n]
        assert torch.equal(i[r, :n], order) and torch.equal(v[r, :n], x[r, order])
        assert (i[r, n:] == 0).all() and (v[r, n:] == -inf).all()


def test_gather_rows_floor_and_wrap():
    x = torch.arange(5 * 8, dtype=F32).to(BF16).reshape(5, 8)
    slot = torch.tensor([0, 7, 8, 39, -1, -8, -9, 40, -41], dtype=I64)
    got = oracle.gather_rows(slot, x.reshape(-1), 8, 8).reshape(-1, 8)
    for j, s in enumerate(slot.tolist()):
        t = math.floor(s / 8)
        t = t + 5 if t < 0 else t
        want = x[t] if 0 <= t < 5 else torch.zeros(8, dtype=BF16)
        assert torch.equal(got[j], want), (s, t)


def _route(x, e, k, seed):
    """A real routing of tokens x [T, C] over e experts: router logits -> softmax -> top-k ->
    normalised weights; then the slot order the dispatch sort gives."""
    t = x.shape[0]
    logits = torch.randn(t, e, generator=gen(seed))
    probs = oracle.softmax_rows(logits.to(BF16), F32)
    tv, ti = oracle.topk_rows(probs.reshape(-1), e, k, True)
    return tv, ti


def test_dispatch_experts_combine_reproduce_the_dense_mixture():
    """Tokens routed to k of e experts (each expert a linear map), through the bundle's kernel
    sequence (sort, histogram, rank, group table, gather, grouped GEMM, combine) equal the dense
    mixture sum_j w_j (x W_{e_j}) within bf16 rounding."""
    t, c, n, e, k = 24, 64, 64, 8, 2
    x = torch.randn(t, c, generator=gen(6)).to(BF16)
    wts = (torch.randn(e, c, n, generator=gen(7)) / 8).to(BF16)
    tv, ti = _route(x, e, k, 8)
    wsum = oracle.row_sum(tv, t)
    # dispatch: sort slots by expert, gather token rows in that order
    sv, order = oracle.sort_rows(ti, 1)
    xs = oracle.gather_rows(order, x.reshape(-1), k, c)
    counts, cum = oracle.expert_count(ti, e)
    ends = oracle.cumsum_int(counts, I32)
    nonempty, starts, rows = oracle.group_table(ends)
    group = (oracle.count_le(nonempty, e)).to(I32)      # program p -> the p-th non-empty group
    y = oracle.grouped_mm(xs, wts.reshape(-1), group, starts.to(I32), rows.to(I32), c, n, c * n)
    rank = oracle.rank_select(cum, ti, e)
    got = oracle.combine(ti, ends.to(I64), counts, rank, y, tv, t, k, n, wsum=wsum,
                         h=torch.zeros(t * n, dtype=BF16), io=torch.zeros(t * n, dtype=BF16)).reshape(t, n).float()
    dense = torch.zeros(t, n, dtype=torch.float64)
    for s in range(t):
        for j in range(k):
            ex = int(ti[s * k + j])
            dense[s] += (tv[s * k + j] / wsum[s]).double() * (x[s].double() @ wts[ex].double()).to(F32).to(BF16).double()
    assert torch.allclose(got.double(), dense, rtol=2e-2, atol=2e-2 * float(dense.abs().mean()))
    # a wrong rank (off by one) or swapped ends/counts breaks the identity
    bad = oracle.combine(ti, counts, ends.to(I64), rank, y, tv, t, k, n, wsum=wsum,
                         h=torch.zeros(t * n, dtype=BF16), io=torch.zeros(t * n, dtype=BF16)).reshape(t, n).float()
    assert not torch.allclose(bad.double(), dense, rtol=2e-2, atol=2e-2 * float(dense.abs().mean()))


def test_combine_bf16_weights_without_residual():
    t, k, c, e = 3, 2, 8, 4
    ids = torch.tensor([0, 1, 1, 3, 0, 3], dtype=I64)
    counts, cum = oracle.expert_count(ids, e)
    ends = oracle.cumsum_int(counts, I64)
    rank = oracle.rank_select(cum, ids, e)
    y = torch.arange(6 * c, dtype=F32).to(BF16)
    w = torch.tensor([0.5, 0.25, 1.0, 2.0, -1.0, 0.5]).to(BF16)
    got = oracle.combine(ids, ends, counts, rank, y, w, t, k, c).reshape(t, c).float()
    yr = y.reshape(6, c).float()
    # expert rows: expert 0 -> rows 0, 1 (slots 0, 4); expert 1 -> 2, 3 (slots 1, 2); expert 3 -> 4, 5 (slots 3, 5)
    want = torch.stack([0.5 * yr[0] + 0.25 * yr[2], 1.0 * yr[3] + 2.0 * yr[4], -1.0 * yr[1] + 0.5 * yr[5]])
    assert torch.equal(got, want.to(BF16).float())


def test_small_row_ops():
    x = torch.rand(10, 8, generator=gen(9)) + 0.1
    nr = oracle.normalize_rows(x.reshape(-1), 8).reshape(10, 8)
    assert torch.equal(nr, (x / x.sum(1, keepdim=True)).to(BF16))
    rs = oracle.row_sum(x.reshape(-1), 10)
    assert all(abs(rs[i].item() - math.fsum(x[i].tolist())) <= 1e-6 * 8 for i in range(10))
    a, b = torch.randn(100, generator=gen(10)).to(BF16), torch.randn(100, generator=gen(11)).to(BF16)
    assert torch.equal(oracle.add_bf16(a, b), (a.double() + b.double()).to(F32).to(BF16))


def test_rope_matches_rotate_half_in_fp64():
    t, h = 5, 3
    x = torch.randn(t, h, 128, generator=gen(12)).to(BF16)
    ang = torch.rand(t, 128, generator=gen(13)) * 6
    cos, sin = torch.cos(ang), torch.sin(ang)
    got = oracle.rope(x.reshape(-1), cos.reshape(-1), sin.reshape(-1), t).reshape(t, h, 128).double()
    xd = x.double()
    rot = torch.cat([-xd[..., 64:], xd[..., :64]], -1)
    want = xd * cos.double()[:, None] + rot * sin.double()[:, None]
    assert torch.allclose(got, want, rtol=1e-2, atol=1e-2)
    ident = oracle.rope(x.reshape(-1), torch.ones(t * 128), torch.zeros(t * 128), t)
    assert torch.equal(ident, x.reshape(-1))                     # cos = 1, sin = 0: the identity


def test_rmsnorm_add_and_broadcast():
    x, a = torch.randn(6, 256, generator=gen(14)).to(BF16), torch.randn(6, 256, generator=gen(15)).to(BF16)
    w = (torch.randn(256, generator=gen(16)) * 0.1 + 1).to(BF16)
    got = oracle.rmsnorm_add(x.reshape(-1), a.reshape(-1), w).reshape(6, 256)
    v = x.double() + a.double()
    want = torch.nn.functional.rms_norm(v, (256,), w.double(), eps=1e-6)
    assert torch.allclose(got.double(), want, rtol=1e-2, atol=1e-2)
    ss = (v[0] * v[0]).sum().float()
    bc = oracle.rms_broadcast(x[0], a[0], ss, w, 3).reshape(3, 256)
    for r in range(3):
        assert torch.allclose(bc[r].float(), got[0].float(), rtol=1e-2, atol=1e-2)


def test_grouped_mm_against_per_group_loops():
    k, n = 16, 24
    rows = torch.tensor([3, 0, 5, 2, 0], dtype=I32)
    starts = torch.tensor([0, 3, 3, 8, 10], dtype=I32)
    a = torch.randn(10, k, generator=gen(17)).to(BF16)
    b = torch.randn(5, k, n, generator=gen(18)).to(BF16)
    group = torch.tensor([2, 0, 3, 4, 4], dtype=I32)          # program order is not group order
    c0 = torch.full((10 * n,), 7.0).to(BF16)
    got = oracle.grouped_mm(a.reshape(-1), b.reshape(-1), group, starts, rows, k, n, k * n, c=c0).reshape(10, n)
    want = c0.reshape(10, n).clone()
    for g in (2, 0, 3):
        s0, nr = int(starts[g]), int(rows[g])
        for i in range(s0, s0 + nr):
            for j in range(n):
                exact = math.fsum(float(a[i, q]) * float(b[g, q, j]) for q in range(k))
                want[i, j] = torch.tensor(exact, dtype=torch.float64).to(F32).to(BF16)
    assert torch.equal(got, want.to(BF16))


def test_fill_zero_cast_and_slice_add_closed_forms():
    """The three small helpers, each against values written out by hand: fill_zero is n zeros of
    the asked dtype; the int64 -> int32 cast keeps the low 32 bits as two's complement; slice_add
    is float(x[first + j]) + s for j < count."""
    z = oracle.fill_zero(5)
    assert z.dtype == torch.int64 and z.tolist() == [0, 0, 0, 0, 0]
    assert oracle.fill_zero(3, torch.int32).dtype == torch.int32
    x = torch.tensor([0, 1, -1, 2 ** 31 - 1, 2 ** 31, 2 ** 32 + 5, -(2 ** 31) - 1, 2 ** 40 + 2 ** 31 + 7])
    want = [0, 1, -1, 2147483647, -2147483648, 5, 2147483647, -2147483641]
    got = oracle.cast_i64_i32(x)
    assert got.dtype == torch.int32 and got.tolist() == want
    v = torch.tensor([1.5, -2.0, 0.25, 3.0, 1e-8], dtype=torch.bfloat16)
    s = oracle.slice_add(v, first=1, count=3, s=1.0)
    assert s.dtype == torch.float32
    assert s.tolist() == [-1.0, 1.25, 4.0]
    assert oracle.slice_add(v).tolist() == [2.5]          # the bundle kernel: x[0] + 1
    tiny = oracle.slice_add(v, first=4, count=1, s=1.0)
    assert tiny.tolist() == [float(torch.tensor(1e-8, dtype=torch.bfloat16).float() + 1.0)]
