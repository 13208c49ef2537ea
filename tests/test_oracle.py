"""Pins for the CPU oracle (CPU only).

Each oracle function is checked against something that does not share its code: a torch library
routine evaluated in fp64, a closed form, an invariant, or brute-force Python loops on tiny inputs,
chosen so that a plausible slip (dropped eps, wrong normaliser, flipped rotate-half sign, transposed
operand, missing causal mask, missing scale) fails.  The second half plants such slips in copies of
the oracle and asserts the pins catch them, and the last test checks the committed golden vectors
(tests/golden/golden.safetensors, written by tests/golden/make_golden.py from independent fp64
computations) against the oracle.
"""
import math
from pathlib import Path

import pytest
import torch
import torch.nn.functional as F

import oracle
from oracle import kernels as K

GOLDEN = Path(__file__).resolve().parent / "golden" / "golden.safetensors"


def rnd(shape, seed, dtype=torch.bfloat16, std=1.0, mean=0.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * std + mean).to(dtype)


def bits_frac(a, b):
    return float((a.contiguous().view(torch.int16) == b.contiguous().view(torch.int16)).float().mean())


# ------------------------------------------------------------------ independent references
def ref_rmsnorm(x, w, eps):
    return F.rms_norm(x.double(), (x.shape[-1],), w.double(), eps)


def ref_softmax(x):
    return torch.softmax(x.double(), dim=-1)


def ref_silu_mul(gu):
    i = gu.shape[-1] // 2
    return F.silu(gu[..., :i].double()) * gu[..., i:].double()


def ref_rope(x, w, cos, sin, eps):
    """HF-style: RMSNorm per head, then q*cos + rotate_half(q)*sin, rotate_half(q) = cat(-q2, q1)."""
    n = F.rms_norm(x.double(), (x.shape[-1],), w.double(), eps)
    half = x.shape[-1] // 2
    q1, q2 = n[..., :half], n[..., half:]
    rot = torch.cat([-q2, q1], dim=-1)
    out = n * cos.double()[:, None, :] + rot * sin.double()[:, None, :]
    return out.permute(1, 0, 2)


def ref_attention(q, k, v, hq, hkv, causal, scale):
    g = hq // hkv
    kk = k.double().repeat_interleave(g, dim=0)
    vv = v.double().repeat_interleave(g, dim=0)
    return F.scaled_dot_product_attention(q.double(), kk, vv, is_causal=causal, scale=scale)


def brute_gemm(a, b):
    m, kk = a.shape
    n = b.shape[1]
    return [[math.fsum(float(a[i, t]) * float(b[t, j]) for t in range(kk)) for j in range(n)] for i in range(m)]


def e4m3_values():
    """All finite OCP e4m3fn values, from the format's definition (bias 7, 3 mantissa bits, no inf,
    S.1111.111 is NaN)."""
    vals = []
    for e in range(16):
        for m in range(8):
            if e == 15 and m == 7:
                continue
            v = (m / 8.0) * 2.0 ** -6 if e == 0 else (1 + m / 8.0) * 2.0 ** (e - 7)
            vals += [v, -v]
    return sorted(set(vals))


def brute_e4m3(x: float) -> float:
    """Round-to-nearest-even onto the e4m3fn grid; beyond the midpoint past 448 -> NaN (torch's cast)."""
    if math.isnan(x):
        return math.nan
    if abs(x) > 464.0:
        return math.nan
    grid = e4m3_values()
    best = min(grid, key=lambda v: (abs(v - x), 0))
    ties = [v for v in grid if abs(v - x) == abs(best - x)]
    if len(ties) > 1:   # tie: even mantissa
        def mant(v):
            a = abs(v)
            if a < 2 ** -6:
                return round(a / 2 ** -9)
            e = math.floor(math.log2(a))
            return round((a / 2 ** e - 1) * 8)
        best = [v for v in ties if mant(v) % 2 == 0][0]
    return best


# ------------------------------------------------------------------ pins
def test_rmsnorm_matches_library_fp64():
    x, w = rnd((64, 4096), 0), rnd((4096,), 1, torch.float32, 0.02, 1.0)
    got = oracle.rmsnorm(x, w, 1e-6)
    want = ref_rmsnorm(x, w, 1e-6).to(torch.bfloat16)
    assert bits_frac(got, want) > 0.999
    assert torch.allclose(got.float(), want.float(), rtol=8e-3, atol=0)


def test_rmsnorm_constant_rows_closed_form():
    """w = 1 and a constant row c: y = c / sqrt(c^2 + eps)."""
    c = torch.tensor([0.5, -2.0, 1e-3]).to(torch.bfloat16)
    x = c[:, None].repeat(1, 256)
    y = oracle.rmsnorm(x, torch.ones(256), 1e-6).float()
    cf = c.double()
    want = (cf / torch.sqrt(cf * cf + 1e-6)).float()
    assert torch.allclose(y[:, 0], want, rtol=4e-3)
    assert (y == y[:, :1]).all()


def test_rmsnorm_brute_force_tiny():
    x, w = rnd((3, 8), 2), rnd((8,), 3)
    got = oracle.rmsnorm(x, w, 1e-6).float()
    for i in range(3):
        ms = math.fsum(float(v) ** 2 for v in x[i]) / 8
        r = 1 / math.sqrt(ms + 1e-6)
        for j in range(8):
            want = torch.tensor(float(x[i, j]) * r * float(w[j])).to(torch.bfloat16).float()
            assert abs(float(got[i, j]) - float(want)) <= abs(float(want)) * 2 ** -8


def test_softmax_matches_library_and_invariants():
    x = rnd((33, 384), 4)
    got = oracle.softmax_rows(x)
    want = ref_softmax(x).to(torch.bfloat16)
    assert bits_frac(got, want) > 0.995
    assert torch.allclose(got.float().sum(-1), torch.ones(33), atol=2e-2)   # rows sum to 1 (bf16)
    shifted = oracle.softmax_rows((x.float() + 3.0).to(torch.bfloat16))
    assert torch.allclose(shifted.float(), got.float(), rtol=2e-2, atol=1e-3)
    xn = x.clone()
    xn[0, 5] = float("nan")
    assert torch.isnan(oracle.softmax_rows(xn)[0]).all()


def test_softmax_fp32_out_is_the_unrounded_library_softmax():
    """The router's fp32-out softmax: within fp32 rounding of the fp64 softmax, rows sum to 1 within
    fp32 error, and rounding it to bf16 gives the bf16-out oracle (one rounding, nothing else)."""
    x = rnd((7, 128), 40)
    got = oracle.softmax_rows(x, torch.float32)
    assert got.dtype == torch.float32
    want = torch.softmax(x.double(), dim=-1)
    assert torch.allclose(got.double(), want, rtol=1e-6, atol=1e-9)
    assert torch.allclose(got.double().sum(-1), torch.ones(7, dtype=torch.float64), atol=1e-6)
    assert torch.equal(got.to(torch.bfloat16), oracle.softmax_rows(x))


def test_silu_mul_matches_library():
    gu = rnd((17, 2 * 1032), 5)
    got = oracle.silu_mul(gu)
    assert bits_frac(got, ref_silu_mul(gu).to(torch.bfloat16)) > 0.995


def test_transpose_brute_force():
    x = rnd((3, 5, 4), 6)
    y = oracle.transpose_heads(x)
    for a in range(3):
        for b in range(5):
            assert torch.equal(y[b, a], x[a, b])


def test_qk_norm_rope_matches_hf_restatement():
    x, w = rnd((64, 4, 128), 7), rnd((128,), 8)
    cos, sin = oracle.rope_tables(64, 128, 1.0e6)
    got = oracle.qk_norm_rope(x, w, cos, sin, 1e-6)
    want = ref_rope(x, w, cos, sin, 1e-6).to(torch.bfloat16)
    assert got.shape == (4, 64, 128)
    assert bits_frac(got, want) > 0.99
    # cos = 1, sin = 0 reduces to the per-head RMSNorm, head-major
    ones, zeros = torch.ones(64, 128), torch.zeros(64, 128)
    plain = oracle.qk_norm_rope(x, w, ones, zeros, 1e-6)
    assert torch.equal(plain, oracle.rmsnorm(x.reshape(-1, 128), w, 1e-6).view(64, 4, 128).permute(1, 0, 2))


def test_rope_tables_closed_form():
    cos, sin = oracle.rope_tables(5, 8, 10000.0)
    assert torch.allclose(cos[3, 1].double(), torch.tensor(math.cos(3 / 10000 ** (2 / 8))).double(), atol=1e-7)
    assert torch.equal(cos[:, :4], cos[:, 4:]) and torch.equal(sin[0], torch.zeros(8))


def test_reductions():
    x = rnd((10007,), 9)
    assert float(oracle.reduce_sum(x)) == pytest.approx(math.fsum(float(v) for v in x), rel=1e-7, abs=1e-6)
    assert float(oracle.reduce_max(x)) == max(float(v) for v in x)
    xn = x.clone()
    xn[77] = float("nan")
    assert math.isnan(float(oracle.reduce_max(xn)))
    assert torch.equal(oracle.add_scalar(x, 1.0), (x.double() + 1).to(torch.bfloat16))


def test_gemm_brute_force_and_residual():
    a, b, r = rnd((3, 16), 10), rnd((16, 5), 11), rnd((3, 5), 12)
    got = oracle.gemm(a, b).float()
    bf = brute_gemm(a, b)
    for i in range(3):
        for j in range(5):
            want = torch.tensor(bf[i][j]).to(torch.bfloat16).float()
            assert float(got[i, j]) == float(want)
    got_r = oracle.gemm(a, b, r).float()
    for i in range(3):
        for j in range(5):
            want = torch.tensor(float(torch.tensor(bf[i][j], dtype=torch.float32)) + float(r[i, j])).to(torch.bfloat16)
            assert float(got_r[i, j]) == float(want)
    # not symmetric in its operands: a transposed B would not even have the right shape here
    assert oracle.gemm(a, b).shape == (3, 5)


def test_e4m3_cast_exhaustive_and_quantisers():
    grid = e4m3_values()
    t = torch.tensor(grid)
    assert torch.equal(t.to(torch.float8_e4m3fn).float(), t)                  # every code round-trips
    probe = [0.3, 1.0625, 1.1875, 447.0, 448.0, 460.0, 464.0, -0.0017, 2 ** -10, 3 * 2 ** -10, 1e-9]
    for v in probe:
        want = brute_e4m3(v)
        gotv = float(torch.tensor(v).to(torch.float8_e4m3fn).float())
        assert (math.isnan(want) and math.isnan(gotv)) or gotv == want, (v, gotv, want)
    assert math.isnan(float(torch.tensor(470.0).to(torch.float8_e4m3fn).float()))
    x = rnd((4, 64), 13)
    x[2] = 0
    xq, sc = oracle.quant_rows_e4m3(x)
    assert sc[2] == 1.0 and torch.all(xq[2].float() == 0)
    amax = x.float().abs().amax(-1)
    assert torch.allclose(sc[[0, 1, 3]], amax[[0, 1, 3]] / 448)
    assert float(xq.float().abs().max()) == 448.0                               # the row max lands on 448
    w = rnd((64, 8), 14, torch.float32, 0.02)
    wq, sw = oracle.quant_weight_e4m3(w)
    assert wq.shape == (8, 64) and torch.allclose(sw, w.abs().amax(0) / 448)
    assert torch.allclose(wq.float().t() * sw, w, rtol=0.07, atol=1e-4)       # dequantised ~ W


def test_gemm_fp8_brute_force():
    a, w = rnd((3, 32), 15), rnd((32, 4), 16, torch.float32, 0.02)
    aq, sa = oracle.quant_rows_e4m3(a)
    wq, sw = oracle.quant_weight_e4m3(w)
    got = oracle.gemm_fp8(aq, sa, wq, sw).float()
    for i in range(3):
        for j in range(4):
            acc = math.fsum(float(aq[i, t].float()) * float(wq[j, t].float()) for t in range(32))
            want = torch.tensor((float(torch.tensor(acc, dtype=torch.float32)) * float(sa[i])) * float(sw[j]),
                                dtype=torch.float32).to(torch.bfloat16)
            assert abs(float(got[i, j]) - float(want)) <= abs(float(want)) * 2 ** -7 + 1e-9


@pytest.mark.parametrize("hq,hkv,s,causal", [(4, 2, 256, True), (2, 2, 128, False), (3, 1, 192, True)])
def test_flash_attention_matches_sdpa(hq, hkv, s, causal):
    q, k, v = rnd((hq, s, 128), 17), rnd((hkv, s, 128), 18), rnd((hkv, s, 128), 19)
    scale = 1 / math.sqrt(128)
    got = oracle.flash_attention(q, k, v, hq, hkv, causal, scale, bq=64, bkv=64)
    want = ref_attention(q, k, v, hq, hkv, causal, scale)
    assert torch.allclose(got.float(), want.float(), rtol=2e-2, atol=2e-2)


def test_flash_attention_invariants():
    q, k, v = rnd((4, 256, 128), 20), rnd((2, 256, 128), 21), rnd((2, 256, 128), 22)
    o = oracle.flash_attention(q, k, v, 4, 2, True, 1 / math.sqrt(128), bq=128, bkv=128)
    for h in range(4):
        assert torch.equal(o[h, 0], v[h // 2, 0])                              # row 0 sees key 0 only
    vc = torch.full((2, 256, 128), 0.75).to(torch.bfloat16)
    oc = oracle.flash_attention(q, k, vc, 4, 2, True, 1 / math.sqrt(128), bq=128, bkv=128).float()
    assert (oc - 0.75).abs().max() <= 0.75 * 2 ** -7                          # V const -> O const


def test_qwen3_layer_matches_fp64_block():
    """The oracle's 14-launch composition against an fp64 Qwen3 block written from the model's
    definition (no bf16 rounding between ops); agreement within the accumulated bf16 error."""
    t, hid, hq, hkv, d, inter = 64, 256, 4, 2, 128, 384
    g = torch.Generator().manual_seed(23)

    def r(*shape, mean=0.0):
        return (torch.randn(*shape, generator=g) * 0.02 + mean).to(torch.bfloat16)

    x = rnd((t, hid), 24)
    w = {"w_in": r(hid, mean=1.0), "wq": r(hid, hq * d), "wk": r(hid, hkv * d), "wv": r(hid, hkv * d),
         "w_qn": r(d, mean=1.0), "w_kn": r(d, mean=1.0), "wo": r(hq * d, hid), "w_post": r(hid, mean=1.0),
         "wgu": r(hid, 2 * inter), "wd": r(inter, hid)}
    cos, sin = oracle.rope_tables(t, d, 1.0e6)
    got = oracle.qwen3_layer(x, w, cos, sin, hq, hkv, d, 1e-6, bq=64)
    W = {k: v.double() for k, v in w.items()}
    X = x.double()
    xn = F.rms_norm(X, (hid,), W["w_in"], 1e-6)
    q, k, v = (xn @ W["wq"]).view(t, hq, d), (xn @ W["wk"]).view(t, hkv, d), (xn @ W["wv"]).view(t, hkv, d)
    qh = ref_rope(q, w["w_qn"], cos, sin, 1e-6)
    kh = ref_rope(k, w["w_kn"], cos, sin, 1e-6)
    oh = ref_attention(qh, kh, v.permute(1, 0, 2), hq, hkv, True, 1 / math.sqrt(d))
    h = X + oh.permute(1, 0, 2).reshape(t, hq * d) @ W["wo"]
    gu = F.rms_norm(h, (hid,), W["w_post"], 1e-6) @ W["wgu"]
    y = h + (F.silu(gu[:, :inter]) * gu[:, inter:]) @ W["wd"]
    assert torch.allclose(got.double(), y, rtol=3e-2, atol=3e-2)


# ------------------------------------------------------------------ decode path pins
def test_sumsq_fsum_and_cross_terms():
    x, a = rnd((4096,), 30), rnd((4096,), 31)
    got = float(oracle.sumsq(x))
    want = math.fsum(float(v) ** 2 for v in x.float())
    assert abs(got - want) <= 1e-6 * want
    got2 = float(oracle.sumsq(x, a))
    s32 = (x.float() + a.float()).double()          # the reference adds in fp32, then squares
    want2 = math.fsum(float(v) ** 2 for v in s32)
    assert abs(got2 - want2) <= 1e-6 * want2
    no_cross = math.fsum(float(v) ** 2 for v in x.float()) + math.fsum(float(v) ** 2 for v in a.float())
    assert abs(no_cross - want2) > 1e-3 * want2      # a slip that drops the cross terms is visible


def test_gemv_variants_match_fp64():
    k, n = 512, 384
    x, a = rnd((k,), 32), rnd((k,), 33)
    g = rnd((k,), 34, std=0.02, mean=1.0)
    w = rnd((k, n), 35, std=0.05)
    tol = dict(rtol=2 ** -7, atol=1e-3)
    assert torch.allclose(oracle.gemv(x, w).double(), x.double() @ w.double(), **tol)
    ss = oracle.sumsq(x, a)
    got = oracle.gemv_rmsnorm(x, ss, g, w, add=a, eps=1e-6)
    h = (x.float() + a.float()).double()
    want = F.rms_norm(h, (k,), g.double(), 1e-6) @ w.double()
    assert torch.allclose(got.double(), want, **tol)
    plain = oracle.gemv_rmsnorm(x, oracle.sumsq(x), g, w, eps=1e-6)
    assert torch.allclose(plain.double(), F.rms_norm(x.double(), (k,), g.double(), 1e-6) @ w.double(), **tol)
    gu = rnd((2 * k,), 36)
    wd = rnd((k, n), 37, std=0.05)
    ra, rb = rnd((n,), 38), rnd((n,), 39)
    got = oracle.gemv_silu(gu, wd, ra, rb)
    gd = gu.double()
    want = (F.silu(gd[:k]) * gd[k:]) @ wd.double() + (ra.float() + rb.float()).double()
    assert torch.allclose(got.double(), want, **tol)
    # a transposed weight or a gate/up swap is caught
    xs, wsq = x[:n], w[:n, :n]
    assert not torch.allclose(oracle.gemv(xs, wsq.t().contiguous()).double(), xs.double() @ wsq.double(), **tol)
    swapped = oracle.gemv_silu(torch.cat([gu[k:], gu[:k]]), wd, ra, rb)
    assert not torch.allclose(swapped.double(), want, **tol)


@pytest.mark.parametrize("nkv,g,s", [(2, 4, 256), (3, 3, 128), (1, 8, 64)])
def test_attention_decode_matches_sdpa(nkv, g, s):
    q, k, v = rnd((nkv, g, 128), 40), rnd((nkv, s, 128), 41), rnd((nkv, s, 128), 42)
    scale = 1 / math.sqrt(128)
    got = oracle.attention_decode(q, k, v, scale)
    want = F.scaled_dot_product_attention(q.double().unsqueeze(2), k.double().unsqueeze(1).expand(nkv, g, s, 128),
                                          v.double().unsqueeze(1).expand(nkv, g, s, 128), scale=scale).squeeze(2)
    assert torch.allclose(got.double(), want, rtol=2e-2, atol=2e-2)
    blocked = oracle.attention_decode(q, k, v, scale, bkv=max(1, s // 4))   # blocking changes only roundings
    assert torch.allclose(blocked.double(), want, rtol=2e-2, atol=2e-2)


def test_attention_decode_invariants():
    q, k = rnd((2, 4, 128), 43), rnd((2, 1, 128), 44)
    v = rnd((2, 1, 128), 45)
    o = oracle.attention_decode(q, k, v)
    for h in range(2):
        for gi in range(4):
            assert torch.equal(o[h, gi], v[h, 0])                      # one key: p = 1 exactly
    kk = rnd((2, 64, 128), 46)
    vc = torch.full((2, 64, 128), -1.25).to(torch.bfloat16)
    oc = oracle.attention_decode(q, kk, vc).float()
    assert (oc + 1.25).abs().max() <= 1.25 * 2 ** -7                   # V const -> O const


def test_qwen3_decode_layer_matches_fp64_step():
    """The 8-launch decode composition against an fp64 Qwen3 decode step written from the model's
    definition over the same KV cache (no bf16 rounding between ops)."""
    hid, hq, hkv, d, inter, s = 256, 4, 2, 128, 384, 96
    g = torch.Generator().manual_seed(47)

    def r(*shape, mean=0.0, std=0.02):
        return (torch.randn(*shape, generator=g) * std + mean).to(torch.bfloat16)

    x = r(hid, std=1.0)
    w = {"w_in": r(hid, mean=1.0), "wq": r(hid, hq * d), "w_qn": r(d, mean=1.0), "wo": r(hq * d, hid),
         "w_post": r(hid, mean=1.0), "wgu": r(hid, 2 * inter), "wd": r(inter, hid)}
    kc, vc = r(hkv, s, d, std=1.0), r(hkv, s, d, std=1.0)
    cos_t, sin_t = oracle.rope_tables(s + 1, d, 1.0e6)
    cos, sin = cos_t[s], sin_t[s]                 # the new token's position
    got = oracle.qwen3_decode_layer(x, w, kc, vc, cos, sin, hq, hkv, d, 1e-6)
    W = {k: v.double() for k, v in w.items()}
    X = x.double()
    q = (F.rms_norm(X, (hid,), W["w_in"], 1e-6) @ W["wq"]).view(1, hq, d)
    qh = ref_rope(q, w["w_qn"], cos[None], sin[None], 1e-6).reshape(hkv, hq // hkv, 1, d)
    o = F.scaled_dot_product_attention(qh, kc.double().unsqueeze(1).expand(hkv, hq // hkv, s, d),
                                       vc.double().unsqueeze(1).expand(hkv, hq // hkv, s, d), scale=1 / math.sqrt(d))
    h = X + o.reshape(hq * d) @ W["wo"]
    gu = F.rms_norm(h, (hid,), W["w_post"], 1e-6) @ W["wgu"]
    y = h + (F.silu(gu[:inter]) * gu[inter:]) @ W["wd"]
    assert torch.allclose(got.double(), y, rtol=3e-2, atol=3e-2)


# ------------------------------------------------------------------ planted slips are caught
def test_pins_catch_planted_slips(monkeypatch):
    x, w = rnd((64, 4096), 0), rnd((4096,), 1, torch.float32, 0.02, 1.0)

    def rms_no_eps(x, w, eps=1e-6):
        xf = x.float()
        return ((xf * torch.rsqrt((xf * xf).sum(-1, keepdim=True) / (x.shape[-1] - 1))) * w.float()).to(torch.bfloat16)

    # the rmsnorm pin demands > 99.9% bit-identical outputs; a 1/4096 normaliser slip already fails it
    assert bits_frac(rms_no_eps(x, w), ref_rmsnorm(x, w, 1e-6).to(torch.bfloat16)) < 0.999

    xr, wr = rnd((64, 4, 128), 7), rnd((128,), 8)
    cos, sin = oracle.rope_tables(64, 128, 1.0e6)

    def rope_flipped(x, w, cos, sin, eps=1e-6):
        t, h, d = x.shape
        xf = x.float()
        a = (xf * torch.rsqrt((xf * xf).sum(-1, keepdim=True) / d + eps)) * w.float()
        rot = torch.cat([a[..., d // 2:], -a[..., : d // 2]], dim=-1)   # sign on the wrong half
        return (a * cos[:, None] + rot * sin[:, None]).to(torch.bfloat16).permute(1, 0, 2)

    assert bits_frac(rope_flipped(xr, wr, cos, sin), ref_rope(xr, wr, cos, sin, 1e-6).to(torch.bfloat16)) < 0.9

    a, b = rnd((16, 16), 10), rnd((16, 16), 11)
    assert not torch.equal(K.gemm(a, b.t().contiguous()), K.gemm(a, b))

    q, k, v = rnd((2, 128, 128), 17), rnd((1, 128, 128), 18), rnd((1, 128, 128), 19)
    good = ref_attention(q, k, v, 2, 1, True, 1 / math.sqrt(128))
    no_mask = oracle.flash_attention(q, k, v, 2, 1, False, 1 / math.sqrt(128), bq=64, bkv=64)
    no_scale = oracle.flash_attention(q, k, v, 2, 1, True, 1.0, bq=64, bkv=64)
    assert not torch.allclose(no_mask.float(), good.float(), rtol=2e-2, atol=2e-2)
    assert not torch.allclose(no_scale.float(), good.float(), rtol=2e-2, atol=2e-2)


# ------------------------------------------------------------------ golden vectors
def test_golden_vectors():
    from safetensors.torch import load_file

    gv = load_file(str(GOLDEN))
    assert torch.equal(oracle.rmsnorm(gv["rmsnorm.x"], gv["rmsnorm.w"], 1e-6), gv["rmsnorm.y"])
    assert torch.equal(oracle.softmax_rows(gv["softmax.x"]), gv["softmax.y"])
    assert torch.equal(oracle.silu_mul(gv["silu.gu"]), gv["silu.y"])
    assert torch.equal(oracle.qk_norm_rope(gv["rope.x"], gv["rope.w"], gv["rope.cos"], gv["rope.sin"], 1e-6),
                       gv["rope.y"])
    assert torch.equal(oracle.gemm(gv["gemm.a"], gv["gemm.b"], gv["gemm.r"]), gv["gemm.c"])
    xq, sx = oracle.quant_rows_e4m3(gv["fp8.x"])
    assert torch.equal(xq.view(torch.uint8), gv["fp8.xq"]) and torch.equal(sx, gv["fp8.sx"])
    assert torch.equal(oracle.flash_attention(gv["attn.q"], gv["attn.k"], gv["attn.v"], 4, 2, True,
                                              1 / math.sqrt(128), bq=128, bkv=128), gv["attn.o"])
    # the independent fp64 references the fixtures were made from agree with the oracle too
    assert bits_frac(gv["rmsnorm.y"], gv["rmsnorm.y64"]) > 0.999
    assert torch.allclose(gv["attn.o"].float(), gv["attn.o64"].float(), rtol=2e-2, atol=2e-2)


# ------------------------------------------------------------------ fp32 vector ops
def test_rmsnorm_f32_matches_library_and_brute_force():
    """The fp32 row arm against torch's rms_norm in fp64 (relative 1e-6: fp32 rounding only) and a
    brute-force fsum loop; a normaliser off by one (dividing by N - 1) fails the fp64 pin."""
    x = rnd((16, 64), 60, torch.float32)
    w = rnd((64,), 61, torch.float32)
    got = oracle.rmsnorm_f32(x, w, 1e-5)
    assert got.dtype == torch.float32
    want = torch.nn.functional.rms_norm(x.double(), (64,), w.double(), 1e-5)
    assert torch.allclose(got.double(), want, rtol=1e-6, atol=1e-7)
    for i in range(3):
        r = 1 / math.sqrt(math.fsum(float(v) ** 2 for v in x[i]) / 64 + 1e-5)
        for j in range(0, 64, 7):
            assert abs(float(got[i, j]) - float(x[i, j]) * r * float(w[j])) <= 1e-6 * (abs(float(got[i, j])) + 1e-6)
    off = (x.double() * torch.rsqrt((x.double() ** 2).sum(-1, keepdim=True) / 63 + 1e-5)) * w.double()
    assert not torch.allclose(got.double(), off, rtol=1e-5, atol=1e-6)


def test_col_rms_f32_closed_form():
    """Column arm: a matrix whose column j is constant c_j gives 1/sqrt(c_j^2 + eps); random input
    against the fp64 formula; a transposed reduction (over columns) fails it."""
    c = torch.tensor([0.5, -2.0, 3.0, 1e-3])
    x = c[None, :].repeat(8, 1)
    got = oracle.col_rms_f32(x, 1e-5)
    assert torch.allclose(got.double(), 1 / torch.sqrt(c.double() ** 2 + 1e-5), rtol=1e-6)
    y = rnd((8, 64), 62, torch.float32)
    want = torch.rsqrt((y.double() ** 2).mean(0) + 1e-5)
    assert torch.allclose(oracle.col_rms_f32(y, 1e-5).double(), want, rtol=1e-6)
    wrong = torch.rsqrt((y.double() ** 2).mean(1) + 1e-5)
    assert wrong.shape != want.shape or not torch.allclose(wrong, want, rtol=1e-3)


def test_softmax_f32_input_matches_library():
    x = rnd((256, 64), 63, torch.float32)
    got = oracle.softmax_rows(x, torch.float32)
    assert torch.allclose(got.double(), torch.softmax(x.double(), -1), rtol=1e-6, atol=1e-9)


def test_silu_mul_f32_and_swiglu_f32_match_library():
    """silu(g) * u in fp32 against F.silu in fp64; the SwiGLU block against fp64 matmuls; swapping
    the gate and up weights (a plausible slip) fails the pin."""
    gu = rnd((9, 2 * 40), 64, torch.float32)
    got = oracle.silu_mul_f32(gu)
    g, u = gu[:, :40].double(), gu[:, 40:].double()
    assert torch.allclose(got.double(), torch.nn.functional.silu(g) * u, rtol=1e-6, atol=1e-7)
    x = rnd((32, 48), 65, torch.float32, 0.1)
    wg, wu = rnd((48, 24), 66, torch.float32, 0.1), rnd((48, 24), 67, torch.float32, 0.1)
    want = torch.nn.functional.silu(x.double() @ wg.double()) * (x.double() @ wu.double())
    o = oracle.swiglu_f32(x, wg, wu)
    assert torch.allclose(o.double(), want, rtol=1e-5, atol=1e-7)
    swapped = torch.nn.functional.silu(x.double() @ wu.double()) * (x.double() @ wg.double())
    assert not torch.allclose(o.double(), swapped, rtol=1e-3, atol=1e-3)
