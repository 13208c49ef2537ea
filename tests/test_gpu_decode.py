"""Parity of the single-token (decode) kernels with the oracle's restatements of
qwen3_8b_layer_decode_1x<S>_bf16/{00..07} and attention_decode_<HQ>x8x<S>_bf16/00__decode_kernel.
bf16 outputs: rtol 2e-2 with the absolute floor at 2e-2 of the output's mean magnitude (the GEMV
outputs are not O(1)); fp32 sums within 1e-6 of the sum of |terms|; exact invariants bit for bit."""
import math

import pytest
import torch

import oracle
from helpers import assert_close, bits_equal, randn
from ptb_amd import _lib, ops

pytestmark = pytest.mark.gpu

DEV = "cuda"
RTOL = 2e-2


def close_scaled(got, want, what):
    scale = float(want.float().abs().mean()) + 1e-6
    assert_close(got, want, RTOL, 2e-2 * max(scale, 1e-3), what)


@pytest.mark.parametrize("n,seed", [(4096, 0), (12288, 1), (4100, 2), (8, 3), (3, 4)])
def test_sumsq(n, seed):
    x, a = randn((n,), seed), randn((n,), seed + 100)
    for y in (None, a):
        got = ops.sumsq(x.to(DEV), None if y is None else y.to(DEV)).cpu()
        want = oracle.sumsq(x, y)
        terms = (x.float() + (0 if y is None else y.float())).double().pow(2).sum()
        assert abs(float(got) - float(want)) <= 1e-6 * float(terms) + 1e-6


@pytest.mark.parametrize("k,n", [(4096, 4096), (4096, 24576), (12288, 4096), (100, 8), (1000, 520), (33, 16)])
def test_gemv_plain_and_rmsnorm(k, n):
    x, a = randn((k,), 5), randn((k,), 6)
    g = randn((k,), 7, std=0.02, mean=1.0)
    w = randn((k, n), 8, std=0.02)
    xd, ad, gd, wd = x.to(DEV), a.to(DEV), g.to(DEV), w.to(DEV)
    close_scaled(ops.gemv(xd, wd).cpu(), oracle.gemv(x, w), f"gemv {k}x{n}")
    ss = oracle.sumsq(x, a)
    got = ops.gemv_rmsnorm(xd, ss.to(DEV), gd, wd, add=ad, eps=1e-6).cpu()
    close_scaled(got, oracle.gemv_rmsnorm(x, ss, g, w, add=a, eps=1e-6), f"gemv_rmsnorm+add {k}x{n}")
    ss1 = oracle.sumsq(x)
    got = ops.gemv_rmsnorm(xd, ss1.to(DEV), gd, wd, eps=1e-6).cpu()
    close_scaled(got, oracle.gemv_rmsnorm(x, ss1, g, w, eps=1e-6), f"gemv_rmsnorm {k}x{n}")
    # no sum of squares passed: the workgroups form it themselves (with and without the add)
    got = ops.gemv_rmsnorm(xd, None, gd, wd, add=ad, eps=1e-6).cpu()
    close_scaled(got, oracle.gemv_rmsnorm(x, ss, g, w, add=a, eps=1e-6), f"gemv_rmsnorm own ss+add {k}x{n}")
    got = ops.gemv_rmsnorm(xd, None, gd, wd, eps=1e-6).cpu()
    close_scaled(got, oracle.gemv_rmsnorm(x, ss1, g, w, eps=1e-6), f"gemv_rmsnorm own ss {k}x{n}")


@pytest.mark.parametrize("k,n", [(12288, 4096), (64, 8), (777, 264)])
def test_gemv_silu_with_residual(k, n):
    gu = randn((2 * k,), 9)
    w = randn((k, n), 10, std=0.02)
    ra, rb = randn((n,), 11), randn((n,), 12)
    gud, wd = gu.to(DEV), w.to(DEV)
    got = ops.gemv_silu(gud, wd, ra.to(DEV), rb.to(DEV)).cpu()
    close_scaled(got, oracle.gemv_silu(gu, w, ra, rb), f"gemv_silu {k}x{n}")
    got = ops.gemv_silu(gud, wd).cpu()
    close_scaled(got, oracle.gemv_silu(gu, w), f"gemv_silu no residual {k}x{n}")


@pytest.mark.parametrize("gk,k,n", [(4096, 12288, 4096), (1000, 260, 264)])
def test_gemv_silu_parts_is_the_two_launches(gk, k, n):
    """The gate/up GEMV's partial pass, then the down GEMV finishing those partials in its prologue,
    gives the bits of gemv_rmsnorm followed by gemv_silu (the decode layer's K06 + K07), with and
    without the residuals."""
    x, a = randn((gk,), 50), randn((gk,), 51)
    g = randn((gk,), 52, std=0.02, mean=1.0)
    wgu, wd = randn((gk, 2 * k), 53, std=0.02), randn((k, n), 54, std=0.02)
    ra, rb = randn((n,), 55), randn((n,), 56)
    xd, ad, gd, wgud, wdd, rad, rbd = (t.to(DEV) for t in (x, a, g, wgu, wd, ra, rb))
    gu = ops.gemv_rmsnorm(xd, None, gd, wgud, add=ad, eps=1e-6)
    parts = ops.gemv_rmsnorm_parts(xd, None, gd, wgud, add=ad, eps=1e-6)
    for r1, r2 in ((rad, rbd), (None, None)):
        want = ops.gemv_silu(gu, wdd, r1, r2).cpu()
        got = ops.gemv_silu_parts(parts, gk, wdd, r1, r2).cpu()
        assert bits_equal(got, want), f"gemv_silu_parts {gk}x{k}x{n} residual={r1 is not None}"
    close_scaled(got, oracle.gemv_silu(oracle.gemv_rmsnorm(x, oracle.sumsq(x, a), g, wgu, add=a, eps=1e-6), w=wd),
                 f"gemv_silu_parts vs oracle {gk}x{k}x{n}")


def test_gemv_exact_small_integers():
    """Small-integer operands: every product and partial sum is exact in fp32, so the split-K order
    cannot matter and the result is bit-exact."""
    g = torch.Generator().manual_seed(13)
    x = torch.randint(-4, 5, (1024,), generator=g).to(torch.bfloat16)
    w = torch.randint(-4, 5, (1024, 512), generator=g).to(torch.bfloat16)
    got = ops.gemv(x.to(DEV), w.to(DEV)).cpu()
    assert bits_equal(got, oracle.gemv(x, w))


@pytest.mark.parametrize("hq,s", [(32, 4096), (16, 128), (24, 1024), (64, 8192), (32, 2048), (8, 256)])
def test_attention_decode_bundle_shapes(hq, s):
    hkv = 8
    g = hq // hkv
    q, k, v = randn((hkv, g, 128), 14), randn((hkv, s, 128), 15), randn((hkv, s, 128), 16)
    got = ops.attention_decode(q.to(DEV), k.to(DEV), v.to(DEV), 1 / math.sqrt(128)).cpu()
    want = oracle.attention_decode(q, k, v, 1 / math.sqrt(128))
    assert_close(got, want, RTOL, 2e-2, f"decode {hq}x{hkv}x{s}")


@pytest.mark.parametrize("nkv,g,s", [(3, 6, 200), (2, 1, 130), (1, 3, 1), (4, 2, 127)])
def test_attention_decode_ragged(nkv, g, s):
    q, k, v = randn((nkv, g, 128), 17), randn((nkv, s, 128), 18), randn((nkv, s, 128), 19)
    got = ops.attention_decode(q.to(DEV), k.to(DEV), v.to(DEV)).cpu()
    assert_close(got, oracle.attention_decode(q, k, v), RTOL, 2e-2, f"decode ragged {nkv}x{g}x{s}")
    if s == 1:   # one key: p = 1, so O = V[0] bit for bit
        for h in range(nkv):
            for gi in range(g):
                assert bits_equal(got[h, gi], v[h, 0])


@pytest.mark.parametrize("nkv,g,s", [(2, 1, 20000), (1, 8, 20000), (1, 4, 16384), (2, 8, 64), (5, 3, 256),
                                     (3, 8, 100), (3, 8, 250), (257, 1, 300), (2, 8, 9000), (2, 6, 3000),
                                     (300, 8, 40), (4, 2, 257), (1, 2, 40000), (1, 8, 131072)])
def test_attention_decode_range_plans(nkv, g, s):
    """Caches past 256 keys (the matrix-core form, 32-key steps, ceil(n/48) steps a range below 256
    steps, ceil(n/64) from there): ten steps a range (20000 keys: pairs of steps, the last range
    ending in a step past S), eight (16384), five (9000: pairs, then a single step), twenty (40000),
    sixty-four (131072 keys, 64 ranges),
    two (3000), one (300, and 257 keys, whose last range holds one key); caches of at most 256 keys
    (one pass of the VALU form, a workgroup per query row): one team (64 and 40 keys), two (100)
    and four (250 and 256 keys), and 2400 row workgroups (300 heads x 8); G = 1, 2, 3, 4, 6 and 8."""
    q, k, v = randn((nkv, g, 128), 20), randn((nkv, s, 128), 21), randn((nkv, s, 128), 22)
    got = ops.attention_decode(q.to(DEV), k.to(DEV), v.to(DEV)).cpu()
    assert_close(got, oracle.attention_decode(q, k, v), RTOL, 2e-2, f"decode plan {nkv}x{g}x{s}")


@pytest.mark.parametrize("nkv,g,s", [(8, 4, 1024), (8, 4, 4096), (2, 8, 9000), (3, 1, 100), (1, 3, 20000),
                                     (4, 6, 600), (2, 2, 300)])
def test_attention_decode_fused_qnorm_rope(nkv, g, s):
    """q-norm + RoPE in the attention prologue gives the same bits as qk_norm_rope followed by
    attention_decode (both round the rotated q to bf16 with the same fp32 arithmetic), over the
    one-pass, team and range plans; and it matches the oracle's pair."""
    qraw = randn((nkv * g, 128), 40)
    w = randn((128,), 41, std=0.1, mean=1.0)
    cos_t, sin_t = oracle.rope_tables(s + 1, 128, 1.0e6)
    cos, sin = cos_t[s], sin_t[s]
    k, v = randn((nkv, s, 128), 42), randn((nkv, s, 128), 43)
    qd, wd, cd, sd, kd, vd = (t.to(DEV) for t in (qraw, w, cos, sin, k, v))
    qh = ops.qk_norm_rope(qd.view(1, nkv * g, 128), wd, cd.view(1, 128), sd.view(1, 128), 1e-6)
    pair = ops.attention_decode(qh.view(nkv, g, 128), kd, vd).cpu()
    fused = ops.attention_decode(qd.view(nkv, g, 128), kd, vd, qnorm=(wd, cd, sd, 1e-6)).cpu()
    assert bits_equal(fused, pair), f"fused q-norm differs from the pair {nkv}x{g}x{s}"
    qo = oracle.qk_norm_rope(qraw.view(1, nkv * g, 128), w, cos.view(1, 128), sin.view(1, 128), 1e-6)
    want = oracle.attention_decode(qo.view(nkv, g, 128), k, v)
    assert_close(fused, want, RTOL, 2e-2, f"fused decode vs oracle {nkv}x{g}x{s}")


def test_attention_decode_workspace_reuse():
    """One caller workspace serves consecutive calls of different shapes (each call's records
    replace the last call's)."""
    shapes = ((8, 4, 4096, 30), (3, 2, 1000, 33), (8, 4, 4096, 36), (8, 4, 1500, 39))
    need = max(_lib.load().ptb_attn_decode_workspace_bytes(nkv, g, s) for nkv, g, s, _ in shapes)
    assert need > 0
    ws = torch.empty(need, dtype=torch.uint8, device=DEV)
    for nkv, g, s, seed in shapes:
        q, k, v = randn((nkv, g, 128), seed), randn((nkv, s, 128), seed + 1), randn((nkv, s, 128), seed + 2)
        got = ops.attention_decode(q.to(DEV), k.to(DEV), v.to(DEV), workspace=ws).cpu()
        assert_close(got, oracle.attention_decode(q, k, v), RTOL, 2e-2, f"decode reuse {nkv}x{g}x{s}")


def test_decode_refusals():
    q = torch.zeros((2, 5, 128), dtype=torch.bfloat16, device=DEV)
    k = torch.zeros((2, 64, 128), dtype=torch.bfloat16, device=DEV)
    with pytest.raises(_lib.UnsupportedError):
        ops.attention_decode(q, k, k)                                   # group 5 is not built
    q4 = torch.zeros((2, 4, 128), dtype=torch.bfloat16, device=DEV)
    k4 = torch.zeros((2, 4096, 128), dtype=torch.bfloat16, device=DEV)   # several key ranges a head
    small = torch.empty(16, dtype=torch.uint8, device=DEV)
    with pytest.raises(_lib.PtbError) as e:
        ops.attention_decode(q4, k4, k4, workspace=small)
    assert e.value.status == _lib.PTB_ERR_WORKSPACE
    x = torch.zeros(64, dtype=torch.bfloat16, device=DEV)
    w = torch.zeros((64, 12), dtype=torch.bfloat16, device=DEV)
    with pytest.raises(_lib.UnsupportedError):
        ops.gemv(x, w)                                                  # n % 8 != 0


def test_qwen3_decode_layer_matches_oracle():
    """The 8 decode launches at Qwen3-8B's full dimensions over a 1024-token cache."""
    from ptb_amd import qwen3

    s = 1024
    wts = qwen3.random_weights(seed=3)
    g = torch.Generator().manual_seed(4)
    x = torch.randn(4096, generator=g).to(torch.bfloat16)
    kc = torch.randn(8, s, 128, generator=g).to(torch.bfloat16)
    vc = torch.randn(8, s, 128, generator=g).to(torch.bfloat16)
    cos_t, sin_t = oracle.rope_tables(s + 1, 128, 1.0e6)
    cos, sin = cos_t[s], sin_t[s]
    layer = qwen3.Qwen3DecodeLayer({k: v.to(DEV) for k, v in wts.items()})
    y = layer(x.to(DEV), kc.to(DEV), vc.to(DEV), cos.to(DEV), sin.to(DEV)).cpu()
    want = oracle.qwen3_decode_layer(x, wts, kc, vc, cos, sin)
    rms = float(want.float().pow(2).mean().sqrt())
    assert_close(y, want, RTOL, 2e-2 * max(1.0, rms), "qwen3 decode layer")


@pytest.mark.parametrize("s", [256, 4096])
def test_decode_layer_graph_replays_match_eager(s):
    """The decode layer (GEMVs with their workspaces, decode attention with its q-norm + RoPE
    prologue and merge pass) captured as a HIP graph: each of several replays, with eager work and
    synchronisations between them, reproduces the eager forward bit for bit (the bench times the
    decode lines this way; no step of the layer records a memset node)."""
    from ptb_amd import qwen3

    layer = qwen3.Qwen3DecodeLayer({k: v.to(DEV) for k, v in qwen3.random_weights(seed=3).items()})
    x = randn((4096,), 30).to(DEV)
    kc = randn((8, s, 128), 31).to(DEV)
    vc = randn((8, s, 128), 32).to(DEV)
    cos_t, sin_t = qwen3.rope_tables(s + 1, 128, 1.0e6, DEV)
    cos, sin = cos_t[s].contiguous(), sin_t[s].contiguous()
    y = torch.empty(4096, dtype=torch.bfloat16, device=DEV)
    want = layer.forward(x, kc, vc, cos, sin).clone()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side), torch.cuda.graph(g, stream=side):
        layer.forward(x, kc, vc, cos, sin, out=y)
    torch.cuda.current_stream().wait_stream(side)
    for i in range(3):
        y.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert bits_equal(y, want), f"replay {i}"
        assert bits_equal(layer.forward(x, kc, vc, cos, sin), want)   # eager work between replays
