"""The Qwen3-8B layer composed from the HIP kernels against the oracle's composition of the same
14 launches (bf16 tolerance rtol = 2e-2, absolute floor 2e-2 times the output's RMS), at T = 256
and at the full T = 2048, and the full-size layer against a chain of the individually
parity-tested GPU ops (bit for bit)."""
import pytest
import torch

import oracle
from helpers import assert_close, bits_equal, randn
from ptb_amd import ops, qwen3

pytestmark = pytest.mark.gpu

DEV = "cuda"


def test_layer_matches_oracle_small():
    cfg = qwen3.QWEN3_8B
    t = 256
    w = qwen3.random_weights(cfg, seed=0)
    x = randn((t, cfg.hidden), 1)
    layer = qwen3.Qwen3Layer({k: v.to(DEV) for k, v in w.items()}, cfg)
    y = layer(x.to(DEV)).cpu()
    cos, sin = oracle.rope_tables(t, cfg.head_dim, cfg.rope_theta)
    cq, sq = qwen3.rope_tables(t, cfg.head_dim, cfg.rope_theta)
    assert torch.equal(cos, cq) and torch.equal(sin, sq)
    want = oracle.qwen3_layer(x, w, cos, sin, cfg.heads, cfg.kv_heads, cfg.head_dim, cfg.eps)
    # 14 launches, each rounding to bf16 in a different summation order than the oracle: the
    # bf16 bound 2e-2, with the absolute floor scaled to the output's RMS (y = h + mlp is not unit)
    rms = float(want.float().pow(2).mean().sqrt())
    assert_close(y, want, 2e-2, 2e-2 * max(1.0, rms), "qwen3 layer T=256")


def test_layer_full_size_matches_oracle():
    """T = S = 2048 at full size against the oracle's composition of the
    manifest's 14 launches (validation/pytorchsim/qwen3_8b_layer_prefill_2048x2048_bf16/
    manifest.json) on the same weights and input, under the T = 256 test's bound."""
    cfg = qwen3.QWEN3_8B
    t = 2048
    w = qwen3.random_weights(cfg, seed=0)
    x = randn((t, cfg.hidden), 3)
    layer = qwen3.Qwen3Layer({k: v.to(DEV) for k, v in w.items()}, cfg)
    y = layer(x.to(DEV)).cpu()
    cos, sin = oracle.rope_tables(t, cfg.head_dim, cfg.rope_theta)
    want = oracle.qwen3_layer(x, w, cos, sin, cfg.heads, cfg.kv_heads, cfg.head_dim, cfg.eps)
    rms = float(want.float().pow(2).mean().sqrt())
    assert torch.isfinite(y.float()).all()
    assert_close(y, want, 2e-2, 2e-2 * max(1.0, rms), "qwen3 layer T=2048")


def test_layer_full_size_is_its_launch_chain():
    """T = S = 2048: the layer's forward is exactly the 14-launch chain, so
    re-running the chain op by op gives bit-identical output (deterministic kernels).  The forward's
    fused q|k|v GEMM (256x256 tiles) and its strided norm / transpose reads give the bits of the
    separate q, k, v products (other tile shapes): every tile issues the same MFMA over K in the
    same order."""
    cfg = qwen3.QWEN3_8B
    t = 2048
    w = {k: v.to(DEV) for k, v in qwen3.random_weights(cfg, seed=0).items()}
    x = randn((t, cfg.hidden), 2).to(DEV)
    layer = qwen3.Qwen3Layer(w, cfg)
    y = layer(x).clone()
    cos, sin = qwen3.rope_tables(t, device=DEV)
    xn = ops.rmsnorm(x, w["w_in"])
    # the q, k, v products single-pass, as the columns of the layer's fused q|k|v GEMM are
    qh = ops.qk_norm_rope(ops.gemm(xn, w["wq"], split_k=False).view(t, 32, 128), w["w_qn"], cos, sin)
    kh = ops.qk_norm_rope(ops.gemm(xn, w["wk"], split_k=False).view(t, 8, 128), w["w_kn"], cos, sin)
    vh = ops.transpose_heads(ops.gemm(xn, w["wv"], split_k=False).view(t, 8, 128))
    o = ops.transpose_heads(ops.flash_attention(qh, kh, vh, 32, 8, True))
    h = ops.gemm(o.view(t, 4096), w["wo"], residual=x)
    a = ops.silu_mul(ops.gemm(ops.rmsnorm(h, w["w_post"]), w["wgu"]))
    y2 = ops.gemm(a, w["wd"], residual=h)
    assert torch.isfinite(y.float()).all()
    assert bits_equal(y, y2)
    # determinism: a second forward reproduces the first bit for bit
    assert bits_equal(layer(x), y)
