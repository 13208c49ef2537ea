"""Parity of the flash-attention kernel with the oracle's restatement of the reference's
_prefill_kernel (P rounded to bf16 before P.V).  The kernel blocks keys by 64 where the reference
blocks by 1024, so the bf16 rounding points of P differ: bf16 tolerance rtol = 2e-2 with the
absolute floor 2e-2 times each output row's RMS (a late row averages thousands of keys, so its
outputs are far below 1 and a fixed absolute floor would hide a skipped key block;
tests/test_tolerances.py shows this bound rejects one skipped 64-key block and an off-by-one causal
mask), and the exact invariants (row 0 = V[0]) are checked bit-for-bit.  Outputs are NaN-filled
before every launch (tests/conftest.py)."""
import math

import pytest
import torch

import oracle
from helpers import assert_close_rows, bits_equal, randn
from ptb_amd import _lib, ops

pytestmark = pytest.mark.gpu

DEV = "cuda"
RTOL = ATOL = 2e-2


def inputs(batch, hq, hkv, s, seed):
    q = randn((batch * hq, s, 128), seed)
    k = randn((batch * hkv, s, 128), seed + 1)
    v = randn((batch * hkv, s, 128), seed + 2)
    return q, k, v


@pytest.mark.parametrize("batch,hq,hkv,s,causal", [
    (1, 32, 8, 4096, True),     # BASELINE config 3 / attention_prefill_32x8x4096_bf16
    (1, 32, 8, 2048, True),     # L2048/06 (the Qwen3-8B layer's attention): paired 128-row tiles
    (1, 56, 8, 896, True),      # paired tiles, odd tile count (the middle unit's second half idle)
    (1, 16, 8, 1024, True),
    (1, 24, 8, 512, True),      # G = 3
    (1, 64, 8, 256, True),      # G = 8
    (2, 4, 2, 384, True),       # batch > 1, S not a multiple of 256
    (1, 8, 8, 128, True),       # MHA, a single (partial) tile
    (1, 8, 2, 640, True),       # S not a multiple of the 256-row tile
    (1, 8, 2, 512, False),      # non-causal path
    (1, 32, 8, 2048, False),    # non-causal, one 256-row workgroup per CU
    (1, 4, 4, 384, False),      # non-causal, partial tile
])
def test_flash_attention(batch, hq, hkv, s, causal):
    q, k, v = inputs(batch, hq, hkv, s, 0)
    o = ops.flash_attention(q.to(DEV), k.to(DEV), v.to(DEV), hq, hkv, causal).cpu()
    # the oracle is the reference's own blocking (1024, or S when shorter); check a subset of
    # heads at the largest sizes to keep the CPU side to seconds
    heads = torch.arange(batch * hq)
    if s >= 2048:
        heads = torch.tensor([0, 5, 13, 31])
    want = oracle.flash_attention(q, k, v, hq, hkv, causal, 1.0 / math.sqrt(128))
    assert_close_rows(o[heads], want[heads], RTOL, ATOL, f"flash {batch}x{hq}x{hkv}x{s} causal={causal}")
    if causal:
        # row 0 attends only to key 0: p = 1 exactly, so O[h, 0] = V[kv(h), 0] bit for bit
        g = hq // hkv
        for bh in range(batch * hq):
            b, h = divmod(bh, hq)
            assert bits_equal(o[bh, 0], v[b * hkv + h // g, 0])


def test_flash_constant_v():
    """V = const c: every output is c * sum(bf16(p)) / sum(p), i.e. c within bf16 rounding."""
    q, k, _ = inputs(1, 8, 2, 512, 3)
    v = torch.full((2, 512, 128), 0.75, dtype=torch.bfloat16)
    o = ops.flash_attention(q.to(DEV), k.to(DEV), v.to(DEV), 8, 2, True).cpu().float()
    assert (o - 0.75).abs().max() <= 0.75 * 2 ** -7


@pytest.mark.parametrize("batch,hq,hkv,s", [(1, 32, 8, 2048), (2, 4, 2, 384), (1, 8, 8, 128)])
def test_flash_tokens_out_is_the_transposed_output(batch, hq, hkv, s):
    """The token-major output ([B, S, hq, D]) holds exactly the head-major output's values,
    transposed: the same kernel, only the store address differs."""
    q = randn((batch * hq, s, 128), 51).to(DEV)
    k = randn((batch * hkv, s, 128), 52).to(DEV)
    v = randn((batch * hkv, s, 128), 53).to(DEV)
    heads = ops.flash_attention(q, k, v, hq, hkv, True).cpu()
    tokens = ops.flash_attention(q, k, v, hq, hkv, True, tokens_out=True).cpu()
    assert tokens.shape == (batch, s, hq, 128)
    assert bits_equal(tokens, heads.view(batch, hq, s, 128).transpose(1, 2).contiguous())


@pytest.mark.parametrize("batch,hq,hkv,s,causal,scale", [
    (1, 32, 8, 2048, True, None),      # the prefill layer's shape: paired heavy/light 128-row tiles
    (1, 56, 8, 896, True, None),       # paired tiles, odd tile count (the middle unit's second half idle)
    (1, 32, 8, 1024, True, None),      # 128-row workgroups (4 waves), causal
    (1, 32, 8, 4096, True, None),      # 256-row workgroups
    (2, 8, 2, 256, False, -0.05),      # batches, no mask, a negative scale
])
def test_flash_qkv_is_the_launch_chain(batch, hq, hkv, s, causal, scale):
    """The fused form (q normalised and rotated in the prologue, q and v read in place from the
    [B*S, ld] projection output, ld wider than q|k|v) equals qk_norm_rope(q) + transpose_heads(v) +
    flash_attention(tokens_out) bit for bit, batch by batch."""
    from ptb_amd import qwen3

    d, eps = 128, 1e-6
    ld = (hq + 2 * hkv) * d + 64
    qkv = randn((batch * s, ld), 40).to(DEV)
    w_qn = (randn((d,), 41).float() * 0.1 + 1).to(torch.bfloat16).to(DEV)
    w_kn = (randn((d,), 42).float() * 0.1 + 1).to(torch.bfloat16).to(DEV)
    cos, sin = qwen3.rope_tables(s, d, 1.0e6, DEV)
    kcol, vcol = hq * d, (hq + hkv) * d
    kh = torch.cat([ops.qk_norm_rope(qkv[i * s:(i + 1) * s, kcol:vcol].view(s, hkv, d), w_kn, cos, sin, eps)
                    for i in range(batch)])
    got = ops.flash_attention_qkv(qkv, kh, w_qn, cos, sin, hq, hkv, eps, causal, scale)
    for i in range(batch):
        rows = qkv[i * s:(i + 1) * s]
        qh = ops.qk_norm_rope(rows[:, :kcol].view(s, hq, d), w_qn, cos, sin, eps)
        vh = ops.transpose_heads(rows[:, vcol:vcol + hkv * d].view(s, hkv, d))
        want = ops.flash_attention(qh, kh[i * hkv:(i + 1) * hkv], vh, hq, hkv, causal, scale, tokens_out=True)
        assert bits_equal(got[i], want[0]), f"batch {i}"


def test_flash_refuses_bad_shapes():
    q = torch.zeros((4, 100, 128), dtype=torch.bfloat16, device=DEV)
    with pytest.raises(_lib.UnsupportedError):
        ops.flash_attention(q, q[:2].contiguous(), q[:2].contiguous(), 4, 2)
    q64 = torch.zeros((4, 128, 64), dtype=torch.bfloat16, device=DEV)
    with pytest.raises(_lib.UnsupportedError):
        ops.flash_attention(q64, q64[:2].contiguous(), q64[:2].contiguous(), 4, 2)
