"""The bounds the GPU parity tests use, shown on the CPU to reject the plausible kernel slips they
are meant to catch (the slips are planted in CPU computations of the oracle's arithmetic, never in
GPU code), and to accept the rounding differences a correct kernel has.

* GEMM at BASELINE config 2's inputs (A, B ~ N(0, 1/64^2), outputs of RMS 1/64): the bound
  rtol = 2e-2, atol = 2e-2 * RMS(C) rejects a product that drops one 32-deep K step, which the
  former absolute atol = 2e-2 (larger than the outputs) accepted.
* Causal attention at BASELINE config 3's shape (S = 4096, D = 128, one head): the per-row bound
  rtol = 2e-2, atol = 2e-2 * RMS(row) rejects a skipped 64-key block and a causal mask that
  excludes the diagonal, and accepts P rounded to bf16 at 64-key blocks instead of the reference's
  1024-key blocks.
"""
import math

import torch

import oracle
from helpers import randn, rms, rows_close

RTOL = 2e-2


def _config2_sample():
    m, k, n = 4096, 4096, 12288
    a = randn((m, k), 0, std=1.0 / 64)
    b = randn((k, n), 1, std=1.0 / 64)
    rows = torch.tensor([0, 1000, 2047, 3001, m - 1])
    return a[rows], b


def test_gemm_bound_rejects_a_dropped_k_step():
    a, b = _config2_sample()
    want = oracle.gemm(a, b)
    atol = RTOL * rms(want)
    # a correct kernel: fp32 accumulation in another order, rounded once to bf16
    other_order = (a.float() @ b.float()).to(torch.bfloat16)
    assert torch.allclose(other_order.float(), want.float(), rtol=RTOL, atol=atol)
    # planted: the last 32-deep K step never multiplied
    k = a.shape[1]
    dropped = oracle.gemm(a[:, : k - 32], b[: k - 32])
    assert not torch.allclose(dropped.float(), want.float(), rtol=RTOL, atol=atol)
    # the former absolute floor let exactly this slip through
    assert torch.allclose(dropped.float(), want.float(), rtol=RTOL, atol=2e-2)


def _attention(q, k, v, scale, allowed):
    """fp64 softmax(q k^T * scale) v over the keys `allowed` [S, S] marks, rounded to bf16."""
    s = (q.double() @ k.double().t()) * scale
    s = s.masked_fill(~allowed, float("-inf"))
    p = torch.softmax(s, dim=-1)
    return (p @ v.double()).to(torch.bfloat16)


def _config3_head():
    s, d = 4096, 128
    q = randn((1, s, d), 0)
    k = randn((1, s, d), 1)
    v = randn((1, s, d), 2)
    return q, k, v


def test_attention_row_bound_rejects_planted_slips():
    q, k, v = _config3_head()
    s = q.shape[1]
    scale = 1.0 / math.sqrt(128)
    want = oracle.flash_attention(q, k, v, 1, 1, True, scale)[0]
    i = torch.arange(s)
    causal = i[:, None] >= i[None, :]
    # exact softmax in fp64 (P never rounded): a correct kernel's result differs from the oracle
    # by P's bf16 rounding only
    exact = _attention(q[0], k[0], v[0], scale, causal)
    ok, report = rows_close(exact, want, RTOL, 2e-2)
    assert ok, report
    # P rounded to bf16 per 64-key block, as the HIP kernel blocks keys
    blocked = oracle.flash_attention(q, k, v, 1, 1, True, scale, bq=64, bkv=64)[0]
    ok, report = rows_close(blocked, want, RTOL, 2e-2)
    assert ok, report
    # planted: key block [1024, 1088) skipped for every query past it
    skip = causal & ~((i[None, :] >= 1024) & (i[None, :] < 1088) & (i[:, None] >= 1088))
    ok, _ = rows_close(_attention(q[0], k[0], v[0], scale, skip), want, RTOL, 2e-2)
    assert not ok
    # planted: the causal mask off by one (the diagonal key excluded; row 0 keeps key 0 so no row
    # is empty)
    off = (i[:, None] > i[None, :]) | (i[:, None] == 0) & (i[None, :] == 0)
    ok, _ = rows_close(_attention(q[0], k[0], v[0], scale, off), want, RTOL, 2e-2)
    assert not ok
