"""Parity of the vector-family HIP kernels with the CPU oracle (bf16 outputs: allclose at the
BASELINE tolerance rtol=atol=2e-2, plus >= 99% of outputs bit-identical; exact ops: bit-equal)."""
import math

import pytest
import torch

import oracle
from helpers import assert_close, bits_equal, randn
from ptb_amd import _lib, ops

pytestmark = pytest.mark.gpu

DEV = "cuda"
RTOL = ATOL = 2e-2


def bit_fraction(got, want):
    a = got.detach().cpu().contiguous().view(torch.int16)
    b = want.detach().cpu().contiguous().view(torch.int16)
    return float((a == b).float().mean())


def check_bf16(got, want, what, min_exact=0.99):
    assert_close(got, want, RTOL, ATOL, what)
    frac = bit_fraction(got, want)
    assert frac >= min_exact, f"{what}: only {frac:.4%} of outputs bit-identical to the oracle"


@pytest.mark.parametrize("rows,cols,wdtype,seed", [
    (2048, 4096, torch.float32, 0),
    (2048, 4096, torch.bfloat16, 1),    # L2048/00 (bf16 weight)
    (3, 128, torch.bfloat16, 2),        # one wave per row, ragged row count
    (5, 2056, torch.float32, 3),        # block per row, partial last chunk group
    (7, 16384, torch.bfloat16, 4),      # largest register-resident row
    (2, 24576, torch.float32, 5),       # long-row two-pass kernel
])
def test_rmsnorm(rows, cols, wdtype, seed):
    x = randn((rows, cols), seed)
    w = randn((cols,), seed + 100, dtype=wdtype, std=0.02, mean=1.0)
    got = ops.rmsnorm(x.to(DEV), w.to(DEV), 1e-6)
    torch.cuda.synchronize()
    check_bf16(got, oracle.rmsnorm(x, w, 1e-6), f"rmsnorm {rows}x{cols}")


def test_rmsnorm_zero_rows_and_empty():
    x = torch.zeros((4, 256), dtype=torch.bfloat16)
    w = torch.ones(256, dtype=torch.bfloat16)
    got = ops.rmsnorm(x.to(DEV), w.to(DEV), 1e-6)
    assert bits_equal(got, oracle.rmsnorm(x, w, 1e-6))
    empty = ops.rmsnorm(torch.empty((0, 256), dtype=torch.bfloat16, device=DEV), w.to(DEV))
    assert empty.shape == (0, 256)


@pytest.mark.parametrize("rows,cols,seed", [
    (2048, 6144, 0),    # vector_softmax_2048x6144_bf16
    (8, 128, 1), (1, 8192, 2), (1024, 1536, 3), (33, 384, 4),
    (4, 24576, 5),      # long-row kernel
])
def test_softmax(rows, cols, seed):
    x = randn((rows, cols), seed)
    got = ops.softmax_rows(x.to(DEV))
    check_bf16(got, oracle.softmax_rows(x), f"softmax {rows}x{cols}")


def test_softmax_nan_and_inf():
    x = randn((4, 512), 7)
    x[1, 17] = float("nan")          # NaN-propagating max: whole row NaN
    x[2, :] = -float("inf")          # all -inf: NaN like the reference's exp(-inf - -inf)
    x[3, 5] = float("inf")
    got = ops.softmax_rows(x.to(DEV)).cpu()
    want = oracle.softmax_rows(x)
    assert torch.isnan(got[1]).all() and torch.isnan(want[1]).all()
    assert torch.isnan(got[2]).all() and torch.isnan(want[2]).all()
    assert torch.equal(torch.isnan(got[3]), torch.isnan(want[3]))
    check_bf16(got[0:1], want[0:1], "softmax clean row")


@pytest.mark.parametrize("rows,inter,seed", [(2048, 12288, 0), (3, 8, 1), (17, 1032, 2)])
def test_silu_mul(rows, inter, seed):
    gu = randn((rows, 2 * inter), seed)
    got = ops.silu_mul(gu.to(DEV))
    check_bf16(got, oracle.silu_mul(gu), f"silu_mul {rows}x{inter}")


@pytest.mark.parametrize("shape", [(2048, 8, 128), (32, 2048, 128), (3, 5, 8), (1, 7, 64)])
def test_transpose_heads_exact(shape):
    x = randn(shape, 11)
    got = ops.transpose_heads(x.to(DEV))
    assert bits_equal(got, oracle.transpose_heads(x))


@pytest.mark.parametrize("tokens,cols", [(2048, (4096, 1024, 1024)), (5, (384, 128, 256)), (1, (128, 128, 128))])
def test_row_strided_slices_exact(tokens, cols):
    """q-norm + RoPE and the head transpose over column slices of a [T, q|k|v] matrix (rows ld
    apart) give the bits of the same calls on contiguous copies of the slices."""
    qd, kd, vd = cols
    qkv = randn((tokens, qd + kd + vd), 50).to(DEV)
    w = randn((128,), 51, std=0.1, mean=1.0).to(DEV)
    cos, sin = (t.to(DEV) for t in oracle.rope_tables(tokens, 128, 1.0e6))
    for lo, width in ((0, qd), (qd, kd)):
        sl = qkv[:, lo:lo + width].view(tokens, width // 128, 128)
        assert not sl.is_contiguous() or tokens == 1
        got = ops.qk_norm_rope(sl, w, cos, sin, 1e-6)
        assert bits_equal(got, ops.qk_norm_rope(sl.contiguous(), w, cos, sin, 1e-6))
    sl = qkv[:, qd + kd:].view(tokens, vd // 128, 128)
    assert bits_equal(ops.transpose_heads(sl), ops.transpose_heads(sl.contiguous()))
    with pytest.raises(ValueError):   # rows must be contiguous inside
        ops.transpose_heads(qkv.view(tokens, -1, 128)[:, :, :64])


@pytest.mark.parametrize("tokens,heads,tables,seed", [
    (2048, 32, "bundle", 0),   # L2048/02: cos/sin drawn by the spec's make_inputs (randn)
    (2048, 8, "rope", 1),      # L2048/04 with real theta=1e6 tables
    (5, 3, "rope", 2),
])
def test_qk_norm_rope(tokens, heads, tables, seed):
    x = randn((tokens, heads, 128), seed)
    w = randn((128,), seed + 1)
    if tables == "bundle":
        cos = randn((tokens, 128), seed + 2, dtype=torch.float32)
        sin = randn((tokens, 128), seed + 3, dtype=torch.float32)
    else:
        cos, sin = oracle.rope_tables(tokens, 128, 1.0e6)
    got = ops.qk_norm_rope(x.to(DEV), w.to(DEV), cos.to(DEV), sin.to(DEV), 1e-6)
    check_bf16(got, oracle.qk_norm_rope(x, w, cos, sin, 1e-6), f"qk_norm_rope {tokens}x{heads}")


@pytest.mark.parametrize("n,seed", [(12288 * 4096, 0), (1024 * 1024, 1), (8 * 128 + 5, 2), (3, 3),
                                    (98304, 4), (98305, 5), (4096 + 8, 6), (16384, 7), (517, 8),
                                    (65536 + 13, 9)])
def test_reduce(n, seed):
    """Two passes above 98304 elements, one workgroup of 64..1024 threads at or below (batches of
    65536 elements, skipped slots, a tail of n % 8 elements)."""
    x = randn((n,), seed)
    xd = x.to(DEV)
    got_max = ops.reduce(xd, "max").cpu()
    assert torch.equal(got_max, oracle.reduce_max(x))
    got_sum = ops.reduce(xd, "sum").cpu()
    want = oracle.reduce_sum(x)
    # fp32 accumulation in a different order than the exact sum: bound by the summation error scale
    bound = 1e-6 * float(x.float().abs().sum()) + 1e-6
    assert abs(float(got_sum) - float(want)) <= bound, (float(got_sum), float(want), bound)
    # shifted input so the sum is far from zero: relative error within 1e-5
    xs = (x.float() + 1.0).to(torch.bfloat16)
    gs, ws = float(ops.reduce(xs.to(DEV), "sum")), float(oracle.reduce_sum(xs))
    assert abs(gs - ws) <= 1e-5 * abs(ws), (gs, ws)


@pytest.mark.parametrize("n,seed", [(8, 0), (1000003, 1), (4096 * 4096, 2), (30003, 3)])
def test_reduce_fp32_input(n, seed):
    """fp32 elements (the MoE router's sum of its top-k weights is the 8-element case)."""
    x = torch.randn(n, generator=torch.Generator().manual_seed(seed)) + 0.5
    xd = x.to(DEV)
    assert torch.equal(ops.reduce(xd, "max").cpu(), oracle.reduce_max(x))
    got, want = float(ops.reduce(xd, "sum")), float(oracle.reduce_sum(x))
    assert abs(got - want) <= 1e-6 * float(x.abs().sum()) + 1e-6, (got, want)


@pytest.mark.parametrize("n", [4096, 1 << 20])
def test_reduce_max_nan(n):
    x = randn((n,), 9)
    x[1234] = float("nan")
    assert math.isnan(float(ops.reduce(x.to(DEV), "max")))


@pytest.mark.parametrize("n", [1024 * 1024, 8 * 128, 37])
def test_add_scalar_exact(n):
    x = randn((n,), 5)
    got = ops.add_scalar(x.to(DEV), 1.0)
    assert bits_equal(got, oracle.add_scalar(x, 1.0))


def test_error_paths_on_device():
    x = torch.zeros((4, 12), dtype=torch.bfloat16, device=DEV)   # 12 % 8 != 0
    w = torch.ones(12, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(_lib.AlignmentError):
        ops.rmsnorm(x, w)
    xh = torch.zeros((4, 3, 64), dtype=torch.bfloat16, device=DEV)
    with pytest.raises(_lib.UnsupportedError):
        ops.qk_norm_rope(xh, torch.ones(64, dtype=torch.bfloat16, device=DEV),
                         torch.ones((4, 64), device=DEV), torch.zeros((4, 64), device=DEV))


# ---- fp32 vector ops: the reference's own fp32 workload cases, at their tolerances -------------

def _case_inputs(seed, *shapes_scales):
    """make_inputs of tests/cases/workloads/{rmsnorm,softmax,swiglu}.py: one generator, fp32 randn per
    argument in order (times the case's scale)."""
    g = torch.Generator().manual_seed(seed)
    return [torch.randn(n, generator=g, dtype=torch.float32) * s for n, s in shapes_scales]


def test_rmsnorm_f32_reference_case():
    """tests/cases/workloads/rmsnorm.py: M=8, N=64, EPS=1e-5, fp32 x and w; outputs o (row arm) and
    c (column arm) within the case's rtol = atol = 1e-4 and the north-star's 1e-5 relative bound."""
    m, n, eps = 8, 64, 1e-5
    x, w = _case_inputs(0, (m * n, 1.0), (n, 1.0))
    x = x.reshape(m, n)
    o = ops.rmsnorm(x.to(DEV), w.to(DEV), eps).cpu()
    c = ops.col_rms(x.to(DEV), eps).cpu()
    want_o, want_c = oracle.rmsnorm_f32(x, w, eps), oracle.col_rms_f32(x, eps)
    assert_close(o, want_o, 1e-5, 1e-6, "rmsnorm.py o")
    assert_close(c, want_c, 1e-5, 1e-6, "rmsnorm.py c")


@pytest.mark.parametrize("rows,cols,seed", [(2048, 4096, 1), (3, 20, 2), (5, 4100, 3), (2, 40000, 4)])
def test_rmsnorm_f32_shapes(rows, cols, seed):
    """Wave-per-row, block-per-row and the two-pass long-row forms, fp32 throughout."""
    x = randn((rows, cols), seed, dtype=torch.float32)
    w = randn((cols,), seed + 1, dtype=torch.float32, std=0.02, mean=1.0)
    got = ops.rmsnorm(x.to(DEV), w.to(DEV), 1e-6).cpu()
    assert_close(got, oracle.rmsnorm_f32(x, w, 1e-6), 1e-5, 1e-6, f"rmsnorm f32 {rows}x{cols}")
    c = ops.col_rms(x.to(DEV), 1e-6).cpu()
    assert_close(c, oracle.col_rms_f32(x, 1e-6), 1e-5, 1e-6, f"col rms {rows}x{cols}")


def test_softmax_f32_reference_case():
    """tests/cases/workloads/softmax.py: 256 rows of 64 fp32 values, rtol 1e-5, atol 1e-6 (:84)."""
    (x,) = _case_inputs(0, (256 * 64, 1.0))
    x = x.reshape(256, 64)
    got = ops.softmax_rows(x.to(DEV)).cpu()
    assert got.dtype == torch.float32
    assert_close(got, oracle.softmax_rows(x, out_dtype=torch.float32), 1e-5, 1e-6, "softmax.py")


@pytest.mark.parametrize("rows,cols,seed", [(2048, 6144, 1), (7, 12, 2), (3, 9000, 3), (2, 40000, 4)])
def test_softmax_f32_shapes(rows, cols, seed):
    x = randn((rows, cols), seed, dtype=torch.float32, std=3.0)
    if rows > 2:
        x[1, 5] = float("nan")          # a NaN row stays NaN
        x[2, :] = -5.0                  # constant row: uniform
    got = ops.softmax_rows(x.to(DEV)).cpu()
    assert_close(got, oracle.softmax_rows(x, out_dtype=torch.float32), 1e-5, 1e-6, f"softmax f32 {rows}x{cols}")
    assert torch.isnan(got[1]).all() if rows > 2 else True


def test_swiglu_f32_reference_case():
    """tests/cases/workloads/swiglu.py: x [128, 256], wg / wu [256, 128], all randn * 0.1 in fp32,
    o = silu(x @ wg) * (x @ wu) at rtol = atol = 1e-3 (:100); the elementwise half alone (silu_mul
    over gate | up) at the fp32 vector bound 1e-5."""
    m, n, k = 128, 128, 256
    x, wg, wu = _case_inputs(0, (m * k, 0.1), (k * n, 0.1), (k * n, 0.1))
    x, wg, wu = x.reshape(m, k), wg.reshape(k, n), wu.reshape(k, n)
    o = ops.swiglu_f32(x.to(DEV), wg.to(DEV), wu.to(DEV)).cpu()
    assert_close(o, oracle.swiglu_f32(x, wg, wu), 1e-3, 1e-3, "swiglu.py")
    gu = torch.cat([x @ wg, x @ wu], dim=1).contiguous()
    got = ops.silu_mul(gu.to(DEV)).cpu()
    assert got.dtype == torch.float32
    assert_close(got, oracle.silu_mul_f32(gu), 1e-5, 1e-6, "silu_mul f32")


@pytest.mark.parametrize("m,n,k", [(300, 200, 100), (64, 1000, 513)])
def test_swiglu_f32_ragged(m, n, k):
    x = randn((m, k), 7, dtype=torch.float32, std=0.1)
    wg = randn((k, n), 8, dtype=torch.float32, std=0.1)
    wu = randn((k, n), 9, dtype=torch.float32, std=0.1)
    o = ops.swiglu_f32(x.to(DEV), wg.to(DEV), wu.to(DEV)).cpu()
    assert_close(o, oracle.swiglu_f32(x, wg, wu), 1e-4, 1e-5, f"swiglu f32 {m}x{n}x{k}")
