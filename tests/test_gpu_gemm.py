"""Parity of the bf16 and fp8 GEMM kernels with the CPU oracle.

Full-size shapes are checked on sampled rows (one random row from every 256-row tile plus the
first and last rows): a row of C depends only on that row of A, so the oracle computes exactly
those rows.  Tolerance: the BASELINE bf16/fp8 bound, rtol = 2e-2, with the absolute floor 2e-2
times the RMS of the expected output wherever outputs are not O(1) (the BASELINE config-2 operands
~N(0, 1/64^2) give outputs of RMS 1/64, so an absolute 2e-2 would exceed the outputs themselves;
tests/test_tolerances.py shows the scaled bound rejects a product that drops one 32-deep K step).
Every output buffer is NaN-filled before the launch (tests/conftest.py), so an unwritten tile
fails.  The quantisers are bit-exact."""
import pytest
import torch

import oracle
from helpers import assert_close, bits_equal, randn, rms
from ptb_amd import _lib, ops

pytestmark = pytest.mark.gpu

DEV = "cuda"
RTOL = ATOL = 2e-2


def sample_rows(m, seed=0):
    g = torch.Generator().manual_seed(seed)
    rows = {0, m - 1}
    for t0 in range(0, m, 256):
        rows.add(t0 + int(torch.randint(0, min(256, m - t0), (1,), generator=g)))
    return torch.tensor(sorted(rows))


def run_gemm(m, k, n, seed, std_a, std_b, resid=False):
    a = randn((m, k), seed, std=std_a)
    b = randn((k, n), seed + 1, std=std_b)
    r = randn((m, n), seed + 2) if resid else None
    c = ops.gemm(a.to(DEV), b.to(DEV), None if r is None else r.to(DEV)).cpu()
    rows = sample_rows(m, seed) if m > 512 else torch.arange(m)
    want = oracle.gemm(a[rows], b, None if r is None else r[rows])
    return c[rows], want


@pytest.mark.parametrize("m,k,n,resid", [
    (4096, 4096, 12288, False),   # BASELINE config 2 (Qwen3-8B gate/up shape)
    (2048, 4096, 4096, False),    # L2048/01 q_proj
    (2048, 4096, 1024, False),    # L2048/03 k/v_proj
    (2048, 4096, 4096, True),     # L2048/08 o_proj + residual
    (2048, 12288, 4096, True),    # L2048/11 down + residual
    (2048, 4096, 6144, False),    # fused q|k|v projection: one round of 256x192 tiles
])
def test_gemm_layer_shapes(m, k, n, resid):
    std = 1.0 / 64.0
    got, want = run_gemm(m, k, n, 0, std, std, resid)
    assert_close(got, want, RTOL, ATOL * rms(want), f"gemm {m}x{k}x{n}")


@pytest.mark.parametrize("m,k,n", [
    (1, 2048, 768), (8, 768, 2048), (16, 2048, 768), (100, 384, 1152), (300, 768, 128),
    (1024, 2048, 128), (257, 64, 264), (128, 4096, 4096),
    (2000, 512, 4088),    # 256x128 tiles, ragged in M and N
    (4000, 256, 4000),    # 256x256 tiles, ragged in M and N
    (2000, 256, 6000),    # 256x192 tiles, ragged in M and N
])
def test_gemm_ragged(m, k, n):
    got, want = run_gemm(m, k, n, 3, 1.0, 1.0 / k ** 0.5)
    assert_close(got, want, RTOL, ATOL, f"gemm {m}x{k}x{n}")


@pytest.mark.parametrize("m,k,n", [
    (4000, 256, 4000),    # 256x256 tiles, ragged in M and N
    (2000, 512, 4088),    # 256x128 tiles, ragged in M and N
    (2000, 512, 6000),    # 256x192 tiles (one round of 256 where 256x256 would leave CUs idle), ragged
])
def test_gemm_ragged_residual_stays_inside_c(m, k, n):
    """The epilogue stages each tile through the LDS and masks rows past M and columns past N with
    buffer resources: on ragged last tiles the residual sum is right and nothing lands past C (a
    NaN-filled guard after C's last element stays NaN)."""
    a = randn((m, k), 5)
    b = randn((k, n), 6, std=1.0 / k ** 0.5)
    r = randn((m, n), 7)
    guard = torch.full((m * n + 8192,), float("nan"), dtype=torch.bfloat16, device=DEV)
    c = guard[: m * n].view(m, n)
    ops.gemm(a.to(DEV), b.to(DEV), r.to(DEV), out=c)
    assert bool(guard[m * n:].isnan().all()), "the GEMM wrote past C"
    rows = sample_rows(m, 5)
    assert_close(c.cpu()[rows], oracle.gemm(a[rows], b, r[rows]), RTOL, ATOL, f"gemm+R {m}x{k}x{n}")


@pytest.mark.parametrize("m,k,n", [
    (4096, 4096, 12288),   # three rounds of 256x256 tiles
    (4300, 256, 8248),     # 561 tiles, ragged in M and N: some workgroups walk three tiles, most two
])
def test_gemm_persistent_walk_is_the_tile_by_tile_product(m, k, n):
    """Two or more rounds of 256x256 tiles run as one workgroup per CU walking its tiles, the next
    tile's first stage loading during the current tile's epilogue.  Every tile keeps its MFMA order
    over K, so each 256-row band equals the product of that band of A alone (a one-round shape,
    other tiles) bit for bit; the sampled rows against the oracle, and nothing written past C."""
    a = randn((m, k), 8, std=1.0 / 64)
    b = randn((k, n), 9, std=1.0 / 64)
    guard = torch.full((m * n + 8192,), float("nan"), dtype=torch.bfloat16, device=DEV)
    c = guard[: m * n].view(m, n)
    ad, bd = a.to(DEV), b.to(DEV)
    ops.gemm(ad, bd, out=c)
    assert bool(guard[m * n:].isnan().all()), "the GEMM wrote past C"
    for r0 in (0, 256 * ((m - 1) // 256)):
        band = ops.gemm(ad[r0:r0 + 256].contiguous(), bd, split_k=False)
        assert bits_equal(c[r0:r0 + 256], band), f"rows {r0}.. differ from the band's own product"
    rows = sample_rows(m, 8)
    want = oracle.gemm(a[rows], b)
    assert_close(c.cpu()[rows], want, RTOL, ATOL * rms(want), f"gemm {m}x{k}x{n}")


def test_gemm_bundle_inputs_exact_products():
    """bf16 operands from the bundle's make_inputs draw (randn): small enough that the fp32
    accumulation is exact for small K -> bit-exact output (tests/baselines/tpuv6e.txt:162 records
    max_abs_err 0 for the reference's bf16 matmul)."""
    a = torch.randint(-8, 9, (64, 64)).to(torch.bfloat16)
    b = torch.randint(-8, 9, (64, 256)).to(torch.bfloat16)
    c = ops.gemm(a.to(DEV), b.to(DEV)).cpu()
    assert bits_equal(c, oracle.gemm(a, b))


def test_gemm_refuses_bad_k():
    a = torch.zeros((4, 100), dtype=torch.bfloat16, device=DEV)
    b = torch.zeros((100, 64), dtype=torch.bfloat16, device=DEV)
    with pytest.raises(_lib.UnsupportedError):
        ops.gemm(a, b)


@pytest.mark.parametrize("rows,cols,seed", [(2048, 12288, 0), (3, 64, 1), (9, 4096, 2), (2, 8, 3)])
def test_quant_rows_exact(rows, cols, seed):
    x = randn((rows, cols), seed)
    if rows > 2:
        x[1] = 0.0                                  # all-zero row -> scale 1
    xq, sc = ops.quant_rows_e4m3(x.to(DEV))
    wq, wsc = oracle.quant_rows_e4m3(x)
    assert torch.equal(sc.cpu(), wsc)
    assert bits_equal(xq, wq)


@pytest.mark.parametrize("k,n,seed", [(12288, 4096, 0), (128, 16, 1), (100, 70, 2), (1000, 4100, 3), (36, 12, 4)])
def test_quant_weight_exact(k, n, seed):
    """The K-split absmax (K, N multiples of 4: ragged column blocks and K slices included) and the
    any-shape path, bit for bit; a zero column takes scale 1, a column holding NaN scale 1 (torch's
    amax propagates NaN and `amax > 0` fails), its NaN the e4m3 NaN."""
    w = randn((k, n), seed, dtype=torch.float32, std=0.02)
    w[:, 3] = 0.0
    w[k // 2, 5] = float("nan")
    wq, sc = ops.quant_weight_e4m3(w.to(DEV))
    owq, osc = oracle.quant_weight_e4m3(w)
    assert torch.equal(sc.cpu(), osc)
    assert bits_equal(wq, owq)


@pytest.mark.parametrize("m,k,n", [(2048, 12288, 4096), (1, 128, 16), (300, 256, 272), (257, 1024, 512),
                                   (4096, 1152, 4096),   # 256x256 tiles, two-stage ring, an odd step count
                                   (2048, 896, 4096),    # 256x128 tiles, 7 steps: a one-step remainder
                                   (4000, 256, 4000),    # 256x256 tiles, ragged in M and N
                                   (2000, 512, 4080)])   # 256x128 tiles, ragged in M and N
def test_gemm_fp8(m, k, n):
    """activations bf16 ~N(0,1) quantised per token, weights from N(0,0.02)
    quantised per output channel; the GPU GEMM and the oracle see the same quantised operands."""
    x = randn((m, k), 10)
    w = randn((k, n), 11, dtype=torch.float32, std=0.02)
    wq_t, sw = ops.quant_weight_e4m3(w.to(DEV))
    xq, sx = ops.quant_rows_e4m3(x.to(DEV))
    c = ops.gemm_fp8(xq, sx, wq_t, sw).cpu()
    rows = sample_rows(m, 1) if m > 512 else torch.arange(m)
    want = oracle.gemm_fp8(xq.cpu()[rows], sx.cpu()[rows], wq_t.cpu(), sw.cpu())
    # outputs are ~N(0, 0.02^2 K): scale the absolute floor with them
    scale = float(want.float().abs().mean()) + 1e-6
    assert_close(c[rows], want, RTOL, ATOL * scale, f"gemm_fp8 {m}x{k}x{n}")


@pytest.mark.parametrize("m,k,n,resid", [
    (128, 2048, 128, False), (8, 2048, 768, False), (512, 2048, 128, True), (32, 3072, 768, False),
    (1000, 4096, 264, True), (64, 1024, 2048, False), (256, 12288, 512, True),
])
def test_split_k_gemm(m, k, n, resid):
    """Shapes with few output tiles run split-K (fp32 partials, one finish pass): the same result as
    the oracle, and as the single-pass kernel within the bf16 bound."""
    assert _lib.load().ptb_gemm_bf16_workspace_bytes(m, n, k) > 0, "this shape is meant to split"
    a = randn((m, k), 31, std=1 / 64)
    b = randn((k, n), 32, std=1.0)
    r = randn((m, n), 33) if resid else None
    ad, bd, rd = a.to(DEV), b.to(DEV), None if r is None else r.to(DEV)
    split = ops.gemm(ad, bd, rd).cpu()
    single = ops.gemm(ad, bd, rd, split_k=False).cpu()
    want = oracle.gemm(a, b, r)
    scale = float(want.float().abs().mean())
    assert_close(split, want, RTOL, 2e-2 * scale, f"split-K {m}x{k}x{n}")
    assert_close(split, single, RTOL, 2e-2 * scale, f"split-K vs single pass {m}x{k}x{n}")


@pytest.mark.parametrize("m,k,n", [(64, 768, 2048), (256, 960, 768), (2048, 4096, 4096), (2048, 12288, 4096),
                                   (1800, 24576, 2000)])
def test_no_split_below_1024(m, k, n):
    """Below K = 1024 a single pass over K is faster than partials plus a finish, and so is a GEMM
    whose 256x256, 256x128 or 128x128 tiles cover 3/4 of the CUs (the o- and down projections, and
    a ragged 24576-deep one with 240 128x128 tiles): no workspace is asked for, and the result
    matches the oracle."""
    assert _lib.load().ptb_gemm_bf16_workspace_bytes(m, n, k) == 0
    a, b = randn((m, k), 35, std=1 / 32), randn((k, n), 36)
    got = ops.gemm(a.to(DEV), b.to(DEV)).cpu()
    want = oracle.gemm(a, b)
    assert_close(got, want, RTOL, 2e-2 * float(want.float().abs().mean()), f"no split {m}x{k}x{n}")


def test_split_k_exact_on_small_integers():
    """Small-integer operands make every partial and sum exact in fp32: split-K equals the oracle bit
    for bit, whatever the slicing."""
    g = torch.Generator().manual_seed(34)
    a = torch.randint(-3, 4, (96, 4096), generator=g).to(torch.bfloat16)
    b = torch.randint(-3, 4, (4096, 136), generator=g).to(torch.bfloat16)
    assert _lib.load().ptb_gemm_bf16_workspace_bytes(96, 136, 4096) > 0
    got = ops.gemm(a.to(DEV), b.to(DEV)).cpu()
    assert bits_equal(got, oracle.gemm(a, b))


@pytest.mark.parametrize("m,k,n,resid", [(2048, 768, 768, False), (1000, 768, 264, True), (768, 3072, 1024, False),
                                         (4000, 384, 512, True), (2048, 4096, 1024, True)])
def test_gemm_64x128_tiles(m, k, n, resid):
    """Mid-size shapes whose 128x128 tiles cover less than 3/4 of the CUs run 64x128 tiles (K split
    when the plan's cost model says so: 768x3072x1024)."""
    c, want = run_gemm(m, k, n, 41, 1 / 32, 1 / 16, resid)
    assert_close(c, want, RTOL, 2e-2 * float(want.float().abs().mean()), f"64x128 {m}x{k}x{n}")


@pytest.mark.parametrize("m,k,n,resid", [(6144, 1024, 1024, False), (6000, 768, 1000, True)])
def test_gemm_256x128_tiles_from_three_quarters(m, k, n, resid):
    """256x128 tiles that cover 3/4 of the CUs or more run as one round of them (192 tiles here),
    ragged rows and columns included."""
    c, want = run_gemm(m, k, n, 43, 1 / 32, 1 / 16, resid)
    assert_close(c, want, RTOL, 2e-2 * float(want.float().abs().mean()), f"256x128 {m}x{k}x{n}")


@pytest.mark.parametrize("m,k,inter", [(2048, 4096, 12288), (300, 512, 256), (64, 128, 128), (1000, 1024, 384)])
def test_gemm_swiglu_fused(m, k, inter):
    """The gate_up GEMM with silu(g) * u in its epilogue equals the two launches it replaces bit for
    bit (same accumulation per output, the same roundings and formula), and the oracle within the
    bf16 bound; rows past a 256-row tile's end (m = 300, 1000) are not stored."""
    a = randn((m, k), 41, std=1 / 16)
    b = randn((k, 2 * inter), 42, std=1 / 4)
    ad, bd = a.to(DEV), b.to(DEV)
    fused = ops.gemm_swiglu(ad, bd).cpu()
    pair = ops.silu_mul(ops.gemm(ad, bd, split_k=False)).cpu()
    assert bits_equal(fused, pair)
    if m * k * inter <= 300 * 512 * 256:
        want = oracle.silu_mul(oracle.gemm(a, b))
        assert_close(fused, want, RTOL, 2e-2 * float(want.float().abs().mean()), f"swiglu {m}x{k}x{inter}")


@pytest.mark.parametrize("m,k,n,resid", [
    (4096, 1088, 4096, False),   # 256x256 tiles, 17 steps of 64: the six-step loop's five-step remainder
    (4096, 832, 4096, True),     # 256x256 tiles, 13 steps: a one-step remainder
    (2048, 1088, 6144, False),   # 256x192 tiles (the same six-step loop), 17 steps
    (2048, 4160, 4096, True),    # 256x128 tiles, 65 steps of 64: the three-step loop's two-step remainder
    (2048, 4224, 4096, True),    # 256x128 tiles, 66 steps: no remainder (4096 deep, 64 steps, leaves one)
])
def test_gemm_odd_step_count(m, k, n, resid):
    """The main loop runs a whole number of turns of its rings a trip (six 64-deep steps for 256x256
    and 256x192 tiles, whose rings hold three A and two B stages; three for 256x128), so a step count that is
    not a multiple ends on remainder steps, which must still read the right slots and drain the DMA
    stream."""
    std = 1.0 / 64.0
    got, want = run_gemm(m, k, n, 1, std, std, resid)
    assert_close(got, want, RTOL, ATOL * rms(want), f"gemm {m}x{k}x{n}")


def test_gemm_swiglu_odd_step_count():
    """The SwiGLU-fused GEMM with K = 1088 (17 steps of 64: a remainder of five) equals the GEMM +
    silu_mul pair."""
    a = randn((2048, 1088), 43, std=1 / 16).to(DEV)
    b = randn((1088, 2 * 6144), 44, std=1 / 4).to(DEV)
    fused = ops.gemm_swiglu(a, b).cpu()
    pair = ops.silu_mul(ops.gemm(a, b, split_k=False)).cpu()
    assert bits_equal(fused, pair)


def test_gemm_swiglu_every_bf16_gate():
    """The SwiGLU epilogue's quotient g / (1 + e^-g) against silu_mul's IEEE division for every bf16
    gate value.  A = I (256 x 256) makes the gate accumulators B's gate columns, which hold the 65280
    finite bf16 bit patterns (subnormals included) in columns 0-254 and the 256 infinities and NaNs
    in column 255 (whose products with A's zeros make that column NaN); -0 becomes +0 in an
    accumulator.  A second call, A = 2^-8 I, puts +inf and -inf alone in row 0 and reaches a -0 gate
    (a subnormal product that rounds to -0 in bf16).  Bit-equal to GEMM + silu_mul, NaN for NaN."""
    n = 256

    def check(ad, bd):
        fused = ops.gemm_swiglu(ad, bd).cpu()
        g = ops.gemm(ad, bd, split_k=False)
        pair = ops.silu_mul(g).cpu()
        nan_f, nan_p = torch.isnan(fused.float()), torch.isnan(pair.float())
        assert torch.equal(nan_f, nan_p)
        assert bits_equal(fused[~nan_f], pair[~nan_p])
        return g.cpu()[:, :n], nan_f

    pats = torch.arange(65536, dtype=torch.int32)
    special = ((pats >> 7) & 0xFF) == 0xFF
    # gate[k, j] = pattern j*256 + k of the finite ones, then the specials: column 255
    vals = torch.cat([pats[~special], pats[special]]).to(torch.int16)
    gate = vals.view(torch.bfloat16).reshape(n, n).t().contiguous()
    b = torch.cat([gate, randn((n, n), 45, std=1.0)], dim=1)          # B [K = 256, 2I = 512]: gate | up
    a = torch.eye(n, dtype=torch.bfloat16)
    g, nan_f = check(a.to(DEV), b.to(DEV))
    want = b[:, :255].clone()
    want[want.view(torch.int16) == -32768] = 0.0                          # -0 accumulates to +0
    assert bits_equal(g[:, :255], want), "the gate accumulators are B's finite gate values"
    assert nan_f[:, 255].all() and not nan_f[:, :255].any()
    b2 = torch.ones((n, 2 * n), dtype=torch.bfloat16)
    b2[0, 0], b2[0, 1] = float("inf"), float("-inf")
    b2[0, 2], b2[0, 3] = -(2.0 ** -133), 2.0 ** -133                      # products +-2^-141: bf16 -0, +0
    g2, _ = check((a * 2.0 ** -8).to(DEV), b2.to(DEV))
    assert g2[0, 0].item() == float("inf") and g2[0, 1].item() == float("-inf")
    # -0 is reached unless the matrix cores flush the subnormal product, in which case no gate is -0
    assert int(g2[0:1, 2].view(torch.int16)) in (-32768, 0) and int(g2[0:1, 3].view(torch.int16)) == 0


def test_gemm_swiglu_refusals():
    a = torch.zeros((64, 128), dtype=torch.bfloat16, device=DEV)
    b = torch.zeros((128, 2 * 192), dtype=torch.bfloat16, device=DEV)     # inter = 192: not a multiple of 128
    with pytest.raises(_lib.UnsupportedError):
        ops.gemm_swiglu(a, b)




def test_quant_rows_extreme_rows_exact():
    """Rows across the scale range, bit-exact with the oracle's torch cast: a tiny row (absmax below
    2^-100, the exact-division path), rows near that bound, a huge one, -0 and bf16 subnormals, a row
    holding a NaN (torch's absmax is NaN, so the scale is 1), infinities, and ordinary rows; wave-per-row
    (256 columns) and block-per-row (12288 columns) kernels."""
    for cols in (256, 12288):
        x = randn((12, cols), 70 + cols)
        x[0] *= 1e-33                         # absmax ~ 4e-33: below 2^-100 (7.9e-31)
        x[1] *= 2.0 ** -100                   # around the bound
        x[2] *= 1e37                          # huge but finite
        x[3, :] = -0.0
        x[3, 1] = 1.0
        x[4, ::2] = torch.tensor(1e-40, dtype=torch.bfloat16)   # subnormal bf16 beside normal values
        x[5, 7] = float("nan")
        x[6, 3] = float("inf")
        x[7, 5] = float("-inf")
        xq, sc = ops.quant_rows_e4m3(x.to(DEV))
        wq, wsc = oracle.quant_rows_e4m3(x)
        assert bits_equal(sc.cpu(), wsc), f"scales differ at {cols} columns"
        got, want = xq.cpu().view(torch.uint8), wq.view(torch.uint8)
        # inf / inf (the infinite rows) is a NaN whose sign is the platform's (x86 makes it negative,
        # the GPU positive): NaN bytes compare as NaN, every other byte bit for bit
        nan_w = (want & 0x7F) == 0x7F
        assert torch.equal((got & 0x7F) == 0x7F, nan_w), f"NaN positions differ at {cols} columns"
        assert torch.equal(got[~nan_w], want[~nan_w]), f"quantised bytes differ at {cols} columns"
        assert torch.equal(got[:6], want[:6]), f"finite rows differ at {cols} columns"
