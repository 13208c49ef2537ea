"""CPU tests of the C ABI: the library loads, exports every entry point include/ptb_amd.h
declares, and refuses bad arguments with the documented status codes before touching a GPU."""
import ctypes
import re
import subprocess
from pathlib import Path

import pytest

from ptb_amd import _lib

REPO = Path(__file__).resolve().parents[1]
HEADER = REPO / "include" / "ptb_amd.h"


def declared_functions():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(ptb_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    if not _lib.LIB_PATH.exists():
        from ptb_amd import build

        build.build()
    return _lib.load()


def test_header_declares_entry_points():
    names = declared_functions()
    assert "ptb_gemm_bf16" in names and "ptb_rmsnorm_bf16" in names
    assert len(names) >= 10


def test_every_declared_symbol_is_exported(lib):
    out = subprocess.run(["nm", "-D", "--defined-only", str(_lib.LIB_PATH)], capture_output=True, text=True,
                         check=True).stdout
    exported = set(re.findall(r"\bT (ptb_\w+)", out))
    missing = [n for n in declared_functions() if n not in exported]
    assert not missing, f"declared in ptb_amd.h but not exported: {missing}"
    for n in declared_functions():
        assert hasattr(lib, n)


def test_binding_covers_header():
    assert set(declared_functions()) == set(_lib.SIGNATURES), "ctypes signatures out of sync with the header"


def test_abi_version_and_status_text(lib):
    assert lib.ptb_abi_version() == 1
    assert lib.ptb_status_string(0) == b"ok"
    assert b"NULL" in lib.ptb_status_string(_lib.PTB_ERR_NULL)
    assert lib.ptb_status_string(-99) == b"unknown status"


# Argument checks run before any HIP call, so they are exercised here with host pointers.
BUF = ctypes.create_string_buffer(1 << 16)
P = ctypes.addressof(BUF)
P16 = (P + 15) & ~15


def test_null_pointers_refused(lib):
    assert lib.ptb_rmsnorm_bf16(None, P16, 0, P16, 4, 64, 1e-6, None) == _lib.PTB_ERR_NULL
    assert lib.ptb_gemm_bf16(P16, None, None, P16, 4, 64, 64, None) == _lib.PTB_ERR_NULL
    assert lib.ptb_softmax_rows_bf16(P16, None, 4, 64, None) == _lib.PTB_ERR_NULL
    assert lib.ptb_gemm_fp8_scaled(P16, P16, P16, None, P16, 4, 16, 128, None) == _lib.PTB_ERR_NULL
    assert lib.ptb_attn_decode_qnorm_rope_bf16(P16, None, P16, P16, 1e-6, P16, P16, P16, 8, 4, 64, 128, 0.1,
                                               None, 0, None) == _lib.PTB_ERR_NULL
    assert lib.ptb_attn_decode_qnorm_rope_bf16(P16, P16 + 2, P16, P16, 1e-6, P16, P16, P16, 8, 4, 64, 128, 0.1,
                                               None, 0, None) == _lib.PTB_ERR_ALIGN


def test_shape_and_alignment_refused(lib):
    assert lib.ptb_rmsnorm_bf16(P16, P16, 0, P16, -1, 64, 1e-6, None) == _lib.PTB_ERR_SHAPE
    assert lib.ptb_rmsnorm_bf16(P16, P16, 0, P16, 4, 12, 1e-6, None) == _lib.PTB_ERR_ALIGN
    assert lib.ptb_rmsnorm_bf16(P16 + 2, P16, 0, P16, 4, 64, 1e-6, None) == _lib.PTB_ERR_ALIGN
    assert lib.ptb_rmsnorm_bf16(P16, P16, 7, P16, 4, 64, 1e-6, None) == _lib.PTB_ERR_DTYPE
    assert lib.ptb_gemm_bf16(P16, P16, None, P16, 4, 64, 100, None) == _lib.PTB_ERR_UNSUPPORTED
    assert lib.ptb_gemm_bf16(P16, P16, None, P16, 4, 60, 64, None) == _lib.PTB_ERR_UNSUPPORTED
    assert lib.ptb_gemm_bf16(P16, P16, None, P16, -4, 64, 64, None) == _lib.PTB_ERR_SHAPE
    assert lib.ptb_gemm_fp8_scaled(P16, P16, P16, P16, P16, 4, 16, 64, None) == _lib.PTB_ERR_UNSUPPORTED
    assert lib.ptb_qk_norm_rope_bf16(P16, P16, P16, P16, P16, 4, 2, 64, 1e-6, None) == _lib.PTB_ERR_UNSUPPORTED
    assert lib.ptb_transpose_heads_bf16(P16, P16, 2, 3, 4, None) == _lib.PTB_ERR_ALIGN
    assert lib.ptb_transpose_heads_ld_bf16(P16, 100, P16, 2, 3, 128, None) == _lib.PTB_ERR_SHAPE   # ld < 3*128
    assert lib.ptb_qk_norm_rope_ld_bf16(P16, 4000, P16, P16, P16, P16, 4, 32, 128, 1e-6, None) == _lib.PTB_ERR_SHAPE
    assert lib.ptb_qk_norm_rope_ld_bf16(P16, 4100, P16, P16, P16, P16, 4, 32, 128, 1e-6, None) == _lib.PTB_ERR_ALIGN
    assert lib.ptb_reduce_bf16(P16, P16, 64, 5, P16, 4096, None) == _lib.PTB_ERR_DTYPE
    assert lib.ptb_reduce_bf16(P16, P16, 64, 0, P16, 4, None) == _lib.PTB_ERR_WORKSPACE


def test_32bit_buffer_offset_limits_refused(lib):
    """The kernels address each operand through a buffer resource with 32-bit byte offsets; shapes
    past that range are refused before any launch (PTB_ERR_UNSUPPORTED / PTB_ERR_GRID)."""
    # B (plus the DMA run-ahead) at or past 4 GiB: (65536 + 128) * 32768 * 2 bytes
    assert lib.ptb_gemm_bf16(P16, P16, None, P16, 256, 32768, 65536, None) == _lib.PTB_ERR_UNSUPPORTED
    assert lib.ptb_gemm_swiglu_bf16(P16, P16, P16, 256, 16384, 65536, None) == _lib.PTB_ERR_UNSUPPORTED
    # one 256-row panel of A at 4 GiB: 256 * 8388608 * 2 bytes
    assert lib.ptb_gemm_bf16(P16, P16, None, P16, 256, 8, 8388608, None) == _lib.PTB_ERR_UNSUPPORTED
    # C wider than 2^22 columns: a 256-row tile of it would pass 2^31 bytes of store offsets
    assert lib.ptb_gemm_bf16(P16, P16, None, P16, 256, (1 << 22) + 8, 64, None) == _lib.PTB_ERR_UNSUPPORTED
    assert lib.ptb_gemm_swiglu_bf16(P16, P16, P16, 256, (1 << 21) + 128, 64, None) == _lib.PTB_ERR_UNSUPPORTED
    assert lib.ptb_gemm_fp8_scaled(P16, P16, P16, P16, P16, 256, (1 << 22) + 16, 128, None) == _lib.PTB_ERR_UNSUPPORTED
    # fp8: a 256-row panel of e4m3 A at 4 GiB
    assert lib.ptb_gemm_fp8_scaled(P16, P16, P16, P16, P16, 256, 16, 1 << 24, None) == _lib.PTB_ERR_UNSUPPORTED
    # attention: one kv head's K at 4 GiB (2^24 keys x 256 bytes)
    assert lib.ptb_flash_attn_fwd_bf16(P16, P16, P16, P16, 1, 1, 1, 1 << 24, 128, 0.1, 1, None) == _lib.PTB_ERR_GRID
    # decode attention: caches of 2^30 keys or more (the kernels' 32-bit key indices); no workspace
    # is quoted for them
    assert lib.ptb_attn_decode_workspace_bytes(1, 4, 1 << 30) == 0
    assert lib.ptb_attn_decode_bf16(P16, P16, P16, P16, 1, 4, 1 << 30, 128, 0.1, P16, 1 << 20, None) == _lib.PTB_ERR_GRID
    assert lib.ptb_attn_decode_workspace_bytes(1, 4, (1 << 30) - 1) > 0


def test_gemv_parts_refusals(lib):
    """The split gate/up + down pair refuses missing partials, a residual pair without its first
    half and a producer K that cannot be, before any launch."""
    assert lib.ptb_gemv_rmsnorm_parts_bf16(P16, None, P16, P16, 1e-6, P16, None, 64, 64, 1 << 20, None) == \
        _lib.PTB_ERR_NULL
    assert lib.ptb_gemv_silu_parts_bf16(None, 64, P16, None, None, P16, 64, 64, P16, 1 << 20, None) == _lib.PTB_ERR_NULL
    assert lib.ptb_gemv_silu_parts_bf16(P16, 64, P16, None, P16, P16, 64, 64, P16, 1 << 20, None) == _lib.PTB_ERR_NULL
    assert lib.ptb_gemv_silu_parts_bf16(P16, 0, P16, None, None, P16, 64, 64, P16, 1 << 20, None) == _lib.PTB_ERR_SHAPE
    assert lib.ptb_gemv_silu_parts_bf16(P16, 64, P16, None, None, P16, 64, 12, P16, 1 << 20, None) == \
        _lib.PTB_ERR_UNSUPPORTED   # n % 8 != 0


def test_fused_attention_refusals(lib):
    # ld narrower than q|k|v; a missing q-norm weight; a row stride that breaks 16-byte rows
    assert lib.ptb_flash_attn_fwd_qkv_bf16(P16, 1000, P16, P16, P16, P16, 1e-6, P16, 1, 4, 2, 128, 128, 0.1, 1,
                                           None) == _lib.PTB_ERR_SHAPE
    assert lib.ptb_flash_attn_fwd_qkv_bf16(P16, 1024, P16, None, P16, P16, 1e-6, P16, 1, 4, 2, 128, 128, 0.1, 1,
                                           None) == _lib.PTB_ERR_NULL
    assert lib.ptb_flash_attn_fwd_qkv_bf16(P16, 1028, P16, P16, P16, P16, 1e-6, P16, 1, 4, 2, 128, 128, 0.1, 1,
                                           None) == _lib.PTB_ERR_ALIGN


def test_empty_work_is_a_no_op(lib):
    # zero rows / zero-size outputs return OK without launching
    assert lib.ptb_rmsnorm_bf16(P16, P16, 0, P16, 0, 64, 1e-6, None) == _lib.PTB_OK
    assert lib.ptb_gemm_bf16(P16, P16, None, P16, 0, 64, 64, None) == _lib.PTB_OK
    assert lib.ptb_silu_mul_bf16(P16, P16, 0, 64, None) == _lib.PTB_OK


def test_error_mapping():
    with pytest.raises(_lib.ShapeError):
        _lib.check("f", _lib.PTB_ERR_SHAPE)
    with pytest.raises(_lib.UnsupportedError):
        _lib.check("f", _lib.PTB_ERR_UNSUPPORTED)
    with pytest.raises(_lib.HipError):
        _lib.check("f", 1)
    _lib.check("f", 0)


def test_missing_library_fails_loudly(tmp_path):
    with pytest.raises(_lib.LibraryMissing):
        _lib.load(tmp_path / "nope.so")


# ---- spec-driven entries (ptb_<family>_args): refusals happen before any HIP call
def _desc(n, dtype=_lib.PTB_DTYPE_BF16, role=_lib.PTB_ROLE_IN, stride=1, ptr=None):
    p = P16 if ptr is None else ptr
    return _lib.PtbTensor(p, p, 0, n, stride, dtype, role)


def _call(lib, fam, descs, ints, floats, grid):
    arr = (_lib.PtbTensor * max(len(descs), 1))(*descs)
    iv = (ctypes.c_int64 * max(len(ints), 1))(*ints)
    fv = (ctypes.c_double * max(len(floats), 1))(*floats)
    gv = (ctypes.c_int32 * 3)(*grid)
    return getattr(lib, f"ptb_{fam}_args")(arr, len(descs), iv, len(ints), fv, len(floats), gv, None)


def test_args_entries_refuse_bad_calls(lib):
    rows, cols, programs = 16, 64, 4
    x, w = _desc(rows * cols), _desc(cols)
    y = _desc(rows * cols, role=_lib.PTB_ROLE_OUT)
    ok_args = [x, w, y]
    # wrong counts
    assert _call(lib, "rmsnorm", ok_args[:2], [rows, cols, programs], [1e-6], (4, 1, 1)) == _lib.PTB_ERR_SHAPE
    assert _call(lib, "rmsnorm", ok_args, [rows, cols], [1e-6], (4, 1, 1)) == _lib.PTB_ERR_SHAPE
    assert _call(lib, "rmsnorm", ok_args, [rows, cols, programs], [], (4, 1, 1)) == _lib.PTB_ERR_SHAPE
    # a size that disagrees with the parameters
    bad = [x, _desc(cols + 1), y]
    assert _call(lib, "rmsnorm", bad, [rows, cols, programs], [1e-6], (4, 1, 1)) == _lib.PTB_ERR_SHAPE
    # the grid past the program bound, below 1, or off the x axis
    assert _call(lib, "rmsnorm", ok_args, [rows, cols, programs], [1e-6], (5, 1, 1)) == _lib.PTB_ERR_GRID
    assert _call(lib, "rmsnorm", ok_args, [rows, cols, programs], [1e-6], (0, 1, 1)) == _lib.PTB_ERR_GRID
    assert _call(lib, "rmsnorm", ok_args, [rows, cols, programs], [1e-6], (4, 2, 1)) == _lib.PTB_ERR_GRID
    # a written tensor declared read-only, an unknown dtype, a strided tensor
    ro = [x, w, _desc(rows * cols)]
    assert _call(lib, "rmsnorm", ro, [rows, cols, programs], [1e-6], (4, 1, 1)) == _lib.PTB_ERR_SHAPE
    assert _call(lib, "rmsnorm", [x, _desc(cols, dtype=9), y], [rows, cols, programs], [1e-6],
                 (4, 1, 1)) == _lib.PTB_ERR_DTYPE
    assert _call(lib, "rmsnorm", [x, w, _desc(rows * cols, role=1, stride=2)], [rows, cols, programs], [1e-6],
                 (4, 1, 1)) == _lib.PTB_ERR_UNSUPPORTED
    # GEMM: M*K, K*N, M*N must agree; only the whole grid runs
    m, n, k = 64, 128, 64
    a, b, c = _desc(m * k), _desc(k * n), _desc(m * n, role=_lib.PTB_ROLE_OUT)
    assert _call(lib, "gemm", [a, b, _desc(m * n + 8, role=1)], [m, n, k, 2], [], (2, 1, 1)) == _lib.PTB_ERR_SHAPE
    assert _call(lib, "gemm", [a, b, c], [m, n, k, 2], [], (3, 1, 1)) == _lib.PTB_ERR_GRID
    assert _call(lib, "gemm", [a, b, c], [m, n, k, 2], [], (1, 1, 1)) == _lib.PTB_ERR_UNSUPPORTED
    # attention: one program per (batch, query head); a partial grid must cover whole batches
    q, kk = _desc(4 * 128 * 128), _desc(2 * 128 * 128)
    o = _desc(4 * 128 * 128, role=_lib.PTB_ROLE_INOUT)
    ints = [1, 4, 2, 128, 128, 1]
    assert _call(lib, "flash_attn", [q, kk, kk, o], ints, [0.088], (5, 1, 1)) == _lib.PTB_ERR_GRID
    assert _call(lib, "flash_attn", [q, kk, kk, o], ints, [0.088], (3, 1, 1)) == _lib.PTB_ERR_UNSUPPORTED
    assert _call(lib, "flash_attn", [q, kk, kk], ints, [0.088], (4, 1, 1)) == _lib.PTB_ERR_SHAPE
    # silu_mul: a partial grid has to end on a whole row
    gu, out = _desc(2 * 4 * 256), _desc(4 * 256, role=_lib.PTB_ROLE_OUT)
    assert _call(lib, "silu_mul", [gu, out], [4, 256, 8], [], (3, 1, 1)) == _lib.PTB_ERR_UNSUPPORTED


def test_args_entries_refuse_bad_calls_more_families(lib):
    f32, i64, outr = _lib.PTB_DTYPE_F32, _lib.PTB_DTYPE_I64, _lib.PTB_ROLE_OUT
    # rmsnorm's fp32 column arm: only with fp32 tensors, c of cols elements
    x32, w32 = _desc(16 * 64, dtype=f32), _desc(64, dtype=f32)
    y32 = _desc(16 * 64, dtype=f32, role=outr)
    assert _call(lib, "rmsnorm", [x32, w32, y32, _desc(63, dtype=f32, role=outr)], [16, 64, 1], [1e-5],
                 (1, 1, 1)) == _lib.PTB_ERR_SHAPE
    assert _call(lib, "rmsnorm", [x32, w32, y32, _desc(64, dtype=f32)], [16, 64, 1], [1e-5],
                 (1, 1, 1)) == _lib.PTB_ERR_SHAPE                       # c declared read-only
    assert _call(lib, "rmsnorm", [_desc(16 * 64), _desc(64), _desc(16 * 64, role=outr),
                                  _desc(64, dtype=f32, role=outr)], [16, 64, 1], [1e-5], (1, 1, 1)) == _lib.PTB_ERR_DTYPE
    # sumsq: one fp32 output, bf16 inputs of n, the whole grid
    one = _desc(1, dtype=f32, role=outr)
    assert _call(lib, "sumsq", [_desc(64), one], [64, 1], [], (2, 1, 1)) == _lib.PTB_ERR_GRID
    assert _call(lib, "sumsq", [_desc(64), _desc(63), one], [64, 1], [], (1, 1, 1)) == _lib.PTB_ERR_SHAPE
    assert _call(lib, "sumsq", [_desc(64), _desc(1, role=outr)], [64, 1], [], (1, 1, 1)) == _lib.PTB_ERR_DTYPE
    # gemv: the layout its mode and extra count name, sizes against k and n
    k, n = 64, 128
    x, w, y = _desc(k), _desc(k * n), _desc(n, role=outr)
    ss, g = _desc(1, dtype=f32), _desc(k)
    assert _call(lib, "gemv", [x, w, y], [3, k, n, 0, 1], [], (1, 1, 1)) == _lib.PTB_ERR_UNSUPPORTED
    assert _call(lib, "gemv", [x, w, y], [0, k, n, 1, 1], [], (1, 1, 1)) == _lib.PTB_ERR_UNSUPPORTED
    assert _call(lib, "gemv", [x, _desc(k * n + 8), y], [0, k, n, 0, 1], [], (1, 1, 1)) == _lib.PTB_ERR_SHAPE
    assert _call(lib, "gemv", [x, ss, g, w, y], [1, k, n, 0, 1], [], (1, 1, 1)) == _lib.PTB_ERR_SHAPE   # no eps
    assert _call(lib, "gemv", [x, g, g, w, y], [1, k, n, 0, 1], [1e-6], (1, 1, 1)) == _lib.PTB_ERR_SHAPE
    assert _call(lib, "gemv", [_desc(2 * k), w, _desc(n + 8), y], [2, k, n, 1, 1], [], (1, 1, 1)) == _lib.PTB_ERR_SHAPE
    assert _call(lib, "gemv", [x, w, y], [0, k, n, 0, 1], [], (2, 1, 1)) == _lib.PTB_ERR_GRID
    assert _call(lib, "gemv", [x, w, y, _desc(8, role=_lib.PTB_ROLE_IN)], [0, k, n, 0, 1], [],
                 (1, 1, 1)) == _lib.PTB_ERR_SHAPE                        # a read-only workspace
    # reduce: a known op, one fp32 output
    assert _call(lib, "reduce", [_desc(64), one], [64, 2, 1], [], (1, 1, 1)) == _lib.PTB_ERR_UNSUPPORTED
    assert _call(lib, "reduce", [_desc(64), _desc(2, dtype=f32, role=outr)], [64, 0, 1], [], (1, 1, 1)) == \
        _lib.PTB_ERR_SHAPE
    assert _call(lib, "reduce", [_desc(64, dtype=i64), one], [64, 0, 1], [], (1, 1, 1)) == _lib.PTB_ERR_DTYPE
    # add_scalar: one float, matching sizes; slice_add: the slice inside x
    assert _call(lib, "add_scalar", [_desc(64), _desc(64, role=outr)], [64, 1], [], (1, 1, 1)) == _lib.PTB_ERR_SHAPE
    assert _call(lib, "add_scalar", [_desc(64), _desc(64, role=outr)], [64, 2], [1.0], (3, 1, 1)) == _lib.PTB_ERR_GRID
    assert _call(lib, "slice_add", [_desc(64), _desc(8, dtype=f32, role=outr)], [60, 8, 1], [1.0], (1, 1, 1)) == \
        _lib.PTB_ERR_SHAPE
    assert _call(lib, "slice_add", [_desc(64), _desc(8, role=outr)], [0, 8, 1], [1.0], (1, 1, 1)) == _lib.PTB_ERR_DTYPE
