"""ctypes binding of ``libptb_amd.so`` (the C ABI in ``include/ptb_amd.h``).

The library is loaded from ``ptb_amd/lib/`` inside the source tree.  There is no fallback: if the
library is missing, every entry point raises :class:`LibraryMissing`, so a GPU run can never pass
on anything but the HIP kernels.
"""
from __future__ import annotations

import ctypes
import threading
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "lib" / "libptb_amd.so"

PTB_OK = 0
PTB_ERR_NULL = -1
PTB_ERR_SHAPE = -2
PTB_ERR_ALIGN = -3
PTB_ERR_DTYPE = -4
PTB_ERR_UNSUPPORTED = -5
PTB_ERR_GRID = -6
PTB_ERR_WORKSPACE = -7

PTB_DTYPE_BF16 = 0
PTB_DTYPE_F32 = 1
PTB_DTYPE_I32 = 2
PTB_DTYPE_I64 = 3
PTB_DTYPE_E4M3 = 4
PTB_ROLE_IN = 0
PTB_ROLE_OUT = 1
PTB_ROLE_INOUT = 2
PTB_REDUCE_SUM = 0
PTB_REDUCE_MAX = 1


class PtbError(RuntimeError):
    """A status the library returned: negative = refused before launch, positive = hipError_t."""

    def __init__(self, fn: str, status: int, text: str):
        super().__init__(f"{fn}: status {status} ({text})")
        self.fn = fn
        self.status = status


class ShapeError(PtbError, ValueError):
    pass


class AlignmentError(PtbError, ValueError):
    pass


class UnsupportedError(PtbError, ValueError):
    pass


class GridError(PtbError, ValueError):
    pass


class HipError(PtbError):
    pass


class LibraryMissing(RuntimeError):
    pass


_ERR_CLASS = {
    PTB_ERR_SHAPE: ShapeError,
    PTB_ERR_ALIGN: AlignmentError,
    PTB_ERR_UNSUPPORTED: UnsupportedError,
    PTB_ERR_GRID: GridError,
}

_c_int, _c_i64, _c_f32, _vp, _c_size = ctypes.c_int, ctypes.c_int64, ctypes.c_float, ctypes.c_void_p, ctypes.c_size_t


class PtbTensor(ctypes.Structure):
    """ptb_tensor: the reference's memref descriptor (codegen/wrapper.py:140-146) plus dtype and role."""
    _fields_ = [("allocated", ctypes.c_void_p), ("aligned", ctypes.c_void_p), ("offset", ctypes.c_int64),
                ("size", ctypes.c_int64), ("stride", ctypes.c_int64), ("dtype", ctypes.c_int32),
                ("role", ctypes.c_int32)]


_ARGS_SIG = (ctypes.c_int, [ctypes.POINTER(PtbTensor), ctypes.c_int, ctypes.POINTER(ctypes.c_int64), ctypes.c_int,
                            ctypes.POINTER(ctypes.c_double), ctypes.c_int, ctypes.POINTER(ctypes.c_int32),
                            ctypes.c_void_p])
ARGS_FAMILIES = ("rmsnorm", "softmax", "silu_mul", "gemm", "flash_attn", "attn_decode", "qk_norm_rope",
                 "transpose_heads", "sumsq", "gemv", "reduce", "add_scalar", "slice_add")

# name -> (restype, argtypes), mirroring include/ptb_amd.h
SIGNATURES = {
    "ptb_abi_version": (_c_int, []),
    "ptb_status_string": (ctypes.c_char_p, [_c_int]),
    "ptb_rmsnorm_bf16": (_c_int, [_vp, _vp, _c_int, _vp, _c_i64, _c_i64, _c_f32, _vp]),
    "ptb_softmax_rows_bf16": (_c_int, [_vp, _vp, _c_i64, _c_i64, _vp]),
    "ptb_softmax_rows_bf16_f32": (_c_int, [_vp, _vp, _c_i64, _c_i64, _vp]),
    "ptb_silu_mul_bf16": (_c_int, [_vp, _vp, _c_i64, _c_i64, _vp]),
    "ptb_transpose_heads_bf16": (_c_int, [_vp, _vp, _c_i64, _c_i64, _c_i64, _vp]),
    "ptb_qk_norm_rope_bf16": (_c_int, [_vp, _vp, _vp, _vp, _vp, _c_i64, _c_i64, _c_i64, _c_f32, _vp]),
    "ptb_transpose_heads_ld_bf16": (_c_int, [_vp, _c_i64, _vp, _c_i64, _c_i64, _c_i64, _vp]),
    "ptb_qk_norm_rope_ld_bf16": (_c_int, [_vp, _c_i64, _vp, _vp, _vp, _vp, _c_i64, _c_i64, _c_i64, _c_f32, _vp]),
    "ptb_reduce_workspace_bytes": (_c_size, [_c_i64]),
    "ptb_reduce_bf16": (_c_int, [_vp, _vp, _c_i64, _c_int, _vp, _c_size, _vp]),
    "ptb_reduce_f32": (_c_int, [_vp, _vp, _c_i64, _c_int, _vp, _c_size, _vp]),
    "ptb_add_scalar_bf16": (_c_int, [_vp, _vp, _c_i64, _c_f32, _vp]),
    "ptb_slice_add_bf16": (_c_int, [_vp, _vp, _c_i64, _c_i64, _c_f32, _vp]),
    "ptb_gemm_bf16": (_c_int, [_vp, _vp, _vp, _vp, _c_i64, _c_i64, _c_i64, _vp]),
    "ptb_gemm_bf16_workspace_bytes": (_c_size, [_c_i64, _c_i64, _c_i64]),
    "ptb_gemm_bf16_ws": (_c_int, [_vp, _vp, _vp, _vp, _c_i64, _c_i64, _c_i64, _vp, _c_size, _vp]),
    "ptb_gemm_swiglu_bf16": (_c_int, [_vp, _vp, _vp, _c_i64, _c_i64, _c_i64, _vp]),
    "ptb_quant_rows_e4m3": (_c_int, [_vp, _vp, _vp, _c_i64, _c_i64, _vp]),
    "ptb_quant_weight_e4m3": (_c_int, [_vp, _vp, _vp, _c_i64, _c_i64, _vp]),
    "ptb_gemm_fp8_scaled": (_c_int, [_vp, _vp, _vp, _vp, _vp, _c_i64, _c_i64, _c_i64, _vp]),
    "ptb_rmsnorm_f32": (_c_int, [_vp, _vp, _vp, _c_i64, _c_i64, _c_f32, _vp]),
    "ptb_col_rms_f32": (_c_int, [_vp, _vp, _c_i64, _c_i64, _c_f32, _vp]),
    "ptb_softmax_rows_f32": (_c_int, [_vp, _vp, _c_i64, _c_i64, _vp]),
    "ptb_silu_mul_f32": (_c_int, [_vp, _vp, _c_i64, _c_i64, _vp]),
    "ptb_swiglu_f32": (_c_int, [_vp, _vp, _vp, _vp, _c_i64, _c_i64, _c_i64, _vp]),
    "ptb_flash_attn_fwd_bf16": (_c_int, [_vp, _vp, _vp, _vp, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_f32,
                                         _c_int, _vp]),
    "ptb_flash_attn_fwd_tokens_bf16": (_c_int, [_vp, _vp, _vp, _vp, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_f32,
                                         _c_int, _vp]),
    "ptb_flash_attn_fwd_qkv_bf16": (_c_int, [_vp, _c_i64, _vp, _vp, _vp, _vp, _c_f32, _vp, _c_i64, _c_i64, _c_i64,
                                             _c_i64, _c_i64, _c_f32, _c_int, _vp]),
    "ptb_sumsq_bf16": (_c_int, [_vp, _vp, _vp, _c_i64, _vp]),
    "ptb_gemv_workspace_bytes": (_c_size, [_c_i64, _c_i64]),
    "ptb_gemv_bf16": (_c_int, [_vp, _vp, _vp, _c_i64, _c_i64, _vp, _c_size, _vp]),
    "ptb_gemv_rmsnorm_bf16": (_c_int, [_vp, _vp, _vp, _vp, _c_f32, _vp, _vp, _c_i64, _c_i64, _vp, _c_size, _vp]),
    "ptb_gemv_silu_bf16": (_c_int, [_vp, _vp, _vp, _vp, _vp, _c_i64, _c_i64, _vp, _c_size, _vp]),
    "ptb_gemv_rmsnorm_parts_bf16": (_c_int, [_vp, _vp, _vp, _vp, _c_f32, _vp, _vp, _c_i64, _c_i64, _c_size, _vp]),
    "ptb_gemv_silu_parts_bf16": (_c_int, [_vp, _c_i64, _vp, _vp, _vp, _vp, _c_i64, _c_i64, _vp, _c_size, _vp]),
    "ptb_fill_zero": (_c_int, [_vp, _c_i64, _vp]),
    "ptb_cast_i64_i32": (_c_int, [_vp, _vp, _c_i64, _vp]),
    "ptb_cumsum_int": (_c_int, [_vp, _c_int, _vp, _vp, _c_int, _c_i64, _vp]),
    "ptb_moe_group_table": (_c_int, [_vp, _c_int, _c_i64, _vp, _vp, _vp, _vp]),
    "ptb_count_le": (_c_int, [_vp, _c_i64, _vp, _c_i64, _vp]),
    "ptb_moe_expert_count": (_c_int, [_vp, _c_i64, _c_i64, _vp, _vp, _vp, _vp]),
    "ptb_moe_rank_select": (_c_int, [_vp, _vp, _c_i64, _c_i64, _vp, _vp]),
    "ptb_sort_workspace_bytes": (_c_size, [_c_i64, _c_i64]),
    "ptb_sort_rows": (_c_int, [_vp, _c_int, _vp, _vp, _c_i64, _c_i64, _c_int, _vp, _c_size, _vp]),
    "ptb_topk_rows_f32": (_c_int, [_vp, _c_i64, _c_i64, _c_i64, _c_int, _vp, _vp, _vp]),
    "ptb_moe_gather_rows_bf16": (_c_int, [_vp, _c_i64, _c_i64, _vp, _c_i64, _c_i64, _vp, _vp]),
    "ptb_moe_combine_bf16": (_c_int, [_vp, _vp, _vp, _vp, _vp, _c_i64, _vp, _c_int, _vp, _vp, _vp, _c_i64, _c_i64,
                                      _c_i64, _c_i64, _vp]),
    "ptb_normalize_rows_f32": (_c_int, [_vp, _c_i64, _c_i64, _vp, _vp, _vp]),
    "ptb_add_bf16": (_c_int, [_vp, _vp, _vp, _c_i64, _vp]),
    "ptb_rope_bf16": (_c_int, [_vp, _vp, _vp, _vp, _c_i64, _c_i64, _c_i64, _vp]),
    "ptb_rmsnorm_add_bf16": (_c_int, [_vp, _vp, _vp, _vp, _c_i64, _c_i64, _c_f32, _vp]),
    "ptb_rms_broadcast_bf16": (_c_int, [_vp, _vp, _vp, _vp, _vp, _c_i64, _c_i64, _c_f32, _vp]),
    "ptb_grouped_gemm_bf16": (_c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
                                       _c_i64, _vp]),
    "ptb_grouped_gemm_workspace_bytes": (_c_size, [_c_i64, _c_i64, _c_i64, _c_i64]),
    "ptb_grouped_gemm_bf16_ws": (_c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
                                          _c_i64, _vp, _c_size, _vp]),
    "ptb_attn_decode_workspace_bytes": (_c_size, [_c_i64, _c_i64, _c_i64]),
    "ptb_attn_decode_bf16": (_c_int, [_vp, _vp, _vp, _vp, _c_i64, _c_i64, _c_i64, _c_i64, _c_f32, _vp, _c_size,
                                      _vp]),
    "ptb_attn_decode_noalloc_max_bytes": (_c_size, []),
    "ptb_attn_decode_bf16_noalloc": (_c_int, [_vp, _vp, _vp, _vp, _c_i64, _c_i64, _c_i64, _c_i64, _c_f32, _vp]),
    "ptb_attn_decode_qnorm_rope_bf16": (_c_int, [_vp, _vp, _vp, _vp, _c_f32, _vp, _vp, _vp, _c_i64, _c_i64, _c_i64,
                                                 _c_i64, _c_f32, _vp, _c_size, _vp]),
}
SIGNATURES.update({f"ptb_{fam}_args": _ARGS_SIG for fam in ARGS_FAMILIES})

_lock = threading.Lock()
_lib = None


def load(path: Path | str | None = None) -> ctypes.CDLL:
    """Load (once) and return the library with every declared signature bound."""
    global _lib
    with _lock:
        if _lib is not None and path is None:
            return _lib
        p = Path(path) if path else LIB_PATH
        if not p.exists():
            raise LibraryMissing(
                f"{p} is not built: run __graft_entry__.build() (or python -m ptb_amd.build); "
                "ptb_amd has no non-HIP fallback")
        # torch ships its own HIP runtime: load it first so the library binds to that one instance
        # (a second runtime loaded ahead of torch's sees no device once torch has claimed it)
        import torch  # noqa: F401

        lib = ctypes.CDLL(str(p))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        if path is None:
            _lib = lib
        return lib


def status_text(status: int) -> str:
    return load().ptb_status_string(status).decode()


def check(fn: str, status: int) -> None:
    """Raise the matching PtbError for a non-zero status."""
    if status == PTB_OK:
        return
    cls = _ERR_CLASS.get(status, HipError if status > 0 else PtbError)
    raise cls(fn, status, status_text(status))


def call(fn: str, *args) -> None:
    check(fn, getattr(load(), fn)(*args))
