"""ptb_amd -- MI355X (gfx950) execution of PSAL-POSTECH/PyTorchSim-Triton-Backend's hot-path kernels.

Hand-written HIP kernels behind the C ABI in ``include/ptb_amd.h`` (``libptb_amd.so``), with the
reference's operator contract on top: kernel specs and args (:mod:`ptb_amd.contract`), the
launcher hook (:mod:`ptb_amd.launcher`), verify semantics (:mod:`ptb_amd.verify`), the Qwen3-8B
layer (:mod:`ptb_amd.qwen3`) and the validation-suite entry points (:mod:`ptb_amd.validation`).
"""
from . import _lib  # noqa: F401
from ._lib import (AlignmentError, GridError, HipError, LibraryMissing, PtbError,  # noqa: F401
                   ShapeError, UnsupportedError)

__version__ = "0.1.0"
