"""The launch hooks the reference's callers use, served by the HIP kernels.

* ``launch(spec_or_manifest, tensors, grid=None, source=None)`` -- run one kernel over device
  tensors keyed by argument name (or given in argument order).
* ``hip_launcher(binary, kernel_object, grid, args, artifacts=None)`` -- a callable with the
  signature PyTorchSim registers through ``pytorchsim_triton_backend.driver.set_launcher``
  (reference: pytorchsim_triton_compiler/triton_extension/python/pytorchsim_triton_backend/
  driver.py:86-100): ``binary`` (the compiled ELF) is not needed here; ``kernel_object`` is the
  kernel.json text or dict; ``args`` are the call's arguments with constexprs dropped, tensors
  first in argument order, then the runtime scalars.
* ``set_launcher`` / ``registered_launcher`` mirror the reference's registry (driver.py:86-100):
  with nothing registered, a launch raises ``RuntimeError`` as the reference's driver does.

The whole grid is one HIP launch: the reference's per-program loop (codegen/wrapper.py:254-265)
has no counterpart, so ``grid`` only has to name the grid the kernel was built for.
"""
from __future__ import annotations

import json

from . import kernels
from .contract import KernelSpec, spec_from_manifest


class GridMismatch(ValueError):
    pass


def _as_spec(obj) -> KernelSpec:
    if isinstance(obj, KernelSpec):
        return obj
    if isinstance(obj, (str, bytes)):
        obj = json.loads(obj)
    return spec_from_manifest(obj)


def _check_tensors(spec: KernelSpec, tensors: dict) -> None:
    import torch

    for a in spec.args:
        if a.name not in tensors:
            raise ValueError(f"{spec.name}: no tensor for argument {a.name}")
        t = tensors[a.name]
        if not isinstance(t, torch.Tensor) or t.device.type != "cuda":
            raise ValueError(f"{spec.name}: argument {a.name} must be a GPU tensor")
        if t.numel() != a.numel:
            raise ValueError(f"{spec.name}: argument {a.name} has {t.numel()} elements, the spec says {a.numel}")
        want = getattr(torch, a.dtype)
        if t.dtype != want:
            raise TypeError(f"{spec.name}: argument {a.name} is {t.dtype}, the spec says {a.dtype}")
        if not t.is_contiguous():
            raise ValueError(f"{spec.name}: argument {a.name} must be contiguous")


def launch(spec_or_manifest, tensors, grid=None, source: str | None = None) -> kernels.Plan:
    """Run one reference kernel on the GPU (asynchronously, on the current stream)."""
    spec = _as_spec(spec_or_manifest)
    if not isinstance(tensors, dict):
        tensors = {a.name: t for a, t in zip(spec.args, tensors)}
    if grid is not None:
        g = tuple(int(x) for x in grid) + (1,) * (3 - len(tuple(grid)))
        want = tuple(spec.grid) + (1,) * (3 - len(spec.grid))
        if g != want:
            raise GridMismatch(f"{spec.name}: launched with grid {g}, built for {want}")
    _check_tensors(spec, tensors)
    return kernels.launch(spec, {a.name: tensors[a.name].view(-1) for a in spec.args}, source)


def hip_launcher(binary, kernel_object, grid, args, artifacts=None):
    """set_launcher-compatible entry: run the kernel object's kernel over `args` on the GPU."""
    spec = _as_spec(kernel_object)
    ko = json.loads(kernel_object) if isinstance(kernel_object, (str, bytes)) else dict(kernel_object)
    tensors = list(args)[: len(spec.args)]
    source = ko.get("source")
    return launch(spec, tensors, grid=grid, source=source)


_LAUNCHER = None


def set_launcher(fn) -> None:
    """Register the function that runs a compiled kernel (None unregisters)."""
    global _LAUNCHER
    _LAUNCHER = fn


def registered_launcher():
    if _LAUNCHER is None:
        raise RuntimeError("no launcher is registered: register one with ptb_amd.launcher.set_launcher "
                           "(ptb_amd.launcher.hip_launcher runs kernels on the GPU)")
    return _LAUNCHER
