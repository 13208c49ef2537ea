"""The launch hooks the reference's callers use, served by the HIP kernels.

* ``launch(spec_or_manifest, tensors, grid=None, source=None, scalars=None, manifest=None)`` -- run
  one kernel over device tensors keyed by argument name (or given in argument order).
* ``hip_launcher(binary, kernel_object, grid, args, artifacts=None)`` -- a callable with the
  signature PyTorchSim registers through ``pytorchsim_triton_backend.driver.set_launcher``
  (reference: pytorchsim_triton_compiler/triton_extension/python/pytorchsim_triton_backend/
  driver.py:86-100): ``binary`` (the compiled ELF) is not needed here; ``kernel_object`` is the
  kernel.json text or dict; ``args`` are the call's arguments with the constexprs dropped, in
  signature order (driver.py:39-44): tensors and runtime scalars interleaved.
* ``set_launcher`` / ``registered_launcher`` mirror the reference's registry (driver.py:86-100):
  with nothing registered, a launch raises ``RuntimeError`` as the reference's driver does.

Launch semantics follow the reference's kernel objects: a grid past the compiled bound (kernel.json's
``grid_bound``; a null bound, or a null axis, is unbounded; a spec launched without a manifest is
bounded by its grid) is refused (contract/kernel_object.py:93-107); a grid within it runs the
programs it names -- the whole kernel at its grid, a prefix of row blocks below it where the
family's programs are row blocks, and programs past the kernel's extent, which the reference's
masks make no-ops, not at all -- through the family's spec-driven C entry
(``ptb_<family>_args``); runtime scalars are taken by name (contract/kernel_object.py:122-127) and a
manifest that disagrees with the spec it is launched beside is refused (:264-286).  The whole grid
is one HIP launch: the reference's per-program loop (codegen/wrapper.py:254-265) has no
counterpart.
"""
from __future__ import annotations

import json

from . import capi, kernels
from .contract import KernelSpec, ObjectError, grid3, grid_bound, refuse_grid_past_bound, refuse_if_it_disagrees
from .contract import spec_from_manifest


class GridMismatch(ObjectError, ValueError):
    """A launch grid the compiled kernel does not take."""


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


def _with_scalars(spec: KernelSpec, scalars: dict | None) -> KernelSpec:
    """The spec with a launch's runtime scalar values in place of its defaults, by name."""
    if not scalars:
        return spec
    known = [n for n, _ in (spec.extra or {}).get("scalar_args", [])]
    unknown = sorted(set(scalars) - set(known))
    if unknown:
        raise ObjectError(f"{spec.name}: no runtime scalar named {', '.join(unknown)} (it takes {known})")
    extra = dict(spec.extra or {})
    extra["scalar_values"] = {**spec.scalar_values, **{k: int(v) if isinstance(v, bool) or float(v).is_integer()
                                                        else float(v) for k, v in scalars.items()}}
    return KernelSpec(name=spec.name, signature=spec.signature, constexprs=spec.constexprs, args=spec.args,
                      grid=spec.grid, extra=extra, graph_prefetch=spec.graph_prefetch)


def _programs(spec: KernelSpec, bound) -> int:
    """The kernel's programs along x for its current extents: ceil(xnumel / XBLOCK) for the
    Inductor kernels that state both (the grid Inductor launches them with; a kernel object rebuilt
    for other extents keeps its XBLOCK and takes the call's xnumel), else the bound, else the spec's
    grid."""
    ce, sv = spec.constexprs or {}, spec.scalar_values
    xnumel, xblock = sv.get("xnumel", ce.get("xnumel")), ce.get("XBLOCK")
    if xnumel is not None and xblock:
        return max(1, -(-int(xnumel) // int(xblock)))
    return bound[0] if bound[0] is not None else grid3(spec.grid)[0]


def launch(spec_or_manifest, tensors, grid=None, source: str | None = None, scalars: dict | None = None,
           manifest: dict | None = None) -> kernels.Plan:
    """Run one reference kernel on the GPU (asynchronously, on the current stream).

    `grid` defaults to the spec's; one past the bound is refused with :class:`GridMismatch`.
    `scalars` maps runtime scalar names to this launch's values.  `manifest`, when given beside a
    spec, must agree with it."""
    spec = _as_spec(spec_or_manifest)
    bound_of = manifest if manifest is not None else (
        spec_or_manifest if isinstance(spec_or_manifest, dict) else spec)
    if manifest is not None:
        refuse_if_it_disagrees(manifest, spec)
    if not isinstance(tensors, dict):
        tensors = {a.name: t for a, t in zip(spec.args, tensors)}
    bound = grid_bound(bound_of)
    try:
        g = refuse_grid_past_bound(spec.name, spec.grid if grid is None else grid, bound)
    except ObjectError as e:
        raise GridMismatch(str(e)) from None
    _check_tensors(spec, tensors)
    spec = _with_scalars(spec, scalars)
    flat = {a.name: tensors[a.name].view(-1) for a in spec.args}
    plan = kernels.resolve(spec, source)
    programs = _programs(spec, bound)
    # programs past the kernel's own extent (allowed where grid_bound leaves the axis unbounded or
    # bounds it further) find no element inside the tensors: masked no-ops, so they are not run
    g = (min(g[0], programs), min(g[1], grid3(spec.grid)[1]), min(g[2], grid3(spec.grid)[2]))
    xblock = (spec.constexprs or {}).get("XBLOCK")
    entry = capi.plan_args(plan, programs, int(xblock) if xblock else None)
    if entry is not None:
        fam, names, ints, floats = entry
        roles = {a.name: a.role for a in spec.args}
        ts = [flat[n] for n in names]
        rs = [roles[n] for n in names]
        ws = capi.workspace_for(plan, ts[0].device)
        if ws is not None:
            ts.append(ws)
            rs.append("out")
        capi.call_args(fam, ts, rs, ints, floats, g)
        return plan
    if g != (programs,) + grid3(spec.grid)[1:]:
        raise kernels.UnsupportedKernel(f"{spec.name}: family {plan.family} runs its whole grid "
                                        f"{grid3(spec.grid)} only, not {g}")
    kernels.run(plan, flat)
    return plan


def hip_launcher(binary, kernel_object, grid, args, artifacts=None):
    """set_launcher-compatible entry: run the kernel object's kernel over `args` on the GPU.  `args`
    are in signature order with the constexprs dropped (driver.py:39-44): the tensors bind to the
    kernel object's arguments in order, the other values to its runtime scalars in order."""
    ko = json.loads(kernel_object) if isinstance(kernel_object, (str, bytes)) else dict(kernel_object)
    spec = _as_spec(ko)
    tensors, values = [], []
    for a in args:
        (tensors if hasattr(a, "data_ptr") else values).append(a)
    if len(tensors) != len(spec.args):
        raise ObjectError(f"{spec.name}: called with {len(tensors)} tensors, the kernel object has {len(spec.args)}")
    names = [s["name"] for s in ko.get("scalars", [])]
    if values and len(values) != len(names):
        raise ObjectError(f"{spec.name}: called with {len(values)} scalars, the kernel object has {len(names)} "
                          "(all or none)")
    return launch(ko, tensors, grid=grid, source=ko.get("source"), scalars=dict(zip(names, values)) or None)


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
