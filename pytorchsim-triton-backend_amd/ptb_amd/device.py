"""A device that runs a kernel object over tensors on disk, on the GPU.

Same shape as the reference's device interface (tests/runtime/device/base.py:25-58): a ``Launch``
names the kernel object's directory, its manifest (name, grid, args with role/dtype/shape, scalars),
and one ``.raw`` file per argument (bf16 as uint16 bits, tests/runtime/stages.py:86-87);
``Device.launch(req)`` runs it and leaves every written argument in its ``.raw`` file.

``HipDevice`` reads the read arguments into device memory, poisons the written-only ones with NaN
bit patterns (so an element the kernel fails to write cannot pass as a plausible value), runs the
matching HIP kernel family and writes the results back.  The Triton source, which two families
read index facts from, comes from ``manifest["source"]`` or a ``*_triton.py`` file in the object
directory.
"""
from __future__ import annotations

import contextlib
import glob
import os

import numpy as np

from . import launcher
from .contract import NP_DTYPE, is_read, is_written, spec_from_manifest
from .verify import read_raw, write_raw


class DeviceError(RuntimeError):
    pass


@contextlib.contextmanager
def _no_step(_name):
    yield


class Launch:
    """One launch: the object directory, its manifest, where its tensors are, and the grid."""

    def __init__(self, obj_dir, manifest, runtime_dir=None, raw_paths=None, log=None, run=None, step=None,
                 error=None, grid=None):
        self.obj_dir = obj_dir
        self.manifest = manifest
        self.runtime_dir = runtime_dir
        self.raw_paths = raw_paths or {}
        self.log = log
        self.run = run
        self.step = step or _no_step
        self.error = error or (lambda message, **kw: DeviceError(message))
        self.grid = grid


class Device:
    name = None

    def launch(self, req):
        raise NotImplementedError


_POISON = {"bfloat16": 0xFFFF, "float16": 0xFFFF, "float32": 0xFFFFFFFF, "float8_e4m3fn": 0xFF, "float8_e5m2": 0xFF}


class HipDevice(Device):
    """Runs kernel objects on the current HIP device."""

    name = "hip"

    def source_of(self, req) -> str | None:
        src = req.manifest.get("source")
        if src:
            return src
        if req.obj_dir:
            hits = sorted(glob.glob(os.path.join(req.obj_dir, "*_triton.py")))
            if hits:
                with open(hits[0]) as fh:
                    return fh.read()
        return None

    def launch(self, req):
        import torch

        spec = spec_from_manifest(req.manifest)
        tensors = {}
        with req.step("hip-upload"):
            for a in spec.args:
                dt = getattr(torch, a.dtype)
                if is_read(a):
                    path = req.raw_paths.get(a.name)
                    if not path or not os.path.exists(path):
                        raise req.error(f"{spec.name}: no .raw file for input {a.name}")
                    host = torch.from_numpy(np.ascontiguousarray(read_raw(path, a)).reshape(-1))
                    tensors[a.name] = host.view(dt).to("cuda")
                else:
                    bits = _POISON.get(a.dtype, 0)
                    carrier = np.full(a.numel, bits, dtype=np.dtype(NP_DTYPE[a.dtype]))
                    tensors[a.name] = torch.from_numpy(carrier).view(dt).to("cuda")
        with req.step("hip-launch"):
            try:
                launcher.launch(spec, tensors, grid=req.grid, source=self.source_of(req))
            except Exception as e:  # noqa: BLE001 - reported through the caller's error type
                raise req.error(f"{spec.name}: {type(e).__name__}: {e}") from e
            torch.cuda.synchronize()
        with req.step("hip-download"):
            for a in spec.args:
                if is_written(a):
                    path = req.raw_paths.get(a.name)
                    if not path:
                        raise req.error(f"{spec.name}: no .raw path for output {a.name}")
                    carrier = getattr(np, NP_DTYPE[a.dtype])
                    host = tensors[a.name].cpu()
                    bits = host.view(getattr(torch, {1: "uint8", 2: "int16", 4: "int32", 8: "int64"}[host.element_size()]))
                    write_raw(path, a, bits.numpy().view(carrier))
        return None


REGISTRY = {"hip": HipDevice}


def get(name: str) -> Device:
    try:
        return REGISTRY[name]()
    except KeyError:
        raise DeviceError(f"unknown device {name!r}; known: {sorted(REGISTRY)}") from None
