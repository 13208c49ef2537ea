"""The operator contract of the reference's kernel files, restated for the HIP path.

A kernel file declares a ``KernelSpec``: name, Triton signature, constexprs, the memory-backed
arguments (``Arg(name, role, dtype, shape)`` with flat shapes), the launch grid, scalars
(``extra["scalar_values"]``), seeded ``make_inputs`` and tolerances
(reference: pytorchsim_triton_compiler/contract/kernel_spec.py:24-139).  A compiled kernel is
described by a manifest with the same facts (contract/kernel_object.py:333-359).  This module
keeps those shapes of data so that a caller of the reference's boundary can hand its specs,
manifests and tensors to the MI355X path unchanged; it holds no compiler state.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Callable

IN = "in"
OUT = "out"
INOUT = "inout"
ROLES = (IN, OUT, INOUT)

# dtype name -> numpy carrier and byte size: bf16 travels as uint16 bits and fp8 as uint8 bits, as in
# the reference's kernel objects (contract/kernel_object.py:43-56); the table is the same mapping.
NP_DTYPE = {
    "float64": "float64", "float32": "float32", "float16": "float16",
    "bfloat16": "uint16", "float8_e5m2": "uint8", "float8_e4m3fn": "uint8",
    "int64": "int64", "int32": "int32", "int16": "int16", "int8": "int8",
    "uint64": "uint64", "uint32": "uint32", "uint16": "uint16", "uint8": "uint8",
    "bool": "int8",
}
ITEMSIZE = {
    "float64": 8, "float32": 4, "float16": 2, "bfloat16": 2, "float8_e5m2": 1, "float8_e4m3fn": 1,
    "int64": 8, "int32": 4, "int16": 2, "int8": 1,
    "uint64": 8, "uint32": 4, "uint16": 2, "uint8": 1,
    "bool": 1,
}
# Triton pointer tokens of a signature -> dtype names
TRITON_DTYPE = {"fp64": "float64", "fp32": "float32", "fp16": "float16", "bf16": "bfloat16", "i64": "int64",
                "i32": "int32", "i16": "int16", "i8": "int8", "i1": "bool", "fp8e4nv": "float8_e4m3fn",
                "fp8e5": "float8_e5m2"}


def is_read(arg) -> bool:
    return arg.role in (IN, INOUT)


def is_written(arg) -> bool:
    return arg.role in (OUT, INOUT)


@dataclass
class Arg:
    """One memory-backed kernel argument (contract/kernel_spec.py:24-38)."""
    name: str
    role: str
    dtype: str
    shape: tuple

    def __post_init__(self):
        if self.role not in ROLES:
            raise ValueError(f"Arg {self.name}: role must be one of {ROLES}, not {self.role!r}")
        if self.dtype not in ITEMSIZE:
            raise ValueError(f"Arg {self.name}: unknown dtype {self.dtype!r}")
        self.shape = tuple(int(s) for s in self.shape)

    @property
    def numel(self) -> int:
        return math.prod(self.shape)

    @property
    def nbytes(self) -> int:
        return self.numel * ITEMSIZE[self.dtype]


@dataclass
class KernelSpec:
    """What a kernel file declares (contract/kernel_spec.py:41-139), minus the compiler-only fields
    (expected IR, scratchpad placement, prefetch plan)."""
    name: str
    signature: dict
    constexprs: dict
    args: list
    grid: tuple
    kernel: Callable | None = None
    reference: Callable | None = None
    make_inputs: Callable | None = None
    rtol: float = 1e-4
    atol: float = 1e-4
    parallel_axes: tuple = ()
    extra: dict = field(default_factory=dict)
    graph_prefetch: object = None

    def __post_init__(self):
        self.grid = tuple(int(g) for g in self.grid)
        if not self.parallel_axes:
            self.parallel_axes = ("x", "y", "z")[:max(1, len(self.grid))]
        names = [a.name for a in self.args]
        if len(set(names)) != len(names):
            raise ValueError(f"{self.name}: argument names repeat: {names}")

    def inputs(self):
        return [a for a in self.args if is_read(a)]

    def outputs(self):
        return [a for a in self.args if is_written(a)]

    def arg(self, name: str) -> Arg:
        for a in self.args:
            if a.name == name:
                return a
        raise KeyError(f"{self.name} has no argument {name!r}")

    @property
    def scalar_values(self) -> dict:
        return dict((self.extra or {}).get("scalar_values", {}))

    def manifest(self) -> dict:
        """The facts a compiled kernel's manifest states (contract/kernel_object.py:333-359) that a
        device needs to run it: name, grid, args, scalars, constexprs."""
        scalars = [{"name": n, "ctype": c, "default": self.scalar_values.get(n)}
                   for n, c in (self.extra or {}).get("scalar_args", [])]
        return {"name": self.name, "grid": list(self.grid),
                "args": [{"name": a.name, "role": a.role, "dtype": a.dtype, "shape": list(a.shape)}
                         for a in self.args],
                "scalars": scalars, "constexprs": dict(self.constexprs)}


def spec_from_manifest(manifest: dict) -> KernelSpec:
    """A KernelSpec from a manifest dict (the kernel.json facts, or :meth:`KernelSpec.manifest`)."""
    args = [Arg(a["name"], a["role"], a["dtype"], tuple(a["shape"])) for a in manifest["args"]]
    scalars = manifest.get("scalars", [])
    extra = dict(manifest.get("extra", {}))
    extra.update({"scalar_args": [(s["name"], s.get("ctype", "int32_t")) for s in scalars],
                  "scalar_values": {s["name"]: s.get("default") for s in scalars if s.get("default") is not None}})
    gp = manifest.get("graph_prefetch")
    return KernelSpec(name=manifest["name"], signature=manifest.get("signature", {}),
                      constexprs=dict(manifest.get("constexprs", {})), args=args,
                      grid=tuple(manifest.get("grid", (1,))), extra=extra,
                      graph_prefetch=None if gp is None else tuple(gp))


def seeded_inputs(spec: KernelSpec, torch, seed: int = 0, recorded: dict | None = None) -> dict:
    """The inputs the reference's generated specs draw (validation/pytorchsim/*/..._spec.py:28-36):
    one generator seeded once, then ``torch.randn(numel, generator=g).to(dtype)`` for every read
    argument in argument order.  Arguments the spec takes from its recorded ``*_inputs.pt`` instead
    (named in ``extra["recorded"]``; the MoE kernels' index tables) come from `recorded` and draw
    nothing from the generator, as the spec's make_inputs does.  CPU tensors, flat."""
    g = torch.Generator().manual_seed(seed)
    taken = set((spec.extra or {}).get("recorded", ()))
    out = {}
    for a in spec.inputs():
        if a.name in taken:
            if recorded is None or a.name not in recorded:
                raise KeyError(f"{spec.name}: argument {a.name} comes from the recorded inputs, which were not given")
            t = torch.as_tensor(recorded[a.name]).reshape(-1)
            if t.numel() != a.numel:
                raise ValueError(f"{spec.name}: recorded {a.name} has {t.numel()} elements, the spec says {a.numel}")
            out[a.name] = t.to(getattr(torch, a.dtype))
            continue
        dt = getattr(torch, a.dtype)
        out[a.name] = torch.randn(a.numel, generator=g).to(dt)
    return out


class ObjectError(RuntimeError):
    """A kernel object the launch cannot take (contract/kernel_object.py:75-76's ObjectError)."""


PROGRAM_ID_LIMIT = 1 << 21
"""Programs per grid axis a kernel object can name (contract/kernel_object.py:32, :125-128: program ids
are packed 21 bits an axis)."""


def grid3(grid) -> tuple:
    """A grid padded to three axes (contract/kernel_object.py:84-87)."""
    g = [int(v) for v in grid] + [1, 1, 1]
    return g[0], g[1], g[2]


def grid_bound(manifest_or_spec) -> tuple:
    """The per-axis program bound a launch may not pass: kernel.json's ``grid_bound``, None on an
    axis where it states none -- a null or absent grid_bound leaves every axis unbounded
    (contract/kernel_object.py:98-100: ``bound or [None]*3``).  A spec launched without a manifest
    is bounded by its grid, the extent its programs were compiled for (driver/stage.py:95)."""
    if isinstance(manifest_or_spec, KernelSpec):
        return grid3(manifest_or_spec.grid)
    bound = manifest_or_spec.get("grid_bound")
    if not bound:
        return (None, None, None)
    b = list(bound) + [1, 1, 1]
    return tuple(None if v is None else int(v) for v in b[:3])


def refuse_grid_past_bound(name: str, grid, bound) -> tuple:
    """contract/kernel_object.py:93-107: refuse a launch grid with an axis past its bound, an axis below
    one, or a program id past PROGRAM_ID_LIMIT; returns the grid padded to three axes."""
    got = grid3(grid)
    over = [f"{a}={g} (bound {b})" for a, g, b in zip("xyz", got, bound) if b is not None and g > b]
    low = [f"{a}={g}" for a, g in zip("xyz", got) if g < 1]
    if over or low or any(g > PROGRAM_ID_LIMIT for g in got):
        raise ObjectError(f"{name}: launch grid {got} is refused; it was compiled for grids within {tuple(bound)}: "
                          f"{', '.join(over + [x + ' is below 1' for x in low]) or 'a program id past the key'}")
    return got


def disagreements(manifest: dict, spec: KernelSpec) -> list:
    """Every question a manifest and a spec both answer, asked of both (contract/kernel_object.py:264-278):
    argument order, scalar names, grid, sizes, written arguments, graph prefetch."""
    scalars = [s["name"] for s in manifest.get("scalars", [])]
    spec_scalars = [n for n, _ in (spec.extra or {}).get("scalar_args", [])]
    checks = (
        ("argv_order", [a["name"] for a in manifest["args"]], [a.name for a in spec.args]),
        ("scalars", scalars, spec_scalars),
        ("grid3", list(grid3(manifest["grid"])), list(grid3(spec.grid))),
        ("numel", [math.prod(a["shape"]) for a in manifest["args"]], [a.numel for a in spec.args]),
        ("writable", [a["name"] for a in manifest["args"] if a["role"] in (OUT, INOUT)],
         [a.name for a in spec.outputs()]),
        ("graph_prefetch", [manifest.get("graph_prefetch")],
         [None if spec.graph_prefetch is None else list(spec.graph_prefetch)]),
    )
    return [what for what, mine, theirs in checks if list(mine) != list(theirs)]


def refuse_if_it_disagrees(manifest: dict, spec: KernelSpec) -> None:
    """Refuse a manifest that answers differently from `spec` (contract/kernel_object.py:281-286)."""
    bad = disagreements(manifest, spec)
    if bad:
        raise ObjectError(f"{spec.name}: the manifest and the spec disagree about {', '.join(bad)}; "
                          "the manifest was written by a different compile")
