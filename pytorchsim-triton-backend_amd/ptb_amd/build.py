"""Build ``libptb_amd.so`` for gfx950 from ``csrc/*.hip`` with hipcc directly (no cmake, no JIT).

Every HIP source is compiled to an object under ``<repo>/_build/ptb_amd`` in parallel, then linked
into ``ptb_amd/lib/libptb_amd.so`` inside the source tree, so the built library travels with the
tree.  Run ``python -m ptb_amd.build`` (with the package's parent directory on ``sys.path``) or call
:func:`build`.
"""
from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
PROJECT = PKG.parent
REPO = PROJECT.parent
CSRC = PROJECT / "csrc"
INCLUDE = REPO / "include"
LIB_DIR = PKG / "lib"
LIB = LIB_DIR / "libptb_amd.so"
BUILD_DIR = REPO / "_build" / "ptb_amd"

ARCH = "gfx950"
# -packed-fp32-ops: keep the compiler from forming v_pk_{add,mul,fma}_f32, some forms of which have
# given wrong results now and then on the MI355X boxes this was built for, with no error; the host
# pass warns that it does not know the feature, which is harmless.
HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-fvisibility=hidden",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def hipcc() -> str:
    exe = os.environ.get("HIPCC") or shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(exe).exists() and shutil.which(exe) is None:
        raise RuntimeError(f"hipcc not found (looked for {exe!r}); ROCm is required to build ptb_amd")
    return exe


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


def _compile(src: Path, obj: Path, cc: str) -> None:
    cmd = [cc, *HIP_FLAGS, f"-I{INCLUDE}", f"-I{CSRC}", "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{res.stdout}\n{res.stderr}")


def build(jobs: int | None = None, verbose: bool = False) -> Path:
    """Compile every csrc/*.hip for gfx950 and link the shared library; returns its path."""
    cc = hipcc()
    srcs = sources()
    if not srcs:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    BUILD_DIR.mkdir(parents=True, exist_ok=True)
    LIB_DIR.mkdir(parents=True, exist_ok=True)
    objs = [BUILD_DIR / (s.stem + ".o") for s in srcs]
    jobs = jobs or min(len(srcs), max(1, min(8, os.cpu_count() or 1)))
    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as ex:
        futs = {ex.submit(_compile, s, o, cc): s for s, o in zip(srcs, objs)}
        for f in concurrent.futures.as_completed(futs):
            f.result()
            if verbose:
                print(f"  compiled {futs[f].name}", flush=True)
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"  linked {LIB}", flush=True)
    return LIB


if __name__ == "__main__":
    build(verbose="-q" not in sys.argv)
