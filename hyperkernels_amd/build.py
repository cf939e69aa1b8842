"""Builds the gfx950 kernel library ``hyperkernels_amd/libhk_amd.so`` in-tree with hipcc.

Each ``csrc/*.hip`` file is compiled to an object in ``hyperkernels_amd/_build/`` (in
parallel) and the objects are linked into one shared library that exports the C ABI declared
in ``include/hk.h``. The library is self-contained: it links only the HIP runtime.

Usage: ``python -m hyperkernels_amd.build`` (or ``__graft_entry__.build()``).
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import pathlib
import shutil
import subprocess
import sys

PKG = pathlib.Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "libhk_amd.so"
ARCH = os.environ.get("HK_OFFLOAD_ARCH", "gfx950")

# -packed-fp32-ops: keep the compiler from emitting packed fp32 VALU instructions on this
# target (hipcc's host pass warns that it does not know the feature; that is harmless).
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-fvisibility=hidden",
    "-munsafe-fp-atomics",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{ROOT / 'include'}",
    f"-I{CSRC}",
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and pathlib.Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (needs ROCm in /opt/rocm)")


def _compile(src: pathlib.Path, hipcc: str, extra: list[str]) -> pathlib.Path:
    obj = BUILD / (src.stem + ".o")
    cmd = [hipcc, *HIPCC_FLAGS, *extra, "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{proc.stderr[-6000:]}")
    return obj


def build(verbose: bool = True, jobs: int | None = None, extra: list[str] | None = None) -> pathlib.Path:
    """Compiles every csrc/*.hip and links libhk_amd.so; returns the library path."""
    hipcc = _hipcc()
    BUILD.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError("no HIP sources under hyperkernels_amd/csrc")
    jobs = jobs or min(len(sources), int(os.environ.get("MAX_JOBS", os.cpu_count() or 4)), 16)
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda s: _compile(s, hipcc, extra or []), sources))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stderr[-6000:]}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"[hyperkernels_amd] built {LIB} from {len(sources)} sources for {ARCH}", flush=True)
    return LIB


if __name__ == "__main__":
    build()
    sys.exit(0)
