"""Build the gfx950 shared library ``_lib/libmoe_mi355x.so`` with hipcc.

Every HIP source is compiled for gfx950 only, with packed-fp32 instruction
selection disabled, and linked with the host-side sources into one shared
library whose C ABI is declared in ``include/*.h``.

    python -m llm_gpu_kernels_amd.build
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
LIBDIR = PKG / "_lib"
LIBNAME = "libmoe_mi355x.so"
LIB = LIBDIR / LIBNAME
OBJDIR = ROOT / "_build" / "obj"

ARCH = "gfx950"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
COMMON = ["-O3", "-fPIC", "-std=c++17", "-Wall", "-Wno-unused-function",
          f"-I{ROOT / 'include'}"]
HIP_FLAGS = [f"--offload-arch={ARCH}", "-Xclang", "-target-feature", "-Xclang",
             "-packed-fp32-ops", "-munsafe-fp-atomics"]


def sources():
    return sorted(CSRC.glob("*.hip")) + sorted(CSRC.glob("*.cpp"))


def _compile(src: Path) -> Path:
    OBJDIR.mkdir(parents=True, exist_ok=True)
    obj = OBJDIR / (src.name + ".o")
    flags = COMMON + (HIP_FLAGS if src.suffix == ".hip" else ["-x", "c++"])
    cmd = [HIPCC, *flags, "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in res.stderr.splitlines() if noise not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{err}")
    if err.strip():
        print(err)
    return obj


def build(verbose: bool = True) -> Path:
    """Compile every source and link the shared library (always rebuilds)."""
    if not Path(HIPCC).exists() and shutil.which("hipcc") is None:
        raise RuntimeError("hipcc not found; the HIP library cannot be built")
    srcs = sources()
    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as pool:
        objs = list(pool.map(_compile, srcs))
    LIBDIR.mkdir(exist_ok=True)
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB.relative_to(ROOT)} from {len(srcs)} sources")
    return LIB


if __name__ == "__main__":
    build()
