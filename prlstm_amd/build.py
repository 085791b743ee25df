"""Builds libhsl.so (the HIP kernels + C ABI of include/hsl.h) in-tree for gfx950.

Usage: ``python -m prlstm_amd.build`` (or ``__graft_entry__.build()``).  Every
``csrc/*.hip`` file is compiled to an object with hipcc in parallel and the
objects are linked into ``prlstm_amd/libhsl.so``.  The library is always
rebuilt; the objects go to ``prlstm_amd/_build/``.
"""

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
SRC = PKG / "csrc"
OUT = PKG / "_build"
LIB = PKG / "libhsl.so"
ARCH = os.environ.get("HSL_OFFLOAD_ARCH", "gfx950")

# -packed-fp32-ops: keep hipcc from emitting v_pk_{add,mul,fma}_f32 for plain float code.
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-variable",
]


def _hipcc():
    exe = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(exe).exists():
        raise RuntimeError("hipcc not found; the ROCm toolchain is required to build libhsl.so")
    return exe


def _compile(hipcc, src, verbose):
    obj = OUT / (src.stem + ".o")
    cmd = [hipcc, *HIPCC_FLAGS, "-c", str(src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    text = "\n".join(l for l in (r.stdout + r.stderr).splitlines()
                     if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{text}")
    if verbose and text.strip():
        print(text)
    return obj


def build(verbose=False):
    hipcc = _hipcc()
    OUT.mkdir(exist_ok=True)
    sources = sorted(SRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no sources under {SRC}")
    workers = min(len(sources), max(1, (os.cpu_count() or 2) // 2), 8)
    with cf.ThreadPoolExecutor(workers) as ex:
        objs = list(ex.map(lambda s: _compile(hipcc, s, verbose), sources))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build(verbose="-q" not in sys.argv)
