"""Compiles the gfx950 HIP kernels and the C-ABI shim into nexttransformer_amd/_lib/libnt_moe.so.

    python -m nexttransformer_amd.build [-v]

Every translation unit is compiled with hipcc for gfx950 only, in parallel, then linked into one
shared library that the package loads through ctypes. Packed-FP32 instructions are disabled for
all device code (-Xclang -target-feature -Xclang -packed-fp32-ops).
"""
from concurrent.futures import ThreadPoolExecutor
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "_lib" / "libnt_moe.so"
ARCH = "gfx950"

FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument", "-Wno-inline-asm",
    f"-I{ROOT / 'include'}", f"-I{CSRC}",
]


def hipcc():
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(path).exists():
        raise RuntimeError("hipcc not found: the MI355X kernels need ROCm's hipcc")
    return path


def sources():
    return sorted(CSRC.glob("*.hip"))


def _compile(src, verbose):
    obj = BUILD / (src.stem + ".o")
    cmd = [hipcc(), *FLAGS, "-c", str(src), "-o", str(obj)]
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{proc.stderr}")
    return obj


def build(verbose=False, jobs=None):
    """Compile every kernel source and link libnt_moe.so; returns the library path."""
    BUILD.mkdir(parents=True, exist_ok=True)
    LIB.parent.mkdir(parents=True, exist_ok=True)
    srcs = sources()
    jobs = jobs or min(len(srcs), int(os.environ.get("MAX_JOBS", "8")))
    with ThreadPoolExecutor(max_workers=jobs) as pool:
        objs = list(pool.map(lambda s: _compile(s, verbose), srcs))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stderr}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
