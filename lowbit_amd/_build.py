"""Build of liblowbit_hip.so: the gfx950 kernels and the C ABI, compiled by hipcc.

The library is built in-tree (lowbit_amd/_lib/) so that it travels with the
source tree to the GPU machine. Unlike the reference's lazy build
(src/lowbit/_build.py:96-140), loading never compiles: `lib_path()` returns the
built file or raises, so a GPU run cannot silently pick up something else.

Environment
  LOWBIT_LIB     path to a prebuilt liblowbit_hip.so (skips the in-tree file)
  HIPCC          compiler (default /opt/rocm/bin/hipcc, else `hipcc` on PATH)
  LOWBIT_ARCH    offload target (default gfx950)
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
INCLUDE = PKG.parent / "include"
LIBDIR = PKG / "_lib"
LIBNAME = "liblowbit_hip.so"
SOURCES = ["lb_api.hip", "lb_kernels.hip", "lb_gemv_g32.hip", "lb_model.hip", "lb_wquant.hip", "lb_probe.hip"]

# -packed-fp32-ops off: the compiler must not emit packed fp32 VALU ops.
# Denormals are kept (the E8M0 scale 2^-127 is a float32 subnormal) and no
# fast-math: the int8 quantizer relies on IEEE float32 division and rounding.
# Device functions start on 4 KiB boundaries, so a kernel's first page holds its
# first 4 KiB of code: the same W4A16 decode kernel took 6.56-7.05 us per launch at
# 1 x 11008 x 4096 cold when the linker placed it 3.5 KiB into a page (its first
# page boundary 512 bytes in, inside the prologue), 6.30-6.40 us page-aligned.
FLAGS = ["-O3", "-std=c++17", "-fPIC", "-shared", "-Wall", "-Wextra", "-Wno-unused-parameter",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
         "-fno-gpu-flush-denormals-to-zero", "-fno-fast-math",
         "-Xarch_device", "-falign-functions=4096"]


def _hipcc() -> str:
    env = os.environ.get("HIPCC")
    if env:
        return env
    if Path("/opt/rocm/bin/hipcc").exists():
        return "/opt/rocm/bin/hipcc"
    found = shutil.which("hipcc")
    if not found:
        raise RuntimeError("hipcc not found; set HIPCC or LOWBIT_LIB")
    return found


def build(verbose: bool = False) -> Path:
    """Compile the library for gfx950 into lowbit_amd/_lib (always recompiles).
    Each source is compiled to an object in parallel, then they are linked."""
    LIBDIR.mkdir(parents=True, exist_ok=True)
    arch = os.environ.get("LOWBIT_ARCH", "gfx950")
    out = LIBDIR / LIBNAME
    tag = f".tmp{os.getpid()}"
    tmp = LIBDIR / (LIBNAME + tag)
    objs = [LIBDIR / (Path(s).stem + f"{tag}.o") for s in SOURCES]
    cflags = [f for f in FLAGS if f != "-shared"]
    jobs = []
    for src, obj in zip(SOURCES, objs):
        cmd = [_hipcc(), f"--offload-arch={arch}", *cflags, f"-I{INCLUDE}", "-c", str(CSRC / src), "-o", str(obj)]
        if verbose:
            print(" ".join(cmd))
        jobs.append(subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True))
    errs = []
    for j in jobs:
        _, err = j.communicate()
        if j.returncode != 0:
            errs.append(err)
        elif verbose and err.strip():
            print(err, file=sys.stderr)
    try:
        if errs:
            raise RuntimeError(f"building {LIBNAME} failed:\n" + "\n".join(errs))
        cmd = [_hipcc(), f"--offload-arch={arch}", "-shared", "-fPIC", *[str(o) for o in objs], "-o", str(tmp)]
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            tmp.unlink(missing_ok=True)
            raise RuntimeError(f"linking {LIBNAME} failed:\n{r.stderr}")
    finally:
        for o in objs:
            o.unlink(missing_ok=True)
    os.replace(tmp, out)  # atomic: a concurrent loader sees the old or the new file
    return out


def lib_path() -> Path:
    """The library to load: $LOWBIT_LIB, else the in-tree build. Never builds."""
    env = os.environ.get("LOWBIT_LIB")
    if env:
        return Path(env)
    p = LIBDIR / LIBNAME
    if not p.exists():
        raise RuntimeError(f"{p} is not built; run `python -m lowbit_amd._build` "
                           "(or __graft_entry__.build()) first")
    return p


if __name__ == "__main__":
    print(build(verbose=True))
