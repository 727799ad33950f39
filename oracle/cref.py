"""ctypes loaders for the C oracle and the reference's own C library. TEST INFRASTRUCTURE ONLY.

oracle_lib()  oracle/_build/liblowbit_oracle.so, the plain-C restatement
              (built by `make -C oracle oracle`; rebuilt here if missing and gcc exists).
ref_lib()     oracle/_ref/liblowbit_ref.so, the reference's C sources compiled in
              place by oracle/Makefile, or None when it was never built (the GPU
              box only has what travelled from the build container).
"""
from __future__ import annotations

import ctypes as C
import os
import shutil
import subprocess
from functools import lru_cache
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ORACLE_SO = HERE / "_build" / "liblowbit_oracle.so"
REF_SO = HERE / "_ref" / "liblowbit_ref.so"

_f32 = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_f64 = np.ctypeslib.ndpointer(np.float64, flags="C_CONTIGUOUS")
_u8 = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")
_i8 = np.ctypeslib.ndpointer(np.int8, flags="C_CONTIGUOUS")
_i32 = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")
_i64 = np.ctypeslib.ndpointer(np.int64, flags="C_CONTIGUOUS")
_vp = C.c_void_p
_int = C.c_int


def build_oracle() -> Path:
    """Compile the C restatement if it is missing (needs gcc and make)."""
    if not ORACLE_SO.exists():
        if shutil.which("make") is None:
            raise RuntimeError("oracle library missing and `make` is not available")
        subprocess.run(["make", "-C", str(HERE), "oracle"], check=True,
                       stdout=subprocess.DEVNULL)
    return ORACLE_SO


@lru_cache(maxsize=1)
def oracle_lib() -> C.CDLL:
    so = C.CDLL(str(build_oracle()))
    sig = {
        "orc_version": ([], _int),
        "orc_quant_act_int8": ([_f32, _int, _int, _i8, _f32, _i32], None),
        "orc_group_acc": ([_i8, _int, _int, _u8, _vp, _int, _i64], None),
        "orc_gemm_w4a16": ([_f32, _int, _int, _u8, _f32, _vp, _int, _f64, _int], None),
        "orc_gemm_mxfp4": ([_f32, _int, _int, _u8, _u8, _int, _f64, _int], None),
        "orc_gemm_w4a8": ([_i8, _f32, _i32, _int, _int, _u8, _f32, _vp, _int, _f64, _vp], None),
    }
    for name, (args, res) in sig.items():
        fn = getattr(so, name)
        fn.argtypes, fn.restype = args, res
    return so


class RefParams(C.Structure):
    """lb_params of the reference ABI (src/lowbit/csrc/lowbit.h:37-45)."""
    _fields_ = [(f, C.c_int) for f in ("isa", "mr", "nr", "nb", "kb", "order", "nthreads")]


def ref_path() -> Path:
    """Where the reference C library is looked for (LOWBIT_REF_LIB overrides)."""
    return Path(os.environ.get("LOWBIT_REF_LIB", str(REF_SO)))


@lru_cache(maxsize=1)
def ref_lib() -> C.CDLL | None:
    """The reference C library, or None if oracle/_ref was never built."""
    path = ref_path()
    if not path.exists():
        return None
    so = C.CDLL(str(path))
    pp = C.POINTER(RefParams)
    sig = {
        "lb_version": ([], _int),
        "lb_cpu_isa": ([], _int),
        "lb_active_isa": ([], _int),
        "lb_has_vnni": ([], _int),
        "lb_max_threads": ([], _int),
        "lb_effective_isa": ([_int, _int], _int),
        "lb_gemm_w4a16": ([_f32, _int, _int, _u8, _f32, _vp, _int, _f32, pp], _int),
        "lb_gemm_mxfp4": ([_f32, _int, _int, _u8, _u8, _int, _f32, pp], _int),
        "lb_gemm_w4a8": ([_f32, _int, _int, _u8, _f32, _vp, _int, _f32, pp], _int),
        "lb_gemm_w4a8_q": ([_i8, _f32, _i32, _int, _int, _u8, _f32, _vp, _int, _f32, pp], _int),
        "lb_quant_act_int8": ([_f32, _int, _int, _i8, _f32, _i32], None),
        "lb_w4a8_group_acc": ([_i8, _i32, _int, _int, _u8, _vp, _int, _i32, _int], _int),
    }
    for name, (args, res) in sig.items():
        fn = getattr(so, name)
        fn.argtypes, fn.restype = args, res
    return so


def zp(z):
    """numpy array or None -> void* (NULL for None)."""
    return None if z is None else np.ascontiguousarray(z).ctypes.data_as(C.c_void_p)


# ------------------------------------------------------------------ C-oracle wrappers

def c_quant_act_int8(xp: np.ndarray):
    xp = np.ascontiguousarray(xp, np.float32)
    m, kp = xp.shape
    xq = np.empty((m, kp), np.int8)
    xs = np.empty(m, np.float32)
    asum = np.empty((m, kp // 128), np.int32)
    oracle_lib().orc_quant_act_int8(xp, m, kp, xq, xs, asum)
    return xq, xs, asum


def c_group_acc(xq: np.ndarray, qw: np.ndarray, zeros) -> np.ndarray:
    xq = np.ascontiguousarray(xq, np.int8)
    m, kp = xq.shape
    n = qw.shape[0]
    out = np.empty((m, n, kp // 128), np.int64)
    z = None if zeros is None else np.ascontiguousarray(zeros, np.uint8)
    oracle_lib().orc_group_acc(xq, m, kp, np.ascontiguousarray(qw), zp(z), n, out)
    return out


def c_gemm_w4a16(xp, qw, scales, zeros, absval: bool = False) -> np.ndarray:
    xp = np.ascontiguousarray(xp, np.float32)
    m, kp = xp.shape
    n = qw.shape[0]
    y = np.empty((m, n), np.float64)
    z = None if zeros is None else np.ascontiguousarray(zeros, np.uint8)
    oracle_lib().orc_gemm_w4a16(xp, m, kp, np.ascontiguousarray(qw),
                                np.ascontiguousarray(scales, np.float32), zp(z), n, y, int(absval))
    return y


def c_gemm_mxfp4(xp, qw, e8m0, absval: bool = False) -> np.ndarray:
    xp = np.ascontiguousarray(xp, np.float32)
    m, kp = xp.shape
    n = qw.shape[0]
    y = np.empty((m, n), np.float64)
    oracle_lib().orc_gemm_mxfp4(xp, m, kp, np.ascontiguousarray(qw),
                                np.ascontiguousarray(e8m0, np.uint8), n, y, int(absval))
    return y


def c_gemm_w4a8(xq, xs, asum, qw, scales, zeros):
    """(y, bound) in float64 from quantized activations."""
    xq = np.ascontiguousarray(xq, np.int8)
    m, kp = xq.shape
    n = qw.shape[0]
    y = np.empty((m, n), np.float64)
    bound = np.empty((m, n), np.float64)
    z = None if zeros is None else np.ascontiguousarray(zeros, np.uint8)
    oracle_lib().orc_gemm_w4a8(xq, np.ascontiguousarray(xs, np.float32),
                               np.ascontiguousarray(asum, np.int32), m, kp,
                               np.ascontiguousarray(qw), np.ascontiguousarray(scales, np.float32),
                               zp(z), n, y, bound.ctypes.data_as(C.c_void_p))
    return y, bound
