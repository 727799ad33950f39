"""ctypes binding to liblowbit_hip.so, the gfx950 fused dequantize+GEMM library.

Mirrors the reference binding (src/lowbit/kernels.py): the same public
functions, arguments and error behaviour (rc < 0 -> ValueError for bad shapes,
tiles and arguments), so callers switch by changing the import. Differences,
all forced by the device:
  * `isa` names a GPU path: "gfx950" (VALU decode kernels, small M) or
    "gfx950-mfma" (matrix cores). The reference's CPU names ("scalar", "avx2",
    "avx512") and "auto"/None mean "choose by shape"; there are no CPU tiers.
  * `threads` is accepted and ignored; `Params` tile fields are validated like
    the reference (an uncompiled (mr, nr) raises) and otherwise ignored.
  * Weights passed as Int4Weights / MXFP4Weights are uploaded once, on their
    first GEMM, and the device copy is reused while the container holds the same
    arrays (implicit residency). To keep that copy exact, the first GEMM marks
    the container's arrays read-only: an in-place edit then raises instead of
    going unseen, and a caller that means to edit sets `flags.writeable = True`
    (the next GEMM sees that and uploads again) or calls `release(w)`. A view
    taken before the first GEMM stays writeable and is not watched. With
    LOWBIT_RESIDENT=0, or inside `implicit_residency(False)`, every call goes
    through the pointer ABI (lb_gemm_*), which uploads the weights per call as the
    reference's C library reads them per call. `to_device(w)` uploads explicitly
    and returns a resident handle that every gemm_* accepts in place of the host
    container.
The library is never compiled here; a missing build raises RuntimeError.
"""
from __future__ import annotations

import contextlib
import ctypes as C
import os
import threading
import weakref
from dataclasses import asdict, dataclass
from functools import lru_cache

import numpy as np

from ._build import lib_path
from .formats import GROUP, GROUPS, MXBLOCK, Int4Weights, Int8Acts, MXFP4Weights, pad_acts, pad_to

ISA_GFX950 = 16
ISA_GFX950_MFMA = 17
ISA_NAMES = {ISA_GFX950: "gfx950", ISA_GFX950_MFMA: "gfx950-mfma"}
ISA_IDS = {v: k for k, v in ISA_NAMES.items()}
LEGACY_ISAS = ("scalar", "avx2", "avx512")  # reference CPU tiers: accepted, mean "auto"
KIND_IDS = {"w4a16": 0, "mxfp4": 1, "w4a8": 2}


class _Params(C.Structure):
    _fields_ = [(f, C.c_int) for f in ("isa", "mr", "nr", "nb", "kb", "order", "nthreads")]


@dataclass(frozen=True)
class Params:
    """Dispatch parameters (include/lowbit_hip.h lb_params). 0 means 'default'.

    Same fields as the reference's Params (src/lowbit/kernels.py:22-33). The GPU
    kernels choose their tiles from the shape regime; (mr, nr) is still checked
    against the reference's micro-tile list so an invalid request fails alike.
    """
    mr: int = 0
    nr: int = 0
    nb: int = 0
    kb: int = 0
    order: int = 0

    def as_dict(self) -> dict:
        return asdict(self)


TILES = [(1, 1), (1, 2), (1, 4), (2, 1), (2, 2), (2, 4), (4, 1), (4, 2), (4, 4), (8, 1), (8, 2)]

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")
_i8p = np.ctypeslib.ndpointer(np.int8, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")
_vp = C.c_void_p
_int = C.c_int
_sz = C.c_size_t
_pp = C.POINTER(_Params)

# name -> (argtypes, restype): every symbol the header declares
SIGNATURES = {
    "lb_version": ([], _int),
    "lb_cpu_isa": ([], _int),
    "lb_active_isa": ([], _int),
    "lb_has_vnni": ([], _int),
    "lb_has_openmp": ([], _int),
    "lb_max_threads": ([], _int),
    "lb_effective_isa": ([_int, _int], _int),
    "lb_device_info": ([C.c_char_p, _int, C.POINTER(_int), C.POINTER(_int)], _int),
    "lb_last_error": ([], C.c_char_p),
    "lb_last_status": ([], _int),
    "lb_gemm_w4a16": ([_f32p, _int, _int, _u8p, _f32p, _vp, _int, _f32p, _pp], _int),
    "lb_gemm_mxfp4": ([_f32p, _int, _int, _u8p, _u8p, _int, _f32p, _pp], _int),
    "lb_gemm_w4a8": ([_f32p, _int, _int, _u8p, _f32p, _vp, _int, _f32p, _pp], _int),
    "lb_gemm_w4a8_q": ([_i8p, _f32p, _i32p, _int, _int, _u8p, _f32p, _vp, _int, _f32p, _pp], _int),
    "lb_quant_act_int8": ([_f32p, _int, _int, _i8p, _f32p, _i32p], None),
    "lb_w4a8_group_acc": ([_i8p, _i32p, _int, _int, _u8p, _vp, _int, _i32p, _int], _int),
    "lbd_gemm_w4a16": ([_vp, _int, _int, _vp, _vp, _vp, _int, _vp, _pp, _vp], _int),
    "lbd_gemm_mxfp4": ([_vp, _int, _int, _vp, _vp, _int, _vp, _pp, _vp], _int),
    "lbd_gemm_w4a8": ([_vp, _int, _int, _vp, _vp, _vp, _int, _vp, _pp, _vp, _sz, _vp], _int),
    "lbd_w4a8_workspace_bytes": ([_int, _int], _sz),
    "lbd_gemm_w4a8_q": ([_vp, _vp, _vp, _int, _int, _vp, _vp, _vp, _int, _vp, _pp, _vp], _int),
    "lbd_quant_act_int8": ([_vp, _int, _int, _vp, _vp, _vp, _vp], _int),
    "lbd_w4a8_group_acc": ([_vp, _vp, _int, _int, _vp, _vp, _int, _vp, _int, _vp], _int),
    "lb_dev_malloc": ([C.POINTER(_vp), _sz], _int),
    "lb_dev_free": ([_vp], _int),
    "lb_memcpy_h2d": ([_vp, _vp, _sz], _int),
    "lb_memcpy_d2h": ([_vp, _vp, _sz], _int),
    "lb_memcpy_h2d_async": ([_vp, _vp, _sz, _vp], _int),
    "lb_memcpy_d2h_async": ([_vp, _vp, _sz, _vp], _int),
    "lb_memcpy_d2d": ([_vp, _vp, _sz], _int),
    "lb_memset_d": ([_vp, _int, _sz], _int),
    "lb_dev_synchronize": ([], _int),
    "lb_stream_create": ([C.POINTER(_vp)], _int),
    "lb_stream_destroy": ([_vp], _int),
    "lb_stream_synchronize": ([_vp], _int),
    "lb_event_create": ([C.POINTER(_vp)], _int),
    "lb_event_destroy": ([_vp], _int),
    "lb_event_record": ([_vp, _vp], _int),
    "lb_event_synchronize": ([_vp], _int),
    "lb_event_elapsed_ms": ([_vp, _vp, C.POINTER(C.c_float)], _int),
    "lb_stream_begin_capture": ([_vp], _int),
    "lb_stream_end_capture": ([_vp, C.POINTER(_vp)], _int),
    "lb_graph_launch": ([_vp, _vp], _int),
    "lb_graph_destroy": ([_vp], _int),
    "lbd_copy_kernel": ([_vp, _vp, _sz, _vp], _int),
    "lbd_read_kernel": ([_vp, _sz, _int, _int, _int, _vp, _vp], _int),
    "lbd_probe_valu": ([_int, _int, _int, _vp, _vp], _int),
    "lbd_probe_forms": ([], _int),
    "lbd_probe_mfma_valu": ([_int, _int, _int, _int, _vp, _vp], _int),
    "lbd_empty_kernel": ([_int, _vp], _int),
    "lbd_probe_div127": ([_vp, _vp], _int),
    "lbd_probe_grid_barrier": ([_int, _int, _int, _vp, _sz, _vp, _vp], _int),
    "lbd_gemm_path": ([_int, _int, _int, _pp], _int),
    "lbd_gemm_plan": ([_int, _int, _int, _int, _pp, C.c_void_p], _int),
    "lbd_int4_t16_bytes": ([_int, _int, C.POINTER(_sz), C.POINTER(_sz), C.POINTER(_sz)], _int),
    "lbd_repack_int4_t16": ([_vp, _vp, _vp, _int, _int, _vp, _vp, _vp, _vp], _int),
    "lbd_gemm_w4a8_t16": ([_vp, _int, _int, _vp, _vp, _vp, _int, _vp, _pp, _vp, _sz, _vp], _int),
    "lbd_gemm_w4a16_t16": ([_vp, _int, _int, _vp, _vp, _vp, _int, _vp, _pp, _vp, _sz, _vp], _int),
    "lbd_int4_t16f8_bytes": ([_int, _int, C.POINTER(_sz), C.POINTER(_sz)], _int),
    "lbd_w4a16_prefers_t16f8": ([_int, _int, _int], _int),
    "lbd_repack_int4_t16f8": ([_vp, _vp, _vp, _int, _int, _vp, _vp, _vp], _int),
    "lbd_gemm_w4a16_t16f8": ([_vp, _int, _int, _vp, _vp, _int, _vp, _pp, _vp, _sz, _vp], _int),
    "lbd_noalloc_scratch_bytes": ([], _sz),
    "lbd_gemm_w4a8_t16_noalloc": ([_vp, _int, _int, _vp, _vp, _vp, _int, _vp, _pp, _vp], _int),
    "lbd_bf16x3_workspace_bytes": ([_int, _int], _sz),
    "lbd_bf16x3_workspace_bytes_split": ([_int, _int, _int, _int], _sz),
    "lbd_mxfp4_t16_bytes": ([_int, _int, C.POINTER(_sz), C.POINTER(_sz)], _int),
    "lbd_repack_mxfp4_t16": ([_vp, _vp, _int, _int, _vp, _vp, _vp], _int),
    "lbd_gemm_mxfp4_t16": ([_vp, _int, _int, _vp, _vp, _int, _vp, _pp, _vp, _sz, _vp], _int),
    "lbd_quantize_int4": ([_vp, _int, _int, _int, _int, _vp, _vp, _vp, _vp], _int),
    "lbd_quantize_mxfp4": ([_vp, _int, _int, _vp, _vp, _vp], _int),
    "lbd_embed": ([_vp, _int, _int, _vp, _int, _vp, _vp], _int),
    "lbd_rmsnorm": ([_vp, _vp, _int, _int, C.c_float, _vp, _vp], _int),
    "lbd_qkv_rope": ([_vp, _vp, _int, _int, _int, _int, _vp, _vp, _vp, _int, _vp, _vp, _int, _vp], _int),
    "lbd_attention": ([_vp, _int, _vp, _vp, _int, _int, _int, _int, _vp, _int, _vp, _vp], _int),
    "lbd_swiglu": ([_vp, _int, _int, _vp, _vp], _int),
    "lbd_swiglu_pairs": ([_vp, _int, _int, _vp, _vp], _int),
    "lbd_add": ([_vp, _vp, _sz, _vp], _int),
    "lbd_argmax": ([_vp, _int, _vp, _vp, _int, _vp, _int, _vp], _int),
    "lbd_gemv_w4a16_fused": ([_vp, _int, _int, _vp, _vp, _vp, _int, _vp, C.c_void_p, _vp], _int),
    "lbd_gemv_mxfp4_fused": ([_vp, _int, _int, _vp, _vp, _int, _vp, C.c_void_p, _vp], _int),
    "lbd_gemv_w4a8_fused": ([_vp, _int, _int, _vp, _vp, _vp, _int, _vp, C.c_void_p, _vp], _int),
    "lbd_argmax_finalize": ([_vp, _vp, _vp, _int, _vp, _int, _vp], _int),
    "lbd_attention_decode": ([_vp, _int, _int, _int, _vp, _vp, _vp, _int, _vp, _vp, _int, _vp, _vp], _int),
    "lbd_attention_decode_ws": ([_vp, _int, _int, _int, _vp, _vp, _vp, _int, _vp, _vp, _int, _vp, _vp, _sz, _vp],
                                _int),
    "lbd_attention_decode_work_bytes": ([_int, _int, _int], _sz),
    "lbd_attention_slices": ([_vp, _int, _int, _int, _vp, _vp, _vp, _int, _vp, _vp, _int, _vp, _sz, _vp], _int),
    "lbd_attention_merge": ([_vp, _sz, _int, _int, _vp, _int, _vp, _vp], _int),
    "lbd_gemm_w4a16_g32": ([_vp, _int, _int, _vp, _vp, _vp, _int, _vp, _vp], _int),
    "lbd_gemm_w4a8_g32": ([_vp, _int, _int, _vp, _vp, _vp, _int, _vp, _vp], _int),
    "lbd_quantize_int4_g32": ([_vp, _int, _int, _int, _int, _vp, _vp, _vp, _vp], _int),
}


class LbdPlan(C.Structure):
    """lbd_plan of include/lowbit_hip.h: the regime and small-M kernel configuration a
    GEMM shape takes."""
    _fields_ = [(f, C.c_int) for f in ("path", "workgroups", "rows_per_wave", "rows_held", "chunks_per_lane",
                                       "two_rows_per_load", "act_rows", "k_slices")]


def gemm_plan(kind: str, m: int, n: int, kp: int, isa=None) -> dict:
    """The path and small-M kernel configuration (lbd_gemm_plan) a GEMM of this shape takes."""
    p = LbdPlan()
    prm = _Params(_isa_id(isa), 0, 0, 0, 0, 0, 0)
    _check(lib().lbd_gemm_plan(KIND_IDS[kind], m, n, kp, C.byref(prm), C.byref(p)), "lbd_gemm_plan", False)
    out = {f: getattr(p, f) for f, _ in LbdPlan._fields_}
    out["path"] = ISA_NAMES.get(p.path, "none")
    return out


class LbdFusion(C.Structure):
    """lbd_fusion of include/lowbit_hip.h: the prologue / epilogue of a fused GEMV
    (pass C.byref(f) as the `f` argument)."""
    _fields_ = [("norm_w", C.c_void_p), ("norm_eps", C.c_float), ("swiglu", C.c_int),
                ("bias", C.c_void_p), ("residual", C.c_void_p), ("argmax_key", C.c_void_p),
                ("glu", C.c_int), ("attn_part", C.c_void_p), ("attn_cap", C.c_int), ("attn_head_dim", C.c_int)]


@lru_cache(maxsize=1)
def lib() -> C.CDLL:
    """Load liblowbit_hip.so (raises if it was never built)."""
    so = C.CDLL(str(lib_path()))
    for name, (args, res) in SIGNATURES.items():
        fn = getattr(so, name)
        fn.argtypes = args
        fn.restype = res
    return so


def _err(rc: int, what: str):
    msg = lib().lb_last_error().decode(errors="replace")
    if rc in (-1, -2, -6):
        raise ValueError(f"{what} failed (rc={rc}): {msg}")
    raise RuntimeError(f"{what} failed (rc={rc}): {msg}")


_LAST = threading.local()


def _check(rc: int, what: str, record: bool = True) -> int:
    """Raise for rc < 0; a GEMM's rc (record=True) is the path last_path() reports."""
    if rc < 0:
        _err(rc, what)
    if record:
        _LAST.rc = rc
    return rc


def last_path() -> str:
    """Name of the path ("gfx950" or "gfx950-mfma") the calling thread's last GEMM ran on,
    the way the reference's GEMMs return the ISA they ran with (src/lowbit/csrc/dispatch.c:202)."""
    return ISA_NAMES.get(getattr(_LAST, "rc", -1), "none")


def device_info() -> dict:
    L = lib()
    name = C.create_string_buffer(64)
    cus, lds = _int(0), _int(0)
    _check(L.lb_device_info(name, 64, C.byref(cus), C.byref(lds)), "lb_device_info", False)
    return {"arch": name.value.decode(), "compute_units": cus.value, "lds_per_workgroup": lds.value}


def cpu_info() -> dict:
    """Library capabilities, with the reference's keys (src/lowbit/kernels.py:77-86).

    `cpu_isa` / `active_isa` name the best device path ("gfx950-mfma" on an
    MI355X); the CPU-only features report False / 1.
    """
    L = lib()
    top, act = L.lb_cpu_isa(), L.lb_active_isa()
    info = {
        "cpu_isa": ISA_NAMES.get(top, "none"),
        "active_isa": ISA_NAMES.get(act, "none"),
        "vnni": bool(L.lb_has_vnni()),
        "openmp": bool(L.lb_has_openmp()),
        "max_threads": L.lb_max_threads(),
        "amx": amx_available(),
    }
    if top >= 0:
        info.update(device_info())
    return info


def amx_available() -> bool:
    """The AMX tile path is CPU-only; the GPU library has none (src/lowbit/kernels.py:89-94)."""
    return False


def _isa_id(isa) -> int:
    if isa is None or isa == "auto" or isa in LEGACY_ISAS:
        return -1
    if isinstance(isa, int):
        return isa
    if isa not in ISA_IDS:
        raise ValueError(f"unknown isa {isa!r}; use one of {sorted(ISA_IDS)} or 'auto'")
    return ISA_IDS[isa]


def effective_isa(kind: str, isa=None) -> str:
    """Path name a GEMM kind runs with for a request (src/lowbit/kernels.py:103-104)."""
    rc = lib().lb_effective_isa(KIND_IDS[kind], _isa_id(isa))
    return ISA_NAMES.get(rc, "none")


def auto_params(kind: str, m: int, n: int, k: int, isa=None, threads=None) -> Params:
    """The reference resolves "auto" through its CPU tile cache (src/lowbit/kernels.py:110-116);
    the GPU kernels pick their tiles from the shape, so "auto" is the default Params."""
    return Params()


def _params(p, isa, threads, kind=None, shape=None) -> _Params:
    if isinstance(p, str):
        if p != "auto":
            raise ValueError(f"params must be a Params, None or 'auto', not {p!r}")
        p = auto_params(kind, *shape, isa=isa, threads=threads)
    p = p or Params()
    return _Params(_isa_id(isa), p.mr, p.nr, p.nb, p.kb, p.order, threads or 0)


def _zp(z: np.ndarray | None):
    return None if z is None else z.ctypes.data_as(C.c_void_p)


class _Prepared:
    """Padded, contiguous X plus an output buffer (src/lowbit/kernels.py:138-146)."""

    def __init__(self, x: np.ndarray, kp: int, n: int):
        x = np.asarray(x, np.float32)
        if x.ndim == 1:
            x = x[None]
        self.x = pad_acts(x, kp)
        self.y = np.empty((x.shape[0], n), np.float32)


# ------------------------------------------------------------------ device residency

class DeviceBuffer:
    """A device allocation owned by Python (freed when garbage collected)."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        p = _vp()
        _check(lib().lb_dev_malloc(C.byref(p), max(1, self.nbytes)), "lb_dev_malloc", False)
        self.ptr = p.value

    @classmethod
    def from_array(cls, a: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(a)
        b = cls(a.nbytes)
        if a.nbytes:
            _check(lib().lb_memcpy_h2d(b.ptr, a.ctypes.data, a.nbytes), "lb_memcpy_h2d", False)
        return b

    def to_array(self, shape, dtype) -> np.ndarray:
        out = np.empty(shape, dtype)
        if out.nbytes:
            _check(lib().lb_memcpy_d2h(out.ctypes.data, self.ptr, out.nbytes), "lb_memcpy_d2h", False)
        return out

    def __del__(self):
        try:
            if getattr(self, "ptr", None):
                lib().lb_dev_free(self.ptr)
                self.ptr = None
        except Exception:  # interpreter shutdown
            pass


_TILE_LOCK = threading.Lock()


@dataclass
class DeviceInt4Weights:
    """int4 g128 weights resident in HBM (same layout as Int4Weights).

    `t16` is the matrix-core tile layout of the same matrix (include/lowbit_hip.h,
    lbd_repack_int4_t16), built on the device the first time a GEMM takes the
    matrix-core path and kept beside the row-major copy, which the decode kernels
    read. `t16f8` is the layout W4A16 reads on the bf16 matrix cores
    (lbd_repack_int4_t16f8: each code less its zero-point as one E4M3 byte, twice the
    bytes of t16), built the same way; it holds the zero-points exactly only up to 15,
    so `zmax`, the largest zero-point (8 when symmetric, None when not known), chooses
    between the two for W4A16.
    """
    qw: DeviceBuffer
    scales: DeviceBuffer
    zeros: DeviceBuffer | None
    n: int
    kp: int
    k: int
    nbytes: int
    group: int = GROUP
    t16: tuple | None = None
    zmax: int | None = None
    t16f8: tuple | None = None

    def tiles(self) -> tuple:
        """(qwt, st, zt or None) in the t16 layout, repacked on first use (once, under a
        lock, and finished before it is returned: calls run on per-thread streams)."""
        if self.group != GROUP:
            raise ValueError("the t16 matrix-core layout holds groups of 128 only")
        with _TILE_LOCK:
            return self._tiles()

    def _tiles(self) -> tuple:
        if self.t16 is None:
            L = lib()
            bq, bs, bz = _sz(0), _sz(0), _sz(0)
            _check(L.lbd_int4_t16_bytes(self.n, self.kp, C.byref(bq), C.byref(bs), C.byref(bz)),
                   "lbd_int4_t16_bytes", False)
            qwt, st = DeviceBuffer(bq.value), DeviceBuffer(bs.value)
            zt = None if self.zeros is None else DeviceBuffer(bz.value)
            _check(L.lbd_repack_int4_t16(self.qw.ptr, self.scales.ptr,
                                         None if self.zeros is None else self.zeros.ptr, self.n, self.kp,
                                         qwt.ptr, st.ptr, None if zt is None else zt.ptr, None),
                   "lbd_repack_int4_t16", False)
            _check(L.lb_stream_synchronize(None), "lb_stream_synchronize", False)
            self.t16 = (qwt, st, zt)
        return self.t16

    def f8_exact(self) -> bool:
        """Whether the t16f8 layout holds this matrix exactly (every zero-point <= 15)."""
        return self.group == GROUP and self.zmax is not None and self.zmax <= 15

    def tiles_f8(self) -> tuple:
        """(qwt8, st) in the t16f8 layout, repacked on first use (as tiles())."""
        if not self.f8_exact():
            raise ValueError("the t16f8 layout needs groups of 128 and zero-points of at most 15")
        with _TILE_LOCK:
            if self.t16f8 is None:
                L = lib()
                bq, bs = _sz(0), _sz(0)
                _check(L.lbd_int4_t16f8_bytes(self.n, self.kp, C.byref(bq), C.byref(bs)), "lbd_int4_t16f8_bytes",
                       False)
                qwt8, st = DeviceBuffer(bq.value), DeviceBuffer(bs.value)
                _check(L.lbd_repack_int4_t16f8(self.qw.ptr, self.scales.ptr,
                                               None if self.zeros is None else self.zeros.ptr, self.n, self.kp,
                                               qwt8.ptr, st.ptr, None), "lbd_repack_int4_t16f8", False)
                _check(L.lb_stream_synchronize(None), "lb_stream_synchronize", False)
                self.t16f8 = (qwt8, st)
            return self.t16f8


@dataclass
class DeviceMXFP4Weights:
    """MXFP4 weights resident in HBM (same layout as MXFP4Weights); `t16` as for
    DeviceInt4Weights (lbd_repack_mxfp4_t16)."""
    qw: DeviceBuffer
    e8m0: DeviceBuffer
    n: int
    kp: int
    k: int
    nbytes: int
    t16: tuple | None = None

    def tiles(self) -> tuple:
        """(qwt, et) in the t16 layout, repacked on first use (as DeviceInt4Weights.tiles)."""
        with _TILE_LOCK:
            return self._tiles()

    def _tiles(self) -> tuple:
        if self.t16 is None:
            L = lib()
            bq, be = _sz(0), _sz(0)
            _check(L.lbd_mxfp4_t16_bytes(self.n, self.kp, C.byref(bq), C.byref(be)), "lbd_mxfp4_t16_bytes", False)
            qwt, et = DeviceBuffer(bq.value), DeviceBuffer(be.value)
            _check(L.lbd_repack_mxfp4_t16(self.qw.ptr, self.e8m0.ptr, self.n, self.kp, qwt.ptr, et.ptr, None),
                   "lbd_repack_mxfp4_t16", False)
            _check(L.lb_stream_synchronize(None), "lb_stream_synchronize", False)
            self.t16 = (qwt, et)
        return self.t16


def to_device(w):
    """Upload packed weights once; the returned handle is accepted by every gemm_*.

    The handle is a snapshot: later edits of the host arrays are not seen.
    """
    if isinstance(w, Int4Weights):
        zmax = 8 if w.zeros is None else int(w.zeros.max(initial=0))
        return DeviceInt4Weights(DeviceBuffer.from_array(w.qw), DeviceBuffer.from_array(w.scales),
                                 None if w.zeros is None else DeviceBuffer.from_array(w.zeros),
                                 w.n, w.kp, w.k, w.nbytes, w.group, zmax=zmax)
    if isinstance(w, MXFP4Weights):
        return DeviceMXFP4Weights(DeviceBuffer.from_array(w.qw), DeviceBuffer.from_array(w.e8m0),
                                  w.n, w.kp, w.k, w.nbytes)
    if isinstance(w, (DeviceInt4Weights, DeviceMXFP4Weights)):
        return w
    raise TypeError(f"cannot upload {type(w).__name__}")


def _device_fp32(w, shape):
    """(DeviceBuffer of fp32 [N, K], N, K) from a host array or a DeviceBuffer + shape."""
    if isinstance(w, DeviceBuffer):
        if shape is None or len(shape) != 2:
            raise ValueError("a DeviceBuffer needs shape=(N, K)")
        n, k = int(shape[0]), int(shape[1])
        if n * k * 4 > w.nbytes:
            raise ValueError(f"DeviceBuffer of {w.nbytes} bytes is smaller than fp32 {n}x{k}")
        return w, n, k
    a = np.ascontiguousarray(w, np.float32)
    if a.ndim != 2:
        raise ValueError("weights must be 2-D [N, K]")
    return DeviceBuffer.from_array(a), a.shape[0], a.shape[1]


def quantize_int4_device(w, asym: bool = False, scale: str = "absmax", shape=None,
                         stream=None, group: int = GROUP) -> "DeviceInt4Weights":
    """quantize_int4 run on the device (lbd_quantize_int4, or lbd_quantize_int4_g32 for
    group=32): the same packed bytes, scales and zero points as the host packer
    (src/lowbit/formats.py:90-142) for finite weights, left in HBM as a handle the
    GEMMs accept. `w` is a host array [N, K] (uploaded as fp32) or a DeviceBuffer
    holding fp32 [N, K] with shape=(N, K)."""
    if scale not in ("absmax", "signed-max"):
        raise ValueError(f"scale must be 'absmax' or 'signed-max', not {scale!r}")
    if asym and scale != "absmax":
        raise ValueError("scale='signed-max' is a symmetric rule (asym=False)")
    if group not in GROUPS:
        raise ValueError(f"group must be one of {GROUPS}, not {group!r}")
    src, n, k = _device_fp32(w, shape)
    kp = pad_to(k, group)
    g = kp // group
    qw, sc = DeviceBuffer(n * kp // 2), DeviceBuffer(n * g * 4)
    z = DeviceBuffer(n * g) if asym else None
    fn = lib().lbd_quantize_int4 if group == GROUP else lib().lbd_quantize_int4_g32
    _check(fn(src.ptr, n, k, int(asym), int(scale == "signed-max"), qw.ptr, sc.ptr, None if z is None else z.ptr,
              stream), "lbd_quantize_int4", False)
    # finished before the handle is returned: src may be freed next, and GEMMs on
    # other streams read the result
    _check(lib().lb_stream_synchronize(stream), "lb_stream_synchronize", False)
    nbytes = n * kp // 2 + n * g * 4 + (n * g if asym else 0)
    # the device packer clips zero-points to 0-15, as the host packer does
    return DeviceInt4Weights(qw, sc, z, n, kp, k, nbytes, group, zmax=15 if asym else 8)


def quantize_mxfp4_device(w, shape=None, stream=None) -> "DeviceMXFP4Weights":
    """quantize_mxfp4 run on the device (lbd_quantize_mxfp4): the same packed codes
    and E8M0 exponents as the host packer (src/lowbit/formats.py:197-212) for finite
    weights; `w` as for quantize_int4_device."""
    src, n, k = _device_fp32(w, shape)
    kp = pad_to(k, MXBLOCK)
    qw, e = DeviceBuffer(n * kp // 2), DeviceBuffer(n * kp // MXBLOCK)
    _check(lib().lbd_quantize_mxfp4(src.ptr, n, k, qw.ptr, e.ptr, stream), "lbd_quantize_mxfp4", False)
    _check(lib().lb_stream_synchronize(stream), "lb_stream_synchronize", False)
    return DeviceMXFP4Weights(qw, e, n, kp, k, n * kp // 2 + n * kp // MXBLOCK)


# ------------------------------------------------------------------ implicit residency

class _ResidencyState(threading.local):
    def __init__(self):
        self.enabled = os.environ.get("LOWBIT_RESIDENT", "1") != "0"


_RES_STATE = _ResidencyState()
_RES_LOCK = threading.RLock()  # re-entrant: a weakref callback may run inside the lock
# id(container) -> (weak reference to it, array key, device copy, arrays this package froze)
_RES: dict[int, tuple] = {}
RESIDENT_UPLOADS = [0]  # device copies made for host containers (a counter for tests and bench)


@contextlib.contextmanager
def implicit_residency(enabled: bool):
    """Within the block, gemm_* on host containers use (True) or bypass (False, the
    pointer ABI: weights uploaded per call) the cached device copy, on this thread."""
    prev = _RES_STATE.enabled
    _RES_STATE.enabled = bool(enabled)
    try:
        yield
    finally:
        _RES_STATE.enabled = prev


def _host_arrays(w) -> tuple:
    return (w.qw, w.scales, w.zeros) if isinstance(w, Int4Weights) else (w.qw, w.e8m0)


def _array_key(w) -> tuple:
    """What identifies the arrays a device copy was made from: each array object, its
    data pointer, shape and dtype (a replaced or reshaped array changes the key), and
    the container's logical K and group size."""
    key = tuple((id(a), a.ctypes.data, a.shape, a.dtype.str) if a is not None else None for a in _host_arrays(w))
    return key + (w.k, getattr(w, "group", None))


def _forget(wid: int):
    with _RES_LOCK:
        _RES.pop(wid, None)


def resident(w):
    """The device copy gemm_* uses for the host container `w` (Int4Weights or
    MXFP4Weights): made on first use, reused while the container holds the same arrays
    and those stay read-only, made again otherwise. Device handles pass through."""
    if isinstance(w, (DeviceInt4Weights, DeviceMXFP4Weights)):
        return w
    if not isinstance(w, (Int4Weights, MXFP4Weights)):
        raise TypeError(f"cannot make {type(w).__name__} resident")
    arrays = [a for a in _host_arrays(w) if a is not None]
    key = _array_key(w)
    with _RES_LOCK:
        ent = _RES.get(id(w))
        if ent is not None and ent[0]() is w and ent[1] == key and not any(a.flags.writeable for a in arrays):
            return ent[2]
        # freeze first, then copy: an edit can no longer land between the upload and
        # the next call without the caller making an array writeable again
        froze = [a for a in arrays if a.flags.writeable]
        if ent is not None and ent[0]() is w:
            froze = list({id(a): a for a in list(ent[3]) + froze}.values())
        for a in arrays:
            a.flags.writeable = False
        d = to_device(w)
        RESIDENT_UPLOADS[0] += 1
        wid = id(w)
        _RES[wid] = (weakref.ref(w, lambda _r, wid=wid: _forget(wid)), key, d, froze)
        return d


def release(w) -> bool:
    """Drop the device copy of host container `w` (freed when no call still uses it)
    and make writeable again the arrays the first GEMM made read-only. True if there
    was a copy."""
    with _RES_LOCK:
        ent = _RES.get(id(w))
        if ent is None or ent[0]() is not w:
            return False
        del _RES[id(w)]
    for a in ent[3]:
        try:
            a.flags.writeable = True
        except ValueError:  # a view whose base is read-only
            pass
    return True


def _use_resident(w, kind: str, m: int, prm: _Params) -> bool:
    """Whether this call takes the resident copy of a host container. The arguments
    are checked first, as the pointer ABI checks them before it reads any weights:
    a bad shape or micro-tile raises ValueError without an upload."""
    if not (_RES_STATE.enabled and isinstance(w, (Int4Weights, MXFP4Weights))):
        return False
    if w.n <= 0:
        raise ValueError(f"lbd_gemm_{kind} failed (rc=-1): bad shape (M, N, Kp <= 0 or Kp % block)")
    _check(lib().lbd_gemm_path(KIND_IDS[kind], m, w.kp, C.byref(prm)), f"lbd_gemm_{kind}", False)
    return True


class _Staging(threading.local):
    """Per-thread device staging for calls on resident weights: a stream and device
    buffers for X, Y and the matrix-core workspace, grown on demand and reused by
    every later call of the thread (so a call allocates nothing once warm)."""

    def __init__(self):
        self.stream = None
        self.bufs: dict[str, DeviceBuffer] = {}

    def get_stream(self):
        if self.stream is None:
            s = _vp()
            _check(lib().lb_stream_create(C.byref(s)), "lb_stream_create", False)
            self.stream = s.value
        return self.stream

    def buffer(self, name: str, nbytes: int) -> DeviceBuffer:
        b = self.bufs.get(name)
        if b is None or b.nbytes < nbytes:
            if b is not None:
                _check(lib().lb_stream_synchronize(self.get_stream()), "lb_stream_synchronize", False)
            b = DeviceBuffer(max(nbytes, 1 << 16))
            self.bufs[name] = b
        return b


_STAGE = _Staging()


def w4a16_uses_t16f8(w, m: int) -> bool:
    """Whether W4A16 at M = m on resident weights `w` reads the t16f8 copy: it holds
    the matrix exactly and the library expects it to be faster at this shape."""
    return w.f8_exact() and _check(lib().lbd_w4a16_prefers_t16f8(m, w.n, w.kp), "lbd_w4a16_prefers_t16f8",
                                   False) == 1


def gemm_w4a16_tiles(w, dx: int, m: int, dy: int, prm: _Params, ws: int, ws_bytes: int, stream) -> int:
    """W4A16 on the bf16 matrix cores for resident weights `w`: lbd_gemm_w4a16_t16f8 on
    the t16f8 copy where w4a16_uses_t16f8, else lbd_gemm_w4a16_t16 on the t16 copy (the
    same results bit for bit). Returns the C call's code."""
    L = lib()
    if w4a16_uses_t16f8(w, m):
        qwt8, st = w.tiles_f8()
        return L.lbd_gemm_w4a16_t16f8(dx, m, w.kp, qwt8.ptr, st.ptr, w.n, dy, C.byref(prm), ws, ws_bytes, stream)
    qwt, st, zt = w.tiles()
    return L.lbd_gemm_w4a16_t16(dx, m, w.kp, qwt.ptr, st.ptr, None if zt is None else zt.ptr, w.n, dy,
                                C.byref(prm), ws, ws_bytes, stream)


def _run_dev(kind: str, w, m: int, dx: int, dy: int, prm: _Params, stream) -> int:
    """Launch one GEMM on resident weights `w` (device pointers dx / dy) on `stream`;
    the matrix-core regime reads the t16 tile layout, repacked on first use."""
    L = lib()
    zp = None if getattr(w, "zeros", None) is None else w.zeros.ptr
    mfma = _check(L.lbd_gemm_path(KIND_IDS[kind], m, w.kp, C.byref(prm)), "lbd_gemm_path", False) == ISA_GFX950_MFMA
    if kind in ("w4a16", "mxfp4") and mfma:
        ws = _STAGE.buffer("ws", L.lbd_bf16x3_workspace_bytes_split(KIND_IDS[kind], m, w.n, w.kp))
        if kind == "w4a16":
            return gemm_w4a16_tiles(w, dx, m, dy, prm, ws.ptr, ws.nbytes, stream)
        qwt, et = w.tiles()
        return L.lbd_gemm_mxfp4_t16(dx, m, w.kp, qwt.ptr, et.ptr, w.n, dy, C.byref(prm), ws.ptr, ws.nbytes, stream)
    if kind == "w4a16":
        return L.lbd_gemm_w4a16(dx, m, w.kp, w.qw.ptr, w.scales.ptr, zp, w.n, dy, C.byref(prm), stream)
    if kind == "mxfp4":
        return L.lbd_gemm_mxfp4(dx, m, w.kp, w.qw.ptr, w.e8m0.ptr, w.n, dy, C.byref(prm), stream)
    ws = _STAGE.buffer("ws", L.lbd_w4a8_workspace_bytes(m, w.kp))
    if mfma:
        qwt, st, zt = w.tiles()
        return L.lbd_gemm_w4a8_t16(dx, m, w.kp, qwt.ptr, st.ptr, None if zt is None else zt.ptr, w.n, dy,
                                   C.byref(prm), ws.ptr, ws.nbytes, stream)
    return L.lbd_gemm_w4a8(dx, m, w.kp, w.qw.ptr, w.scales.ptr, zp, w.n, dy, C.byref(prm), ws.ptr, ws.nbytes,
                           stream)


def _dev_gemm(kind: str, pr: _Prepared, w, prm: _Params) -> np.ndarray:
    """One call on resident weights: X up, the GEMM, Y down, all on the calling thread's
    stream and staging buffers, then a synchronisation (the reference's calls are
    synchronous, src/lowbit/kernels.py:127-135)."""
    L = lib()
    m = pr.x.shape[0]
    s = _STAGE.get_stream()
    dx = _STAGE.buffer("x", pr.x.nbytes)
    dy = _STAGE.buffer("y", pr.y.nbytes)
    _check(L.lb_memcpy_h2d_async(dx.ptr, pr.x.ctypes.data, pr.x.nbytes, s), "lb_memcpy_h2d_async", False)
    _check(_run_dev(kind, w, m, dx.ptr, dy.ptr, prm, s), f"lbd_gemm_{kind}")
    _check(L.lb_memcpy_d2h_async(pr.y.ctypes.data, dy.ptr, pr.y.nbytes, s), "lb_memcpy_d2h_async", False)
    _check(L.lb_stream_synchronize(s), "lb_stream_synchronize", False)
    return pr.y


def _dev_gemm_q(a: Int8Acts, w, prm: _Params, y: np.ndarray) -> np.ndarray:
    """gemm_w4a8_q on resident weights: codes, token scales and group sums up, the GEMM
    (lbd_gemm_w4a8_q), Y down, on the calling thread's stream."""
    L = lib()
    m = a.xq.shape[0]
    xq = np.ascontiguousarray(a.xq, np.int8)
    xs = np.ascontiguousarray(a.scale, np.float32)
    gs = np.ascontiguousarray(a.gsum, np.int32)
    s = _STAGE.get_stream()
    dq, ds, dg = _STAGE.buffer("xq", xq.nbytes), _STAGE.buffer("xs", xs.nbytes), _STAGE.buffer("gs", gs.nbytes)
    dy = _STAGE.buffer("y", y.nbytes)
    for d, h in ((dq, xq), (ds, xs), (dg, gs)):
        _check(L.lb_memcpy_h2d_async(d.ptr, h.ctypes.data, h.nbytes, s), "lb_memcpy_h2d_async", False)
    _check(L.lbd_gemm_w4a8_q(dq.ptr, ds.ptr, dg.ptr, m, w.kp, w.qw.ptr, w.scales.ptr,
                             None if w.zeros is None else w.zeros.ptr, w.n, dy.ptr, C.byref(prm), s),
           "lbd_gemm_w4a8_q")
    _check(L.lb_memcpy_d2h_async(y.ctypes.data, dy.ptr, y.nbytes, s), "lb_memcpy_d2h_async", False)
    _check(L.lb_stream_synchronize(s), "lb_stream_synchronize", False)
    return y


def _g32_gemm(kind: str, pr: _Prepared, w) -> np.ndarray:
    """Group-32 int4 GEMMs (lbd_gemm_w4a16_g32 / lbd_gemm_w4a8_g32): host containers
    are uploaded for the call, device handles used in place."""
    d = w if isinstance(w, DeviceInt4Weights) else to_device(w)
    L = lib()
    m = pr.x.shape[0]
    s = _STAGE.get_stream()
    dx = _STAGE.buffer("x", pr.x.nbytes)
    dy = _STAGE.buffer("y", pr.y.nbytes)
    _check(L.lb_memcpy_h2d_async(dx.ptr, pr.x.ctypes.data, pr.x.nbytes, s), "lb_memcpy_h2d_async", False)
    fn = L.lbd_gemm_w4a16_g32 if kind == "w4a16" else L.lbd_gemm_w4a8_g32
    _check(fn(dx.ptr, m, d.kp, d.qw.ptr, d.scales.ptr, None if d.zeros is None else d.zeros.ptr, d.n, dy.ptr, s),
           f"lbd_gemm_{kind}_g32")
    _check(L.lb_memcpy_d2h_async(pr.y.ctypes.data, dy.ptr, pr.y.nbytes, s), "lb_memcpy_d2h_async", False)
    _check(L.lb_stream_synchronize(s), "lb_stream_synchronize", False)
    return pr.y


def _int4_group(w) -> int:
    return getattr(w, "group", GROUP)


# ------------------------------------------------------------------ GEMMs

def gemm_w4a16(x, w, params: Params | None = None, isa=None, threads: int | None = None,
               _prep: _Prepared | None = None) -> np.ndarray:
    """Y = X @ dequant(W)^T, fp32 activations and accumulation (src/lowbit/kernels.py:149-156)."""
    pr = _prep or _Prepared(x, w.kp, w.n)
    prm = _params(params, isa, threads, "w4a16", (pr.x.shape[0], w.n, w.k))
    if _use_resident(w, "w4a16", pr.x.shape[0], prm):
        w = resident(w)
    if _int4_group(w) != GROUP:
        return _g32_gemm("w4a16", pr, w)
    if isinstance(w, DeviceInt4Weights):
        return _dev_gemm("w4a16", pr, w, prm)
    rc = lib().lb_gemm_w4a16(pr.x, pr.x.shape[0], w.kp, w.qw, w.scales, _zp(w.zeros), w.n, pr.y,
                             C.byref(prm))
    _check(rc, "lb_gemm_w4a16")
    return pr.y


def gemm_mxfp4(x, w, params: Params | None = None, isa=None, threads: int | None = None,
               _prep: _Prepared | None = None) -> np.ndarray:
    """Y = X @ dequant(W)^T for OCP MXFP4 weights (src/lowbit/kernels.py:159-166)."""
    pr = _prep or _Prepared(x, w.kp, w.n)
    prm = _params(params, isa, threads, "mxfp4", (pr.x.shape[0], w.n, w.k))
    if _use_resident(w, "mxfp4", pr.x.shape[0], prm):
        w = resident(w)
    if isinstance(w, DeviceMXFP4Weights):
        return _dev_gemm("mxfp4", pr, w, prm)
    rc = lib().lb_gemm_mxfp4(pr.x, pr.x.shape[0], w.kp, w.qw, w.e8m0, w.n, pr.y, C.byref(prm))
    _check(rc, "lb_gemm_mxfp4")
    return pr.y


def gemm_w4a8(x, w, params: Params | None = None, isa=None, threads: int | None = None,
              _prep: _Prepared | None = None) -> np.ndarray:
    """fp32 X in; X is quantized per token to int8 on the device inside the call
    (src/lowbit/kernels.py:169-177)."""
    pr = _prep or _Prepared(x, w.kp, w.n)
    prm = _params(params, isa, threads, "w4a8", (pr.x.shape[0], w.n, w.k))
    if _use_resident(w, "w4a8", pr.x.shape[0], prm):
        w = resident(w)
    if _int4_group(w) != GROUP:
        return _g32_gemm("w4a8", pr, w)
    if isinstance(w, DeviceInt4Weights):
        return _dev_gemm("w4a8", pr, w, prm)
    rc = lib().lb_gemm_w4a8(pr.x, pr.x.shape[0], w.kp, w.qw, w.scales, _zp(w.zeros), w.n, pr.y,
                            C.byref(prm))
    _check(rc, "lb_gemm_w4a8")
    return pr.y


def gemm_w4a8_q(a: Int8Acts, w: Int4Weights, params: Params | None = None, isa=None,
                threads: int | None = None) -> np.ndarray:
    """W4A8 on already-quantized activations (src/lowbit/kernels.py:180-187)."""
    if _int4_group(w) != GROUP:
        raise ValueError("gemm_w4a8_q takes the reference's group-128 weights and group sums")
    y = np.empty((a.xq.shape[0], w.n), np.float32)
    prm = _params(params, isa, threads, "w4a8", (a.xq.shape[0], w.n, w.k))
    if isinstance(w, DeviceInt4Weights) or _use_resident(w, "w4a8", a.xq.shape[0], prm):
        return _dev_gemm_q(a, resident(w), prm, y)
    rc = lib().lb_gemm_w4a8_q(np.ascontiguousarray(a.xq), np.ascontiguousarray(a.scale, np.float32),
                              np.ascontiguousarray(a.gsum, np.int32), a.xq.shape[0], w.kp, w.qw,
                              w.scales, _zp(w.zeros), w.n, y, C.byref(prm))
    _check(rc, "lb_gemm_w4a8_q")
    return y


def quant_act_int8(x: np.ndarray, kp: int) -> Int8Acts:
    """The device per-token int8 quantizer (src/lowbit/kernels.py:190-197)."""
    xp = pad_acts(np.atleast_2d(x), kp)
    m = xp.shape[0]
    xq = np.empty((m, kp), np.int8)
    xs = np.empty(m, np.float32)
    gs = np.empty((m, kp // GROUP), np.int32)
    L = lib()
    L.lb_quant_act_int8(xp, m, kp, xq, xs, gs)
    _check(L.lb_last_status(), "lb_quant_act_int8")
    return Int8Acts(xq, xs, gs)


def w4a8_group_acc(a: Int8Acts, w: Int4Weights, isa=None) -> np.ndarray:
    """Exact int32 group accumulators [M, N, G] from the device integer path named by
    `isa` ("gfx950" dot4 VALU, "gfx950-mfma" int8 MFMA) (src/lowbit/kernels.py:200-205)."""
    if _int4_group(w) != GROUP:
        raise ValueError("w4a8_group_acc takes the reference's group-128 weights")
    m = a.xq.shape[0]
    out = np.empty((m, w.n, w.kp // GROUP), np.int32)
    _check(lib().lb_w4a8_group_acc(np.ascontiguousarray(a.xq), np.ascontiguousarray(a.gsum, np.int32),
                                   m, w.kp, w.qw, _zp(w.zeros), w.n, out, _isa_id(isa)),
           "lb_w4a8_group_acc")
    return out


GEMMS = {"w4a16": gemm_w4a16, "mxfp4": gemm_mxfp4, "w4a8": gemm_w4a8}
BLOCKS = {"w4a16": GROUP, "mxfp4": MXBLOCK, "w4a8": GROUP}
