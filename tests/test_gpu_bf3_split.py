"""The bf16x3 GEMMs with K split over the workgroups of a column (rows of at least
8192 elements, a workspace of lbd_bf16x3_workspace_bytes_split bytes or NULL),
against the float64 oracle within the reference's bound (tests/test_kernels.py:
29-67 of the reference), against the unsplit GEMM of the same call with the smaller
workspace (same bound; the sums are associated differently), and t16 against t16f8
bit for bit with both split alike."""
import ctypes as C

import numpy as np
import pytest

import lowbit_amd as lb
from lowbit_amd import kernels as K
from oracle import reference as O

pytestmark = pytest.mark.gpu


def _run(fmt, D, x, m, split, f8=False):
    """split True: a workspace of lbd_bf16x3_workspace_bytes_split bytes; False: of
    lbd_bf16x3_workspace_bytes; None: no workspace (the library's per-thread buffer)."""
    L = K.lib()
    dx = K.DeviceBuffer.from_array(x)
    dy = K.DeviceBuffer(m * D.n * 4)
    kind = 0 if fmt == "w4a16" else 1
    nb = L.lbd_bf16x3_workspace_bytes_split(kind, m, D.n, D.kp) if split else L.lbd_bf16x3_workspace_bytes(m, D.kp)
    ws = K.DeviceBuffer(nb) if split is not None else None
    wp, nb = (ws.ptr, nb) if ws is not None else (None, 0)
    prm = K._Params(-1, 0, 0, 0, 0, 0, 0)
    if fmt == "mxfp4":
        qwt, et = D.tiles()
        rc = L.lbd_gemm_mxfp4_t16(dx.ptr, m, D.kp, qwt.ptr, et.ptr, D.n, dy.ptr, C.byref(prm), wp, nb, None)
    elif f8:
        qwt8, st8 = D.tiles_f8()
        rc = L.lbd_gemm_w4a16_t16f8(dx.ptr, m, D.kp, qwt8.ptr, st8.ptr, D.n, dy.ptr, C.byref(prm), wp, nb, None)
    else:
        qwt, st, zt = D.tiles()
        rc = L.lbd_gemm_w4a16_t16(dx.ptr, m, D.kp, qwt.ptr, st.ptr, None if zt is None else zt.ptr, D.n, dy.ptr,
                                  C.byref(prm), wp, nb, None)
    assert rc == K.ISA_GFX950_MFMA
    assert L.lb_dev_synchronize() == 0
    return dy.to_array((m, D.n), np.float32)


@pytest.mark.parametrize("fmt,asym", [("w4a16", False), ("w4a16", True), ("mxfp4", False)])  # MXFP4: no zero-point
@pytest.mark.parametrize("m,n,k", [(16, 520, 11008), (64, 300, 11008), (5, 77, 8200), (16, 96, 16384),
                                   (128, 200, 11008)])
def test_split_within_bound(rng, fmt, asym, m, n, k):
    x = rng.standard_normal((m, k)).astype(np.float32)
    w = (rng.standard_normal((n, k)) * rng.lognormal(0, 0.5, (n, 1))).astype(np.float32)
    W = lb.quantize_mxfp4(w) if fmt == "mxfp4" else lb.quantize_int4(w, asym=asym)
    D = lb.to_device(W)
    xp = lb.formats.pad_acts(x, W.kp)
    dense = O.dequant_mxfp4(W.qw, W.e8m0) if fmt == "mxfp4" else O.dequant_int4(W.qw, W.scales, W.zeros)
    ref, bound = xp.astype(np.float64) @ dense.T, O.fp_bound(xp, dense)
    ys = _run(fmt, D, xp, m, True)
    yu = _run(fmt, D, xp, m, False)
    O.assert_fp_close(ys, ref, bound, 1e-5)
    O.assert_fp_close(yu, ref, bound, 1e-5)
    if fmt == "w4a16" and D.f8_exact():
        np.testing.assert_array_equal(_run(fmt, D, xp, m, True, f8=True), ys)
    # no workspace: the per-thread buffer has room for the partial outputs, so the
    # call takes the split, bit for bit the result with a split-sized workspace
    np.testing.assert_array_equal(_run(fmt, D, xp, m, None), ys)
    # the Python call takes the split (its staging workspace has room for it)
    y = K.gemm_mxfp4(x, D) if fmt == "mxfp4" else K.gemm_w4a16(x, D)
    np.testing.assert_array_equal(y, ys)
