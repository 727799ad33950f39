"""Implicit device residency of host containers, and the pointer ABI's batch path.

The reference's callers pass host containers to every GEMM (its decoder's linear
layers call gemm_*(x, self.wq), src/lowbit/model.py:139-141). lowbit_amd makes such
a container resident on its first GEMM and reuses the device copy while the
container holds the same arrays and those stay read-only (the first GEMM marks them
read-only). These tests pin that contract:

* one upload per container, results bit for bit those of an explicit to_device
  handle, in every format and both regimes;
* an in-place edit after a GEMM raises (the copy can never be silently stale); an
  edit made after setting `flags.writeable = True`, a replaced array, or release()
  makes the next GEMM upload again and see the edit (the reference edits W.qw in
  place before its GEMMs, tests/test_kernels.py:81-97);
* implicit_residency(False) runs the host-pointer ABI (lb_gemm_*), whose matrix-core
  calls repack the uploaded weights to t16 inside the call and take the bf16x3 path:
  bit for bit the resident result;
* the fp32 MFMA kernel, which only row-major device pointers at M >= 5 still reach
  (lbd_gemm_w4a16 / lbd_gemm_mxfp4), within the reference's bound.
"""
import ctypes as C

import numpy as np
import pytest

import lowbit_amd as lb
from lowbit_amd import kernels as K
from oracle import cref
from oracle import reference as O

pytestmark = pytest.mark.gpu

FORMATS = ["w4a16", "w4a8", "mxfp4"]


def _w(rng, fmt, n, k, asym=True, group=128):
    w = rng.standard_normal((n, k)).astype(np.float32)
    if fmt == "mxfp4":
        return lb.quantize_mxfp4(w)
    return lb.quantize_int4(w, asym=asym, group=group)


def uploads():
    return K.RESIDENT_UPLOADS[0]


@pytest.mark.parametrize("fmt", FORMATS)
@pytest.mark.parametrize("m", [1, 3, 16, 64])
def test_one_upload_and_handle_results(rng, fmt, m):
    W = _w(rng, fmt, 1100, 1024)
    x = rng.standard_normal((m, 1024)).astype(np.float32)
    fn = K.GEMMS[fmt]
    want = fn(x, lb.to_device(W))
    n0 = uploads()
    y1 = fn(x, W).copy()
    assert uploads() == n0 + 1
    y2 = fn(x, W).copy()
    assert uploads() == n0 + 1  # reused
    np.testing.assert_array_equal(y1, want)
    np.testing.assert_array_equal(y2, want)
    assert not W.qw.flags.writeable


def test_in_place_edit_raises_then_uploads_again(rng):
    W = _w(rng, "w4a8", 300, 512)
    x = rng.standard_normal((1, 512)).astype(np.float32)
    y0 = K.gemm_w4a8(x, W).copy()
    with pytest.raises(ValueError):
        W.qw[0, 0] ^= 0xFF          # read-only: the edit cannot go unseen
    n0 = uploads()
    W.qw.flags.writeable = True     # the caller says it means to edit
    W.zeros.flags.writeable = True
    W.qw[0, :] ^= 0x5A
    W.zeros[1, 0] = 3
    y1 = K.gemm_w4a8(x, W).copy()
    assert uploads() == n0 + 1
    np.testing.assert_array_equal(y1, K.gemm_w4a8(x, lb.to_device(W)))
    assert not np.array_equal(y1[0, :2], y0[0, :2])
    np.testing.assert_array_equal(y1[0, 2:], y0[0, 2:])
    assert not W.qw.flags.writeable  # frozen again


@pytest.mark.parametrize("fmt", FORMATS)
def test_replaced_array_uploads_again(rng, fmt):
    W = _w(rng, fmt, 200, 256)
    x = rng.standard_normal((2, 256)).astype(np.float32)
    fn = K.GEMMS[fmt]
    fn(x, W)
    n0 = uploads()
    if fmt == "mxfp4":
        W.e8m0 = (W.e8m0.astype(np.int32) + 1).astype(np.uint8)
    else:
        W.scales = (W.scales * np.float32(2.0)).astype(np.float32)
    y = fn(x, W).copy()
    assert uploads() == n0 + 1
    np.testing.assert_array_equal(y, fn(x, lb.to_device(W)))


def test_release_restores_writeable_arrays(rng):
    W = _w(rng, "w4a16", 128, 384, asym=False)
    x = rng.standard_normal((1, 384)).astype(np.float32)
    K.gemm_w4a16(x, W)
    assert not W.qw.flags.writeable and not W.scales.flags.writeable
    assert K.release(W) and not K.release(W)
    assert W.qw.flags.writeable and W.scales.flags.writeable
    W.scales[:] = np.float32(0.5)
    n0 = uploads()
    y = K.gemm_w4a16(x, W)
    assert uploads() == n0 + 1
    np.testing.assert_array_equal(y, K.gemm_w4a16(x, lb.to_device(W)))


def test_arrays_read_only_before_stay_so_after_release(rng):
    W = _w(rng, "w4a16", 64, 256)
    W.zeros.flags.writeable = False   # the caller's own read-only array
    K.gemm_w4a16(rng.standard_normal((1, 256)).astype(np.float32), W)
    K.release(W)
    assert W.qw.flags.writeable and not W.zeros.flags.writeable


def test_reference_edit_before_first_gemm(rng):
    """The reference's worst-case fixture edits W.qw and W.zeros in place before any
    GEMM (tests/test_kernels.py:81-97); the first GEMM uploads the edited arrays."""
    m, n, k = 3, 4, 512
    W = lb.quantize_int4(np.zeros((n, k), np.float32), asym=True)
    codes = np.zeros((n, k), np.uint8)
    codes[0] = 15
    codes[1, ::2] = 15
    codes[2] = np.arange(k) % 16
    W.qw[:] = lb.formats.pack_nibbles(codes, 128)
    W.zeros[:] = np.array([0, 15, 7, 8], np.uint8)[:, None]
    W.scales[:] = np.float32(1.0)
    xq = np.full((m, k), 127, np.int8)
    xq[1] = -127
    a = lb.Int8Acts(xq, np.ones(m, np.float32), xq.astype(np.int32).reshape(m, -1, 128).sum(-1).astype(np.int32))
    y = K.gemm_w4a8_q(a, W)
    ref = O.gemm_w4a8_ref(a.xq, a.scale, W.qw, W.scales, W.zeros)
    np.testing.assert_array_equal(y, ref.astype(np.float32))  # small integers: exact


def test_group32_container(rng):
    W = _w(rng, "w4a16", 300, 1024, group=32)
    x = rng.standard_normal((1, 1024)).astype(np.float32)
    n0 = uploads()
    y = K.gemm_w4a16(x, W)
    K.gemm_w4a8(x, W)
    assert uploads() == n0 + 1
    np.testing.assert_array_equal(y, K.gemm_w4a16(x, lb.to_device(W)))


@pytest.mark.parametrize("m", [1, 16, 64])
def test_w4a8_q_resident_equals_pointer(rng, m):
    W = _w(rng, "w4a8", 700, 1024)
    a = lb.quantize_act_int8(rng.standard_normal((m, 1024)).astype(np.float32))
    y = K.gemm_w4a8_q(a, W).copy()
    with K.implicit_residency(False):
        np.testing.assert_array_equal(y, K.gemm_w4a8_q(a, W))


@pytest.mark.parametrize("fmt", ["w4a16", "mxfp4"])
@pytest.mark.parametrize("m,n,k", [(16, 1100, 4096), (64, 4096, 4096), (16, 520, 11008), (5, 77, 1024)])
def test_pointer_abi_batch_takes_bf16x3(rng, fmt, m, n, k):
    """The host-pointer ABI at M >= 5 repacks the uploaded weights to t16 in the call
    and runs the same bf16x3 GEMM (with the K split where the shape takes it) as a
    resident handle: the same bits."""
    W = _w(rng, fmt, n, k, asym=(m == 16))
    x = rng.standard_normal((m, k)).astype(np.float32)
    fn = K.GEMMS[fmt]
    want = fn(x, lb.to_device(W))
    with K.implicit_residency(False):
        y = fn(x, W)
        assert K.last_path() == "gfx950-mfma"
    np.testing.assert_array_equal(y, want)


@pytest.mark.parametrize("fmt", ["w4a16", "mxfp4"])
@pytest.mark.parametrize("m,n,k", [(16, 300, 4096), (40, 129, 1024)])
def test_row_major_device_batch_fp32_mfma(rng, fmt, m, n, k):
    """Row-major device pointers at M >= 5 (lbd_gemm_w4a16 / lbd_gemm_mxfp4, no
    workspace argument) still run the fp32 MFMA kernel: within 1e-5 (|X| @ |W|^T)."""
    W = _w(rng, fmt, n, k)
    D = lb.to_device(W)
    x = rng.standard_normal((m, k)).astype(np.float32)
    L = K.lib()
    dx, dy = K.DeviceBuffer.from_array(x), K.DeviceBuffer(4 * m * n)
    prm = K._Params(-1, 0, 0, 0, 0, 0, 0)
    if fmt == "mxfp4":
        rc = L.lbd_gemm_mxfp4(dx.ptr, m, D.kp, D.qw.ptr, D.e8m0.ptr, n, dy.ptr, C.byref(prm), None)
        ref, bound = cref.c_gemm_mxfp4(x, W.qw, W.e8m0), cref.c_gemm_mxfp4(x, W.qw, W.e8m0, absval=True)
    else:
        rc = L.lbd_gemm_w4a16(dx.ptr, m, D.kp, D.qw.ptr, D.scales.ptr, D.zeros.ptr, n, dy.ptr, C.byref(prm), None)
        ref = cref.c_gemm_w4a16(x, W.qw, W.scales, W.zeros)
        bound = cref.c_gemm_w4a16(x, W.qw, W.scales, W.zeros, absval=True)
    assert rc == K.ISA_GFX950_MFMA
    assert L.lb_stream_synchronize(None) == 0
    O.assert_fp_close(dy.to_array((m, n), np.float32), ref, bound, 1e-5)
