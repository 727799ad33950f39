"""The allocation-free W4A8 entry point (GPU), through the C ABI.

lbd_gemm_w4a8_t16_noalloc must give, bit for bit, what lbd_gemm_w4a8_t16 gives with a
workspace of its own, on two calls in a row on one device (the second smaller, so
the scratch array still holds the first call's larger contents), and both must stay
within the reference's W4A8 bound (tests/test_kernels.py:108-119 of the reference).
"""
import ctypes as C

import numpy as np
import pytest

import lowbit_amd as lb
from lowbit_amd import kernels as K
from oracle import cref
from oracle import reference as O

pytestmark = pytest.mark.gpu


def _call(L, fn_name, dx, m, D, dy, ws=None):
    qwt, st, zt = D.tiles()
    prm = K._Params(-1, 0, 0, 0, 0, 0, 0)
    zp = None if zt is None else zt.ptr
    if fn_name == "noalloc":
        rc = L.lbd_gemm_w4a8_t16_noalloc(dx.ptr, m, D.kp, qwt.ptr, st.ptr, zp, D.n, dy.ptr, C.byref(prm), None)
    else:
        rc = L.lbd_gemm_w4a8_t16(dx.ptr, m, D.kp, qwt.ptr, st.ptr, zp, D.n, dy.ptr, C.byref(prm), ws.ptr, ws.nbytes,
                                 None)
    assert rc == K.ISA_GFX950_MFMA, (rc, L.lb_last_error())
    assert L.lb_stream_synchronize(None) == 0


@pytest.mark.parametrize("asym", [True, False])
def test_noalloc_matches_workspace_entry_point(rng, asym):
    L = K.lib()
    n, k = 4096, 4096
    W = lb.quantize_int4(rng.standard_normal((n, k)).astype(np.float32), asym=asym)
    D = lb.to_device(W)
    for m in (64, 17):  # the second call is smaller than the first
        print(f"noalloc call M={m} N={n} K={k} asym={asym}", flush=True)
        x = rng.standard_normal((m, k)).astype(np.float32)
        dx = K.DeviceBuffer.from_array(x)
        y_ws, y_na = K.DeviceBuffer(m * n * 4), K.DeviceBuffer(m * n * 4)
        ws = K.DeviceBuffer(L.lbd_w4a8_workspace_bytes(m, k))
        _call(L, "workspace", dx, m, D, y_ws, ws)
        _call(L, "noalloc", dx, m, D, y_na)
        a, b = y_ws.to_array((m, n), np.float32), y_na.to_array((m, n), np.float32)
        np.testing.assert_array_equal(b, a)
        q = lb.quantize_act_int8(x)
        ref, bound = cref.c_gemm_w4a8(q.xq, q.scale, q.gsum, W.qw, W.scales, W.zeros)
        O.assert_fp_close(b, ref, bound, 1e-5)


def test_noalloc_rejects_sizes_past_its_scratch():
    L = K.lib()
    cap = L.lbd_noalloc_scratch_bytes()
    assert cap == 8 << 20
    m, kp = 4096, 4096  # 16 MiB of int8 codes
    assert L.lbd_w4a8_workspace_bytes(m, kp) > cap
    fake = 1 << 20  # never dereferenced: the size check comes first
    prm = K._Params(-1, 0, 0, 0, 0, 0, 0)
    rc = L.lbd_gemm_w4a8_t16_noalloc(fake, m, kp, fake, fake, None, 16, fake, C.byref(prm), None)
    assert rc == -1 and "scratch" in L.lb_last_error().decode()
