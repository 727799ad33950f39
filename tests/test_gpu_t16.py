"""The matrix-core tile layout (t16) of int4 weights and the W4A8 GEMM that reads it.

The layout is this library's own (include/lowbit_hip.h, lbd_repack_int4_t16), so
it is pinned two ways: the repacked bytes against a direct statement of the
documented order, and the GEMM on t16 weights against the same GEMM on the
row-major matrix (bit for bit: both run the same arithmetic in the same order)
and against the float64 oracle within the reference's W4A8 bound.
"""
import numpy as np
import pytest

import lowbit_amd as lb
from lowbit_amd import kernels as K
from oracle import cref
from oracle import reference as O

pytestmark = pytest.mark.gpu


def t16_expected(W):
    """The documented t16 order, element by element (include/lowbit_hip.h)."""
    n, kp = W.n, W.kp
    g = kp // 128
    g4 = (g + 3) // 4 * 4
    s = (n + 15) // 16
    qw = np.zeros((s * 16, g4 * 64), np.uint8)
    qw[:n, :g * 64] = W.qw
    # [s][c][g][q][16] -> [s][g][q][c][16]
    qwt = qw.reshape(s, 16, g4, 4, 16).transpose(0, 2, 3, 1, 4).reshape(-1)
    def groups(a, dtype):
        full = np.zeros((s * 16, g4), dtype)
        full[:n, :g] = a
        # [s][c][g/4][4] -> [s][g/4][c][4]
        return full.reshape(s, 16, g4 // 4, 4).transpose(0, 2, 1, 3).reshape(-1)
    return qwt, groups(W.scales, np.float32), None if W.zeros is None else groups(W.zeros, np.uint8)


def _random_int4(rng, n, kp, asym):
    g = kp // 128
    return lb.formats.Int4Weights(
        rng.integers(0, 256, (n, kp // 2), dtype=np.uint8),
        (rng.standard_normal((n, g)) * 0.05).astype(np.float32),
        rng.integers(0, 16, (n, g), dtype=np.uint8) if asym else None, kp)


@pytest.mark.parametrize("n,kp,asym", [(16, 512, True), (33, 256, False), (70, 1152, True), (300, 4352, True)])
def test_t16_repack_matches_documented_layout(rng, n, kp, asym):
    W = _random_int4(rng, n, kp, asym)
    D = lb.to_device(W)
    qwt, st, zt = D.tiles()
    eq, es, ez = t16_expected(W)
    np.testing.assert_array_equal(qwt.to_array(eq.shape, np.uint8), eq)
    np.testing.assert_array_equal(st.to_array(es.shape, np.float32), es)
    if asym:
        np.testing.assert_array_equal(zt.to_array(ez.shape, np.uint8), ez)
    else:
        assert zt is None


# (M, N, Kp, asym): row-block heights 16/32/64 rows, M tails, N tails, groups padded
# to a multiple of 4 (G = 2, 9, 34), a second K phase (G = 34) and many subtiles.
T16 = [(5, 33, 256, True), (16, 11008, 4096, True), (17, 70, 1152, False), (64, 11008, 4096, True),
       (70, 4100, 4352, False), (64, 33000, 4096, True), (40, 96, 512, True), (33, 20, 256, False)]


@pytest.mark.parametrize("m,n,kp,asym", T16)
def test_w4a8_t16_matches_row_major_and_oracle(rng, m, n, kp, asym):
    W = _random_int4(rng, n, kp, asym)
    x = rng.standard_normal((m, kp)).astype(np.float32)
    D = lb.to_device(W)
    y16 = K.gemm_w4a8(x, D, isa="gfx950-mfma")
    assert K.last_path() == "gfx950-mfma" and D.t16 is not None
    y = K.gemm_w4a8(x, W, isa="gfx950-mfma")
    np.testing.assert_array_equal(y16, y)
    a = lb.quantize_act_int8(x)
    ref, bound = cref.c_gemm_w4a8(a.xq, a.scale, a.gsum, W.qw, W.scales, W.zeros)
    O.assert_fp_close(y16, ref, bound, 1e-5)


def test_w4a8_t16_entry_point_any_m(rng):
    """lbd_gemm_w4a8_t16 takes any M (matrix cores even at M = 1) and reports the path."""
    import ctypes as C
    W = _random_int4(rng, 40, 384, True)
    D = lb.to_device(W)
    qwt, st, zt = D.tiles()
    L = K.lib()
    for m in (1, 2):
        x = rng.standard_normal((m, 384)).astype(np.float32)
        dx = K.DeviceBuffer.from_array(x)
        dy = K.DeviceBuffer(m * 40 * 4)
        ws = K.DeviceBuffer(L.lbd_w4a8_workspace_bytes(m, 384))
        prm = K._Params(-1, 0, 0, 0, 0, 0, 0)
        rc = L.lbd_gemm_w4a8_t16(dx.ptr, m, 384, qwt.ptr, st.ptr, zt.ptr, 40, dy.ptr, C.byref(prm),
                                 ws.ptr, ws.nbytes, None)
        assert rc == K.ISA_GFX950_MFMA
        K.lib().lb_dev_synchronize()
        y = dy.to_array((m, 40), np.float32)
        a = lb.quantize_act_int8(x)
        ref, bound = cref.c_gemm_w4a8(a.xq, a.scale, a.gsum, W.qw, W.scales, W.zeros)
        O.assert_fp_close(y, ref, bound, 1e-5)
