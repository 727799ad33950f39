"""The t16f8 layout of int4 weights (each code less its zero-point as one E4M3 byte)
and the W4A16 bf16x3 GEMM that reads it.

The layout is this library's own (include/lowbit_hip.h, lbd_repack_int4_t16f8), so
the repacked bytes are pinned against the documented order through the oracle's
unpacking of the codes (src/lowbit/formats.py:40-54 order, oracle.reference.
unpack_codes) and against the OCP E4M3 definition of a byte's value; the GEMM is
pinned bit for bit against the same GEMM on the t16 layout (the operands are the
same bf16 values, summed in the same order) and against the float64 oracle within
the reference's bound.
"""
import ctypes as C
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest

import lowbit_amd as lb
from lowbit_amd import kernels as K
from oracle import cref
from oracle import reference as O

pytestmark = pytest.mark.gpu


def e4m3_value(b: np.ndarray) -> np.ndarray:
    """OCP E4M3 (FN) byte -> float64: sign, 4 exponent bits (bias 7), 3 mantissa bits,
    subnormal at exponent 0, NaN at S.1111.111."""
    b = b.astype(np.int64)
    e, m = (b >> 3) & 15, b & 7
    v = np.where(e == 0, m * 2.0 ** -9, (8 + m) * 2.0 ** (e - 10))
    v = np.where((b & 0x7F) == 0x7F, np.nan, v)
    return np.where(b >> 7, -v, v)


def t16f8_diffs(W):
    """code - z of every qwt8 byte in the documented order [S][G4][2][64][16]:
    half h, lane 16q + c of tile (s, g), byte b is the code at k = 128g + 64h + 16q + b
    of row 16s + c (nibble h of byte 64g + 16q + b) less its group's zero-point.
    Returns (diffs, valid) with padding marked invalid."""
    n, kp = W.n, W.kp
    g = kp // 128
    g4 = (g + 3) // 4 * 4
    s = (n + 15) // 16
    codes = O.unpack_codes(W.qw, 128).astype(np.int64)  # [n, kp] in k order
    z = np.full((n, g), 8, np.int64) if W.zeros is None else W.zeros.astype(np.int64)
    d = np.zeros((s * 16, g4 * 128), np.int64)
    valid = np.zeros((s * 16, g4 * 128), bool)
    d[:n, :kp] = codes - np.repeat(z, 128, axis=1)
    valid[:n, :kp] = True
    # k = 128g + 64h + 16q + b: [s][c][g][h][q][b] -> [s][g][h][q][c][b]
    order = lambda a: a.reshape(s, 16, g4, 2, 4, 16).transpose(0, 2, 3, 4, 1, 5).reshape(-1)
    return order(d), order(valid)


def _random_int4(rng, n, kp, asym):
    g = kp // 128
    return lb.formats.Int4Weights(
        rng.integers(0, 256, (n, kp // 2), dtype=np.uint8),
        (rng.standard_normal((n, g)) * 0.05).astype(np.float32),
        rng.integers(0, 16, (n, g), dtype=np.uint8) if asym else None, kp)


@pytest.mark.parametrize("n,kp,asym", [(16, 512, True), (33, 256, False), (70, 1152, True), (300, 4352, True),
                                       (17, 128, False)])
def test_t16f8_repack_matches_documented_layout(rng, n, kp, asym):
    W = _random_int4(rng, n, kp, asym)
    if asym:
        W.zeros[0, :] = 0    # differences up to +15
        W.zeros[1, :] = 15   # and down to -15
    D = lb.to_device(W)
    qwt8, st = D.tiles_f8()
    want, valid = t16f8_diffs(W)
    got = qwt8.to_array(want.shape, np.uint8)
    val = e4m3_value(got) * 512.0
    np.testing.assert_array_equal(val[valid], want[valid].astype(np.float64))
    assert np.all(got[~valid] == 0)
    assert np.all(got[valid & (want == 0)] == 0)  # +0, as (float)code - z is
    # scales as in t16: [S][G4/4][16][4]
    g, s = kp // 128, (n + 15) // 16
    g4 = (g + 3) // 4 * 4
    full = np.zeros((s * 16, g4), np.float32)
    full[:n, :g] = W.scales
    es = full.reshape(s, 16, g4 // 4, 4).transpose(0, 2, 1, 3).reshape(-1)
    np.testing.assert_array_equal(st.to_array(es.shape, np.float32), es)


def _t16_both(D, x, m):
    """y of lbd_gemm_w4a16_t16 (t16 tiles) and of lbd_gemm_w4a16_t16f8 (t16f8 tiles)."""
    L = K.lib()
    qwt, st, zt = D.tiles()
    qwt8, st8 = D.tiles_f8()
    dx = K.DeviceBuffer.from_array(x)
    ws = K.DeviceBuffer(L.lbd_bf16x3_workspace_bytes(m, D.kp))
    prm = K._Params(-1, 0, 0, 0, 0, 0, 0)
    out = []
    for f8 in (False, True):
        dy = K.DeviceBuffer(m * D.n * 4)
        if f8:
            rc = L.lbd_gemm_w4a16_t16f8(dx.ptr, m, D.kp, qwt8.ptr, st8.ptr, D.n, dy.ptr, C.byref(prm), ws.ptr,
                                        ws.nbytes, None)
        else:
            rc = L.lbd_gemm_w4a16_t16(dx.ptr, m, D.kp, qwt.ptr, st.ptr, None if zt is None else zt.ptr, D.n,
                                      dy.ptr, C.byref(prm), ws.ptr, ws.nbytes, None)
        assert rc == K.ISA_GFX950_MFMA
        assert L.lb_dev_synchronize() == 0
        out.append(dy.to_array((m, D.n), np.float32))
    return out


# (M, N, K): 16- and 32-row blocks, M and N tails, groups padded to a multiple of 4,
# two K phases (K = 11008: 86 groups), M = 1, and the LLaMA up- and down-proj shapes.
F8 = [(5, 33, 256), (16, 11008, 4096), (17, 70, 1152), (64, 11008, 4096), (64, 4096, 11008),
      (70, 300, 4352), (1, 64, 128), (33, 20, 256), (100, 4100, 1024)]


@pytest.mark.parametrize("m,n,k", F8)
@pytest.mark.parametrize("asym", [False, True])
def test_w4a16_t16f8_equals_t16_and_oracle(rng, m, n, k, asym):
    x = rng.standard_normal((m, k)).astype(np.float32)
    w = (rng.standard_normal((n, k)) * rng.lognormal(0, 0.5, (n, 1))).astype(np.float32)
    W = lb.quantize_int4(w, asym=asym)
    D = lb.to_device(W)
    xp = lb.formats.pad_acts(x, W.kp)
    y16, y8 = _t16_both(D, xp, m)
    np.testing.assert_array_equal(y8, y16)
    ref = cref.c_gemm_w4a16(xp, W.qw, W.scales, W.zeros)
    bound = cref.c_gemm_w4a16(xp, W.qw, W.scales, W.zeros, absval=True)
    O.assert_fp_close(y8, ref, bound, 1e-5)


def test_zero_points_above_15_take_the_t16_layout(rng):
    """A zero-point above 15 (outside what the packers write, but accepted by the
    row-major kernels) is not exact in t16f8: handles route such matrices to the t16
    layout (exact, within the bound), and the t16f8 entry point itself gives NaN in
    the rows whose differences it cannot hold, never a wrong finite value."""
    m, n, kp = 24, 40, 512
    W = _random_int4(rng, n, kp, True)
    W.zeros[5, 1] = 20   # codes 0-4 of row 5, group 1 differ by more than 15
    W.zeros[9, 2] = 200
    x = rng.standard_normal((m, kp)).astype(np.float32)
    D = lb.to_device(W)
    assert D.zmax == 200 and not D.f8_exact()
    y = K.gemm_w4a16(x, D, isa="gfx950-mfma")
    assert K.last_path() == "gfx950-mfma" and D.t16 is not None and D.t16f8 is None
    ref = cref.c_gemm_w4a16(x, W.qw, W.scales, W.zeros)
    bound = cref.c_gemm_w4a16(x, W.qw, W.scales, W.zeros, absval=True)
    O.assert_fp_close(y, ref, bound, 1e-5)
    with pytest.raises(ValueError):
        D.tiles_f8()
    # the entry point on a repack of the same arrays
    L = K.lib()
    bq, bs = C.c_size_t(0), C.c_size_t(0)
    assert L.lbd_int4_t16f8_bytes(n, kp, C.byref(bq), C.byref(bs)) == 0
    qwt8, st = K.DeviceBuffer(bq.value), K.DeviceBuffer(bs.value)
    assert L.lbd_repack_int4_t16f8(D.qw.ptr, D.scales.ptr, D.zeros.ptr, n, kp, qwt8.ptr, st.ptr, None) == 0
    dx = K.DeviceBuffer.from_array(x)
    dy = K.DeviceBuffer(m * n * 4)
    ws = K.DeviceBuffer(L.lbd_bf16x3_workspace_bytes(m, kp))
    prm = K._Params(-1, 0, 0, 0, 0, 0, 0)
    rc = L.lbd_gemm_w4a16_t16f8(dx.ptr, m, kp, qwt8.ptr, st.ptr, n, dy.ptr, C.byref(prm), ws.ptr, ws.nbytes, None)
    assert rc == K.ISA_GFX950_MFMA and L.lb_dev_synchronize() == 0
    y8 = dy.to_array((m, n), np.float32)
    nan = np.zeros((m, n), bool)
    nan[:, [5, 9]] = True
    np.testing.assert_array_equal(np.isnan(y8), nan)
    np.testing.assert_array_equal(y8[~nan], y[~nan])


def test_device_quantizer_handles_take_t16f8(rng):
    """Handles from the device quantizer (zero-points clipped to 0-15) read t16f8, with
    the same results as uploaded host-packed weights (the same bytes)."""
    w = rng.standard_normal((8192, 640)).astype(np.float32)
    x = rng.standard_normal((64, 640)).astype(np.float32)
    for asym in (False, True):
        Dd = K.quantize_int4_device(w, asym=asym)
        assert Dd.f8_exact() and K.w4a16_uses_t16f8(Dd, 64)
        y = K.gemm_w4a16(x, Dd, isa="gfx950-mfma")
        assert Dd.t16f8 is not None and Dd.t16 is None
        Dh = lb.to_device(lb.quantize_int4(w, asym=asym))
        np.testing.assert_array_equal(y, K.gemm_w4a16(x, Dh, isa="gfx950-mfma"))
        assert Dh.t16f8 is not None


def test_threads_share_one_t16f8_repack(rng):
    """Threads that share a handle whose t16f8 tiles are not built yet: the repack runs
    once and every thread's result equals the serial one."""
    x = rng.standard_normal((64, 1024)).astype(np.float32)
    W = lb.quantize_int4(rng.standard_normal((8192, 1024)).astype(np.float32), asym=True)
    want = K.gemm_w4a16(x, lb.to_device(W), isa="gfx950-mfma")  # serial, on its own handle
    D = lb.to_device(W)
    assert D.t16f8 is None and K.w4a16_uses_t16f8(D, 64)
    with ThreadPoolExecutor(max_workers=6) as ex:
        outs = list(ex.map(lambda _: K.gemm_w4a16(x, D, isa="gfx950-mfma"), range(12)))
    assert D.t16f8 is not None and D.t16 is None
    for y in outs:
        np.testing.assert_array_equal(y, want)


@pytest.mark.parametrize("m,n,k,want", [(64, 11008, 4096, True), (128, 11008, 4096, True), (256, 4096, 4096, True),
                                        (512, 4096, 4096, True), (16, 11008, 4096, False),
                                        (32, 11008, 4096, False), (16, 4096, 11008, False),
                                        (32, 4096, 11008, False), (64, 4096, 11008, True),
                                        (128, 4096, 11008, True)])
def test_w4a16_layout_choice_at_measured_shapes(m, n, k, want):
    """The shapes whose timings set the rule (256 compute units): t16f8 where each
    workgroup of the launch as it runs (K split in two at K = 11008 up to 64 rows) has
    4 or more weight subtiles, t16 below."""
    if K.device_info()["compute_units"] != 256:
        pytest.skip("the measured rule is stated for 256 compute units")
    assert K.lib().lbd_w4a16_prefers_t16f8(m, n, k) == int(want)
