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


# ---------------------------------------------------------------- W4A16 / MXFP4, bf16x3 path

def mx_t16_expected(W):
    """The documented MXFP4 t16 order: qwt tiles of block 4g + q, et in lane order."""
    n, kp = W.n, W.kp
    g = -(-kp // 128)
    g4 = (g + 3) // 4 * 4
    s = (n + 15) // 16
    qw = np.zeros((s * 16, g4 * 64), np.uint8)
    qw[:n, :kp // 2] = W.qw
    qwt = qw.reshape(s, 16, g4, 4, 16).transpose(0, 2, 3, 1, 4).reshape(-1)
    e = np.zeros((s * 16, g4 * 4), np.uint8)
    e[:n, :kp // 32] = W.e8m0
    et = e.reshape(s, 16, g4, 4).transpose(0, 2, 3, 1).reshape(-1)  # [s][g][q][c]
    return qwt, et


def _random_mx(rng, n, kp, lo=118, hi=136):
    return lb.formats.MXFP4Weights(rng.integers(0, 256, (n, kp // 2), dtype=np.uint8),
                                   rng.integers(lo, hi, (n, kp // 32), dtype=np.uint8), kp)


@pytest.mark.parametrize("n,kp", [(16, 128), (33, 288), (70, 4128)])
def test_mxfp4_t16_repack_matches_documented_layout(rng, n, kp):
    W = _random_mx(rng, n, kp)
    qwt, et = lb.to_device(W).tiles()
    eq, ee = mx_t16_expected(W)
    np.testing.assert_array_equal(qwt.to_array(eq.shape, np.uint8), eq)
    np.testing.assert_array_equal(et.to_array(ee.shape, np.uint8), ee)


# (M, N, K): M tails and both row-block heights, N tails, the LLaMA up- and down-proj
# shapes (K = 11008: 86 groups, 11 per wave over 2 phases) and MXFP4 K not a multiple of 128.
BF3 = [(5, 33, 256), (16, 11008, 4096), (17, 70, 1152), (64, 11008, 4096), (64, 4096, 11008),
       (70, 300, 4352), (33, 20, 256), (1, 64, 128), (4, 100, 1024)]


def _lognormal_rows(rng, n, k):
    # config 4: W ~ N(0,1) scaled per row by LogNormal(0, 0.5) to spread the block exponents
    return (rng.standard_normal((n, k)) * rng.lognormal(0, 0.5, (n, 1))).astype(np.float32)


@pytest.mark.parametrize("m,n,k", BF3)
@pytest.mark.parametrize("asym", [False, True])
def test_w4a16_bf16x3_within_bound(rng, m, n, k, asym):
    x = rng.standard_normal((m, k)).astype(np.float32)
    W = lb.quantize_int4(_lognormal_rows(rng, n, k), asym=asym)
    D = lb.to_device(W)
    y = K.gemm_w4a16(x, D, isa="gfx950-mfma")
    f8 = K.w4a16_uses_t16f8(D, m)
    assert K.last_path() == "gfx950-mfma" and (D.t16f8 if f8 else D.t16) is not None
    assert (D.t16 if f8 else D.t16f8) is None
    xp = lb.formats.pad_acts(x, W.kp)
    ref = cref.c_gemm_w4a16(xp, W.qw, W.scales, W.zeros)
    bound = cref.c_gemm_w4a16(xp, W.qw, W.scales, W.zeros, absval=True)
    O.assert_fp_close(y, ref, bound, 1e-5)


@pytest.mark.parametrize("m,n,k", BF3 + [(64, 40, 4096 + 32), (20, 17, 96)])
def test_mxfp4_bf16x3_within_bound(rng, m, n, k):
    x = rng.standard_normal((m, k)).astype(np.float32)
    W = lb.quantize_mxfp4(_lognormal_rows(rng, n, k))
    D = lb.to_device(W)
    y = K.gemm_mxfp4(x, D, isa="gfx950-mfma")
    assert K.last_path() == "gfx950-mfma" and D.t16 is not None
    xp = lb.formats.pad_acts(x, W.kp)
    ref = cref.c_gemm_mxfp4(xp, W.qw, W.e8m0)
    bound = cref.c_gemm_mxfp4(xp, W.qw, W.e8m0, absval=True)
    O.assert_fp_close(y, ref, bound, 1e-5)


def test_bf16x3_zero_rows_and_negative_scales_exact(rng):
    """Zero weight rows give exact zeros (q - z = 0 / E2M1 0 in every product) and
    signed-max (negative) scales stay within the bound."""
    x = rng.standard_normal((24, 512)).astype(np.float32)
    w = rng.standard_normal((40, 512)).astype(np.float32)
    w[3] = 0.0
    w[17] = 0.0
    for W in (lb.quantize_int4(w), lb.quantize_int4(w, asym=True), lb.quantize_int4(w, scale="signed-max")):
        y = K.gemm_w4a16(x, lb.to_device(W), isa="gfx950-mfma")
        assert np.all(y[:, 3] == 0) and np.all(y[:, 17] == 0)
        ref = cref.c_gemm_w4a16(x, W.qw, W.scales, W.zeros)
        bound = cref.c_gemm_w4a16(x, W.qw, W.scales, W.zeros, absval=True)
        O.assert_fp_close(y, ref, bound, 1e-5)
    Wm = lb.quantize_mxfp4(w)
    y = K.gemm_mxfp4(x, lb.to_device(Wm), isa="gfx950-mfma")
    assert np.all(y[:, 3] == 0) and np.all(y[:, 17] == 0)


def test_mxfp4_bf16x3_extreme_exponents(rng):
    """E8M0 0 (2^-127, a float32 subnormal scale), 1 and 2, 230 and 254 within the
    bound, blocks 2^126 apart in one group, and 255 (NaN) propagating to exactly the
    rows the float64 oracle makes NaN. (Sums stay below the float32 range, where
    the reference's fp32 kernels would overflow too.)"""
    m, n, kp = 20, 48, 512
    x = rng.standard_normal((m, kp)).astype(np.float32)
    W = _random_mx(rng, n, kp)
    e = W.e8m0
    e[0, :] = 0                          # whole row at 2^-127
    e[1, :] = rng.integers(0, 3, kp // 32)
    e[2, ::2] = 1                        # tiny and normal blocks in the same groups
    e[3, :] = 230
    e[4, 0] = 254                        # one huge block next to normal ones:
    W.qw[4, :16] = 0
    W.qw[4, 0] = 0x01                    # a single 0.5 there, 2^126 * x stays finite
    e[5, 7] = 255                        # NaN block
    y = K.gemm_mxfp4(x, lb.to_device(W), isa="gfx950-mfma")
    ref = cref.c_gemm_mxfp4(x, W.qw, W.e8m0)
    bound = cref.c_gemm_mxfp4(x, W.qw, W.e8m0, absval=True)
    nan = np.isnan(ref)
    np.testing.assert_array_equal(np.isnan(y), nan)
    assert nan[:, 5].all() and nan.sum() == m
    keep = ~nan
    assert np.all(np.abs(y[keep] - ref[keep]) <= 1e-5 * bound[keep])


# ---------------------------------------------------------------- prefill-sized M

@pytest.mark.parametrize("m,n,k", [(512, 300, 4096), (2048, 48, 1024), (1000, 70, 1152)])
def test_prefill_m_within_bound(rng, m, n, k):
    """Prompt-sized M (many 16-row blocks per column of workgroups) on all three
    matrix-core paths: W4A8 int8 MFMA, W4A16 / MXFP4 bf16x3 on t16 weights, and the
    fp32 MFMA kernel of the pointer ABI (row-major weights)."""
    x = rng.standard_normal((m, k)).astype(np.float32)
    w = _lognormal_rows(rng, n, k)
    W4 = lb.quantize_int4(w, asym=True)
    y8 = K.gemm_w4a8(x, lb.to_device(W4))
    assert K.last_path() == "gfx950-mfma"
    a = lb.quantize_act_int8(x, W4.kp)
    ref, bound = cref.c_gemm_w4a8(a.xq, a.scale, a.gsum, W4.qw, W4.scales, W4.zeros)
    O.assert_fp_close(y8, ref, bound, 1e-5)
    xp = lb.formats.pad_acts(x, W4.kp)
    ref = cref.c_gemm_w4a16(xp, W4.qw, W4.scales, W4.zeros)
    bound = cref.c_gemm_w4a16(xp, W4.qw, W4.scales, W4.zeros, absval=True)
    for y in (K.gemm_w4a16(x, lb.to_device(W4)), K.gemm_w4a16(x, W4)):
        assert K.last_path() == "gfx950-mfma"
        O.assert_fp_close(y, ref, bound, 1e-5)
    Wm = lb.quantize_mxfp4(w)
    xp = lb.formats.pad_acts(x, Wm.kp)
    ref = cref.c_gemm_mxfp4(xp, Wm.qw, Wm.e8m0)
    bound = cref.c_gemm_mxfp4(xp, Wm.qw, Wm.e8m0, absval=True)
    for y in (K.gemm_mxfp4(x, lb.to_device(Wm)), K.gemm_mxfp4(x, Wm)):
        O.assert_fp_close(y, ref, bound, 1e-5)


# ---------------------------------------------------------------- launch variants

# Subtiles (16 weight rows) per workgroup pick the compiled chunk length and the
# number of weight stages in flight (1, 2, 3, 4, 5, 6, 8, the largest, and more
# than one chunk per workgroup, whose last chunk is short). With 256 compute units
# a 16-row activation block spreads S = N / 16 subtiles over 256 workgroups, a
# 64-row block over 128 (32-row tiles) or 64 (16-row tiles).
SHARES = [1, 2, 3, 4, 5, 6, 8, 12, 14]


@pytest.mark.parametrize("share", SHARES)
@pytest.mark.parametrize("fmt", ["w4a8", "w4a16", "mxfp4"])
@pytest.mark.parametrize("m", [16, 64])
def test_batch_kernels_every_share_of_subtiles(rng, fmt, m, share):
    """Each compiled variant of the batch kernels (chunk length, stages in flight,
    multi-chunk workgroups) against the float64 oracle within the reference's
    bound (the counts assume 256 compute units; on another part the same shapes
    still check correctness)."""
    n = 16 * (256 if m == 16 else 128) * share  # M = 64: 2 row blocks x 128 workgroups
    kp = 1152 if share == 5 else 256  # one share with two K phases of the bf16x3 kernel
    x = rng.standard_normal((m, kp)).astype(np.float32)
    if fmt == "mxfp4":
        W = lb.quantize_mxfp4(_lognormal_rows(rng, n, kp))
        D = lb.to_device(W)
        y = K.gemm_mxfp4(x, D, isa="gfx950-mfma")
        ref = cref.c_gemm_mxfp4(x, W.qw, W.e8m0)
        bound = cref.c_gemm_mxfp4(x, W.qw, W.e8m0, absval=True)
    elif fmt == "w4a16":
        W = lb.quantize_int4(_lognormal_rows(rng, n, kp), asym=True)
        D = lb.to_device(W)
        y = K.gemm_w4a16(x, D, isa="gfx950-mfma")
        ref = cref.c_gemm_w4a16(x, W.qw, W.scales, W.zeros)
        bound = cref.c_gemm_w4a16(x, W.qw, W.scales, W.zeros, absval=True)
    else:
        W = _random_int4(rng, n, kp, True)
        D = lb.to_device(W)
        y = K.gemm_w4a8(x, D, isa="gfx950-mfma")
        a = lb.quantize_act_int8(x)
        ref, bound = cref.c_gemm_w4a8(a.xq, a.scale, a.gsum, W.qw, W.scales, W.zeros)
    f8 = fmt == "w4a16" and K.w4a16_uses_t16f8(D, m)
    assert K.last_path() == "gfx950-mfma" and (D.t16f8 if f8 else D.t16) is not None
    O.assert_fp_close(y, ref, bound, 1e-5)
