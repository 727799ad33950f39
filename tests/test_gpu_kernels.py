"""GPU parity: the gfx950 kernels, through the C ABI, against the CPU oracle.

Bar (from the reference's tests): bit-exact for the int8 quantizer and the W4A8
int32 group accumulators; |y - ref| <= 1e-5 * (|X| @ |W|^T) against float64 for
W4A16 / MXFP4, and 1e-5 times the lane magnitudes sum_k q|a| + z|sum a| (times
|s| and xs) for W4A8 (tests/conftest.py:22-27, tests/test_kernels.py:100-146).
Both device regimes are exercised: "gfx950" (VALU decode kernels, M <= 4) and
"gfx950-mfma" (matrix cores). Host containers go through the host-pointer ABI
(lb_gemm_*, weights uploaded per call) here; implicit residency has its own tests
(tests/test_gpu_resident.py).
"""
import numpy as np
import pytest

import lowbit_amd as lb
from lowbit_amd import kernels as K
from oracle import cref
from oracle import reference as O
from problems import outlier_int4_problem

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def _pointer_abi():
    with K.implicit_residency(False):
        yield

# (M, N, K): the reference's odd shapes (tests/test_kernels.py:39-40) plus M tails
# for the 16-row MFMA tiles.
SHAPES = [(1, 1, 1), (1, 64, 128), (3, 5, 127), (7, 33, 129), (5, 37, 300),
          (17, 70, 1000), (2, 16, 4096 + 32), (33, 20, 256), (64, 40, 384), (4, 300, 2048)]
PATHS = ["gfx950", "gfx950-mfma"]
RTOL = 1e-5


def _problem(rng, m, n, k):
    return (rng.standard_normal((m, k)).astype(np.float32),
            rng.standard_normal((n, k)).astype(np.float32))


def _int4_bound(xp, W):
    return cref.c_gemm_w4a16(xp, W.qw, W.scales, W.zeros, absval=True)


def _expected_path(isa, m, kp, fmt_bytes_per_x):
    valu_ok = m <= 4 and m * kp * fmt_bytes_per_x <= 60 * 1024
    return "gfx950" if (isa == "gfx950" and valu_ok) else "gfx950-mfma"


# ------------------------------------------------------------------ quantizer

@pytest.mark.parametrize("shape", [(1, 1), (3, 127), (4, 1000), (2, 4096), (64, 4096), (1, 11008), (7, 4224)])
def test_quantizer_bit_exact(rng, shape):
    x = rng.standard_normal(shape).astype(np.float32) * 3
    x[0, 0] = 0.5 * np.abs(x).max() / 127 * 3  # near an exact .5 tie
    if shape[0] > 2:
        x[1] = 0.0  # zero row: scale 1, codes 0
    kp = lb.formats.pad_to(shape[1], 128)
    a = K.quant_act_int8(x, kp)
    xq, xs, asum = O.quant_act_int8(x, kp)
    np.testing.assert_array_equal(a.xq, xq)
    np.testing.assert_array_equal(a.scale, xs)
    np.testing.assert_array_equal(a.gsum, asum)


def test_quantizer_exact_ties():
    x = np.zeros((2, 256), np.float32)
    x[0, :6] = [0.5, 1.5, 2.5, -2.5, -0.5, 127.0]  # amax 127 -> sc = 1: exact .5 ties
    x[1, :3] = [1e-38, -5e-39, 1e-40]  # sc = 1e-38/127 is a float32 subnormal: must not flush
    a = K.quant_act_int8(x, 256)
    xq, xs, asum = O.quant_act_int8(x)
    assert a.xq[0, :6].tolist() == [0, 2, 2, -2, 0, 127]
    np.testing.assert_array_equal(a.xq, xq)
    np.testing.assert_array_equal(a.scale, xs)
    np.testing.assert_array_equal(a.gsum, asum)


def test_quantizer_golden_vectors():
    g = np.load(__file__.rsplit("/", 1)[0] + "/golden/ref_vectors.npz")
    a = K.quant_act_int8(g["q_x"], g["q_xq"].shape[1])
    np.testing.assert_array_equal(a.xq, g["q_xq"])
    np.testing.assert_array_equal(a.scale, g["q_xs"])
    np.testing.assert_array_equal(a.gsum, g["q_asum"])


# ------------------------------------------------------------------ exact group accumulators

@pytest.mark.parametrize("isa", PATHS)
@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("asym", [False, True])
def test_group_acc_bit_exact(rng, isa, shape, asym):
    x, w = _problem(rng, *shape)
    W = lb.quantize_int4(w, asym=asym)
    a = lb.quantize_act_int8(x)
    got = K.w4a8_group_acc(a, W, isa=isa)
    assert K.last_path() == isa
    np.testing.assert_array_equal(got, O.w4a8_group_acc_ref(a.xq, W.qw, W.zeros))


@pytest.mark.parametrize("isa", PATHS)
def test_group_acc_worst_case_operands(isa):
    # codes 15 / 0 / all, zero-points 0, 15, 7, 8, activations 127 and -128
    g = np.load(__file__.rsplit("/", 1)[0] + "/golden/ref_vectors.npz")
    m, kp = g["wc_xq"].shape
    W = lb.Int4Weights(g["wc_qw"], np.ones(g["wc_zeros"].shape, np.float32), g["wc_zeros"], kp)
    a = lb.Int8Acts(g["wc_xq"], np.ones(m, np.float32), g["wc_asum"])
    np.testing.assert_array_equal(K.w4a8_group_acc(a, W, isa=isa), g["wc_out"])


@pytest.mark.parametrize("isa", PATHS)
def test_group_acc_extreme_tiles(rng, isa):
    # a full 64 x 64 tile of worst-case operands through the MFMA tile shape
    m, n, k = 64, 64, 512
    codes = rng.choice(np.array([0, 15], np.uint8), size=(n, k))
    W = lb.Int4Weights(lb.formats.pack_nibbles(codes, 128), np.ones((n, k // 128), np.float32),
                       rng.choice(np.array([0, 7, 8, 15], np.uint8), size=(n, k // 128)), k)
    xq = rng.choice(np.array([127, -128, -127], np.int8), size=(m, k))
    a = lb.Int8Acts(xq, np.ones(m, np.float32), xq.astype(np.int32).reshape(m, -1, 128).sum(-1).astype(np.int32))
    np.testing.assert_array_equal(K.w4a8_group_acc(a, W, isa=isa), O.w4a8_group_acc_ref(xq, W.qw, W.zeros))


# ------------------------------------------------------------------ fp32 GEMMs

@pytest.mark.parametrize("isa", PATHS)
@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("asym", [False, True])
def test_w4a16(rng, isa, shape, asym):
    x, w = _problem(rng, *shape)
    W = lb.quantize_int4(w, asym=asym)
    y = K.gemm_w4a16(x, W, isa=isa)
    assert y.shape == (shape[0], shape[1])
    assert K.last_path() == _expected_path(isa, shape[0], W.kp, 4)
    xp = lb.formats.pad_acts(x, W.kp)
    O.assert_fp_close(y, O.gemm_w4a16_ref(xp, W.qw, W.scales, W.zeros), _int4_bound(xp, W), RTOL)


@pytest.mark.parametrize("isa", PATHS)
@pytest.mark.parametrize("shape", SHAPES)
def test_mxfp4(rng, isa, shape):
    x, w = _problem(rng, *shape)
    W = lb.quantize_mxfp4(w)
    y = K.gemm_mxfp4(x, W, isa=isa)
    assert K.last_path() == _expected_path(isa, shape[0], W.kp, 4)
    xp = lb.formats.pad_acts(x, W.kp)
    O.assert_fp_close(y, O.gemm_mxfp4_ref(xp, W.qw, W.e8m0),
                      cref.c_gemm_mxfp4(xp, W.qw, W.e8m0, absval=True), RTOL)


@pytest.mark.parametrize("isa", PATHS)
@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("asym", [False, True])
def test_w4a8(rng, isa, shape, asym):
    x, w = _problem(rng, *shape)
    W = lb.quantize_int4(w, asym=asym)
    a = lb.quantize_act_int8(x)
    ref, bound = cref.c_gemm_w4a8(a.xq, a.scale, a.gsum, W.qw, W.scales, W.zeros)
    y = K.gemm_w4a8(x, W, isa=isa)
    assert K.last_path() == _expected_path(isa, shape[0], W.kp, 1)
    O.assert_fp_close(y, ref, bound, RTOL)
    O.assert_fp_close(K.gemm_w4a8_q(a, W, isa=isa), ref, bound, RTOL)


def _random_int4(rng, n, kp, asym):
    """Random packed int4 weights (any code, any zero-point), without quantizing a matrix."""
    g = kp // 128
    return lb.formats.Int4Weights(
        rng.integers(0, 256, (n, kp // 2), dtype=np.uint8),
        (rng.standard_normal((n, g)) * 0.05).astype(np.float32),
        rng.integers(0, 16, (n, g), dtype=np.uint8) if asym else None, kp)


# Shapes that give the persistent MFMA kernel several 16-row weight subtiles per
# workgroup (N = 11008), more than one pass of subtiles and more than one phase of
# 32 groups (N = 33000, K = 4352: G = 34, not a multiple of 4), and M tails. The
# row-block height follows the shape: 16 rows (M = 16, 17), 32 rows (M = 40, 64 at
# N = 11008) and 64 rows (M = 64 at N = 33000).
BIG = [(64, 11008, 4096, True), (40, 11008, 4096, False), (16, 11008, 4096, True),
       (17, 33000, 4352, True), (70, 4100, 4352, False), (64, 33000, 4352, True),
       (64, 33000, 4096, False)]


@pytest.mark.parametrize("m,n,kp,asym", BIG)
def test_w4a8_mfma_persistent_schedule(rng, m, n, kp, asym):
    W = _random_int4(rng, n, kp, asym)
    x = rng.standard_normal((m, kp)).astype(np.float32)
    a = lb.quantize_act_int8(x)
    ref, bound = cref.c_gemm_w4a8(a.xq, a.scale, a.gsum, W.qw, W.scales, W.zeros)
    O.assert_fp_close(K.gemm_w4a8(x, W, isa="gfx950-mfma"), ref, bound, RTOL)
    O.assert_fp_close(K.gemm_w4a8_q(a, W, isa="gfx950-mfma"), ref, bound, RTOL)


@pytest.mark.parametrize("m,n,kp", [(17, 33000, 4352), (64, 5000, 4096)])
def test_group_acc_mfma_persistent_schedule(rng, m, n, kp):
    W = _random_int4(rng, n, kp, True)
    xq = rng.integers(-128, 128, (m, kp), dtype=np.int8)
    xq[0, :128] = -128
    a = lb.formats.Int8Acts(xq, np.ones(m, np.float32),
                            xq.reshape(m, -1, 128).sum(axis=2, dtype=np.int32))
    np.testing.assert_array_equal(K.w4a8_group_acc(a, W, isa="gfx950-mfma"),
                                  cref.c_group_acc(xq, W.qw, W.zeros))


@pytest.mark.parametrize("isa", PATHS)
def test_int4_negative_scales(rng, isa):
    x, w = _problem(rng, 5, 37, 300)
    W = lb.quantize_int4(w, scale="signed-max")
    assert (W.scales < 0).any()
    xp = lb.formats.pad_acts(x, W.kp)
    O.assert_fp_close(K.gemm_w4a16(x, W, isa=isa), O.gemm_w4a16_ref(xp, W.qw, W.scales, W.zeros),
                      _int4_bound(xp, W), RTOL)
    a = lb.quantize_act_int8(x)
    np.testing.assert_array_equal(K.w4a8_group_acc(a, W, isa=isa), O.w4a8_group_acc_ref(a.xq, W.qw, W.zeros))
    ref, bound = cref.c_gemm_w4a8(a.xq, a.scale, a.gsum, W.qw, W.scales, W.zeros)
    O.assert_fp_close(K.gemm_w4a8(x, W, isa=isa), ref, bound, RTOL)


@pytest.mark.parametrize("isa", PATHS)
def test_zero_activation_row(rng, isa):
    x = rng.standard_normal((3, 256)).astype(np.float32)
    x[1] = 0
    W = lb.quantize_int4(rng.standard_normal((8, 256)).astype(np.float32))
    for gemm in (K.gemm_w4a8, K.gemm_w4a16):
        y = gemm(x, W, isa=isa)
        assert np.all(y[1] == 0) and np.all(np.isfinite(y))


@pytest.mark.parametrize("isa", PATHS)
@pytest.mark.parametrize("m,n,k", [(1, 40, 256), (3, 40, 256), (1, 300, 4096), (1, 200, 8320), (2, 64, 2048),
                                   (16, 70, 1024), (1, 24, 1152)])
def test_w4a16_outliers_at_zero_point_codes(isa, m, n, k):
    """Huge activations (1e6) where every weight code equals its zero-point: they add
    nothing to the reference's bound, and a kernel forming sum q x - z sum x misses it
    by a factor of tens to thousands (tests/test_w4a16_outliers.py). Every W4A16 path
    (the paced and split one-row GEMVs, the M = 2..4 GEMV, the matrix-core GEMM, host
    pointers and resident handles) must stay within it."""
    rng = np.random.default_rng(1000 + m * 7 + k)
    x, W = outlier_int4_problem(rng, m, n, k)
    xp = lb.formats.pad_acts(x, W.kp)
    ref, bound = O.gemm_w4a16_ref(xp, W.qw, W.scales, W.zeros), O.fp_bound(xp, W.dequantize())
    O.assert_fp_close(K.gemm_w4a16(x, W, isa=isa), ref, bound, RTOL)
    with K.implicit_residency(True):
        O.assert_fp_close(K.gemm_w4a16(x, lb.to_device(W), isa=isa), ref, bound, RTOL)


@pytest.mark.parametrize("isa", PATHS)
def test_zero_weight_rows_give_exact_zero(rng, isa):
    # symmetric zero rows quantize to q == z == 8: (q - z) * x must cancel exactly
    x = rng.standard_normal((2, 512)).astype(np.float32)
    w = rng.standard_normal((6, 512)).astype(np.float32)
    w[2] = 0
    W = lb.quantize_int4(w)
    for gemm in (K.gemm_w4a16, K.gemm_w4a8):
        assert np.all(gemm(x, W, isa=isa)[:, 2] == 0)
    Wm = lb.quantize_mxfp4(w)
    assert np.all(K.gemm_mxfp4(x, Wm, isa=isa)[:, 2] == 0)


def test_one_dimensional_x_and_params_auto(rng):
    x, w = _problem(rng, 1, 24, 200)
    W = lb.quantize_int4(w, asym=True)
    y1 = K.gemm_w4a16(x[0], W, params="auto", threads=3)
    y2 = K.gemm_w4a16(x, W, K.Params(mr=1, nr=4))
    assert y1.shape == (1, 24)
    np.testing.assert_array_equal(y1, y2)


# Rows of at most 1024 elements at one activation row take two weight rows per
# wave load (one per half-wave; the last slot of an odd share holds one). The
# same rows through the two-activation-row kernel, which loads one weight row per
# wave load, must give the same bits (both reduce each row over the same lanes in
# the same order), and both stay within the oracle's bound.
@pytest.mark.parametrize("fmt", ["w4a16", "w4a8", "mxfp4"])
@pytest.mark.parametrize("n,k", [(8191, 896), (12345, 1024), (151936, 128), (5000, 640), (9001, 256), (4097, 96)])
def test_two_rows_per_wave_load_match_one(rng, fmt, n, k):
    x = rng.standard_normal((1, k)).astype(np.float32)
    w = rng.standard_normal((n, k)).astype(np.float32)
    W = lb.quantize_mxfp4(w) if fmt == "mxfp4" else lb.quantize_int4(w, asym=(fmt == "w4a8"))
    D = lb.to_device(W)
    fn = {"w4a16": K.gemm_w4a16, "w4a8": K.gemm_w4a8, "mxfp4": K.gemm_mxfp4}[fmt]
    y1 = fn(x, D, isa="gfx950")
    y2 = fn(np.concatenate([x, x]), D, isa="gfx950")
    assert K.last_path() == "gfx950"
    np.testing.assert_array_equal(y1[0], y2[0])
    np.testing.assert_array_equal(y1[0], y2[1])
    xp = lb.formats.pad_acts(x, W.kp)
    if fmt == "w4a16":
        O.assert_fp_close(y1, O.gemm_w4a16_ref(xp, W.qw, W.scales, W.zeros), _int4_bound(xp, W), RTOL)
    elif fmt == "mxfp4":
        O.assert_fp_close(y1, O.gemm_mxfp4_ref(xp, W.qw, W.e8m0),
                          cref.c_gemm_mxfp4(xp, W.qw, W.e8m0, absval=True), RTOL)
    else:
        a = lb.quantize_act_int8(x)
        ref, bound = cref.c_gemm_w4a8(a.xq, a.scale, a.gsum, W.qw, W.scales, W.zeros)
        O.assert_fp_close(y1, ref, bound, RTOL)


def test_device_resident_weights_match_host_path(rng):
    x, w = _problem(rng, 3, 130, 700)
    for Wq in (lb.quantize_int4(w, asym=True), lb.quantize_int4(w)):
        D = lb.to_device(Wq)
        np.testing.assert_array_equal(K.gemm_w4a16(x, D), K.gemm_w4a16(x, Wq))
        np.testing.assert_array_equal(K.gemm_w4a8(x, D), K.gemm_w4a8(x, Wq))
    Wm = lb.quantize_mxfp4(w)
    np.testing.assert_array_equal(K.gemm_mxfp4(x, lb.to_device(Wm)), K.gemm_mxfp4(x, Wm))
    x64, w64 = _problem(rng, 40, 96, 512)
    W = lb.quantize_int4(w64, asym=True)
    np.testing.assert_array_equal(K.gemm_w4a8(x64, lb.to_device(W)), K.gemm_w4a8(x64, W))


def test_cpu_info_reports_device():
    info = K.cpu_info()
    assert info["cpu_isa"] == "gfx950-mfma"
    assert info["arch"].startswith("gfx950") and info["compute_units"] > 0
    assert K.effective_isa("w4a16", "avx512") == "gfx950-mfma"
    assert K.effective_isa("w4a8", "gfx950") == "gfx950"
