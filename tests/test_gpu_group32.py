"""int4 with groups of 32 on the device (lbd_gemm_w4a16_g32, lbd_gemm_w4a8_g32,
lbd_quantize_int4_g32) against the oracle.

Bar: the device packer writes the host packer's bytes (the host packer is pinned to
the reference-pinned group-128 path in tests/test_group32.py); W4A16 within
1e-5 * (|X| @ |W|^T) of the float64 oracle, W4A8 within 1e-5 of the lane magnitudes
(sum_k q|a| + z|sum a| per group, times |s| and the token scale) of the int64
oracle on the same per-token int8 activations (the reference's bound,
tests/conftest.py:22-27 and tests/test_kernels.py:100-146 of the reference).
"""
import numpy as np
import pytest

import lowbit_amd as lb
from lowbit_amd import kernels as K
from oracle import reference as O

pytestmark = pytest.mark.gpu


def _quant(x, kp):
    """(xq [M, kp], xs) of the per-token quantizer; the oracle's group-128 sums need a
    row padded to 128, whose zero padding changes neither amax nor any code."""
    xq, xs, _ = O.quant_act_int8(x, lb.formats.pad_to(kp, 128))
    return xq[:, :kp], xs


def _w(rng, n, k):
    return (rng.standard_normal((n, k)) * rng.lognormal(0, 0.5, (n, 1))).astype(np.float32)


@pytest.mark.parametrize("asym,scale", [(False, "absmax"), (False, "signed-max"), (True, "absmax")])
@pytest.mark.parametrize("n,k", [(5, 32), (7, 100), (33, 4113), (64, 896)])
def test_device_packer_matches_host(rng, asym, scale, n, k):
    w = _w(rng, n, k)
    w[0, :33] = 0.0
    w[min(1, n - 1), 5:9] = 0.625
    ref = lb.quantize_int4(w, asym=asym, scale=scale, group=32)
    D = K.quantize_int4_device(w, asym=asym, scale=scale, group=32)
    assert D.group == 32 and (D.n, D.kp, D.k, D.nbytes) == (ref.n, ref.kp, ref.k, ref.nbytes)
    np.testing.assert_array_equal(D.qw.to_array(ref.qw.shape, np.uint8), ref.qw)
    np.testing.assert_array_equal(D.scales.to_array(ref.scales.shape, np.float32), ref.scales)
    if asym:
        np.testing.assert_array_equal(D.zeros.to_array(ref.zeros.shape, np.uint8), ref.zeros)


# M = 1 with rows past 1024 elements runs the paced kernels: (1, 45, 2080) holds its
# activations in registers with byte-wise zero-point loads (65 groups, not a multiple
# of four); (1, 33, 4160), (1, 50, 6000) and (1, 37, 11008) are W4A16's split variant
# (2-3 slices, partial last slice) and W4A8's longer-row instantiations
SHAPES = [(1, 64, 32), (1, 300, 896), (2, 33, 100), (3, 70, 4096), (4, 17, 4864), (5, 40, 1024),
          (9, 11, 320), (1, 11008, 4096), (64, 96, 4096), (1, 40, 14336), (2, 20, 11008),
          (1, 45, 2080), (1, 33, 4160), (1, 50, 6000), (1, 37, 11008)]


@pytest.mark.parametrize("m,n,k", SHAPES)
@pytest.mark.parametrize("asym", [False, True])
def test_w4a16_g32_within_bound(rng, m, n, k, asym):
    x = rng.standard_normal((m, k)).astype(np.float32)
    W = lb.quantize_int4(_w(rng, n, k), asym=asym, group=32)
    xp = lb.formats.pad_acts(x, W.kp)
    dense = O.dequant_int4(W.qw, W.scales, W.zeros, group=32)
    ref, bound = xp.astype(np.float64) @ dense.T, O.fp_bound(xp, dense)
    for w in (W, lb.to_device(W)):
        y = K.gemm_w4a16(x, w)
        assert K.last_path() == "gfx950"
        O.assert_fp_close(y, ref, bound, 1e-5)


@pytest.mark.parametrize("m,n,k", SHAPES)
@pytest.mark.parametrize("asym", [False, True])
def test_w4a8_g32_within_bound(rng, m, n, k, asym):
    x = rng.standard_normal((m, k)).astype(np.float32)
    x[0, :7] = 0.5 * np.abs(x).max() / 127 * np.arange(1, 8) * 2  # a few exact .5 ties
    W = lb.quantize_int4(_w(rng, n, k), asym=asym, group=32)
    xq, xs = _quant(x, W.kp)
    asum32 = xq.astype(np.int64).reshape(m, -1, 32).sum(axis=2)
    ref = O.gemm_w4a8_ref(xq, xs, W.qw, W.scales, W.zeros, group=32)
    bound = O.w4a8_lane_bound(xq, xs, asum32, W.qw, W.scales, W.zeros, group=32)
    for w in (W, lb.to_device(W)):
        y = K.gemm_w4a8(x, w)
        assert K.last_path() == "gfx950"
        O.assert_fp_close(y, ref, bound, 1e-5)


def test_g32_zero_rows_exact_and_limits(rng):
    x = rng.standard_normal((3, 256)).astype(np.float32)
    w = rng.standard_normal((10, 256)).astype(np.float32)
    w[4] = 0.0
    for asym in (False, True):
        W = lb.quantize_int4(w, asym=asym, group=32)
        for f in (K.gemm_w4a16, K.gemm_w4a8):
            assert np.all(f(x, W)[:, 4] == 0)
    # row limits: fp32 activations in LDS (W4A16) up to 14336, int8 (W4A8) up to 16384
    x1 = rng.standard_normal((1, 16384)).astype(np.float32)
    W = lb.quantize_int4(rng.standard_normal((8, 16384)).astype(np.float32), group=32)
    xq, xs = _quant(x1, W.kp)
    ref = O.gemm_w4a8_ref(xq, xs, W.qw, W.scales, W.zeros, group=32)
    bound = O.w4a8_lane_bound(xq, xs, xq.astype(np.int64).reshape(1, -1, 32).sum(axis=2), W.qw, W.scales, W.zeros,
                              group=32)
    O.assert_fp_close(K.gemm_w4a8(x1, W), ref, bound, 1e-5)
    with pytest.raises(ValueError):
        K.gemm_w4a16(x1, W)
    big = lb.quantize_int4(np.zeros((2, 16384 + 32), np.float32), group=32)
    with pytest.raises(ValueError):
        K.gemm_w4a8(np.zeros((1, 16384 + 32), np.float32), big)
