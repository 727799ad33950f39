"""Weight quantizers on the device (lbd_quantize_int4 / lbd_quantize_mxfp4) against the
host packers, byte for byte.

The host packers restate the reference's quantize_int4 / quantize_mxfp4
(src/lowbit/formats.py:90-142, 197-212) and are pinned by the known-answer and
property tests of tests/test_formats.py, so equality here carries that parity to
the device. Inputs
cover what changes a byte: ragged K (padding), all three int4 scale rules, exact
rounding ties, zero / subnormal / huge groups, repeated maxima of both signs
(signed-max takes the first), E2M1 decision points, and MXFP4 block maxima just
below powers of two, where float32 log2 rounds up to the next exponent.
"""
import numpy as np
import pytest

import lowbit_amd as lb
from lowbit_amd import kernels as K

pytestmark = pytest.mark.gpu


def dev_int4(D):
    g = D.kp // 128
    qw = D.qw.to_array((D.n, D.kp // 2), np.uint8)
    s = D.scales.to_array((D.n, g), np.float32)
    z = None if D.zeros is None else D.zeros.to_array((D.n, g), np.uint8)
    return qw, s, z


def check_int4(w, **kw):
    ref = lb.quantize_int4(w, **kw)
    D = lb.quantize_int4_device(w, **kw)
    assert (D.n, D.kp, D.k, D.nbytes) == (ref.n, ref.kp, ref.k, ref.nbytes)
    qw, s, z = dev_int4(D)
    np.testing.assert_array_equal(qw, ref.qw)
    np.testing.assert_array_equal(s.view(np.uint32), ref.scales.view(np.uint32))
    if ref.zeros is None:
        assert z is None
    else:
        np.testing.assert_array_equal(z, ref.zeros)


def check_mx(w):
    ref = lb.quantize_mxfp4(w)
    D = lb.quantize_mxfp4_device(w)
    assert (D.n, D.kp, D.k, D.nbytes) == (ref.n, ref.kp, ref.k, ref.nbytes)
    np.testing.assert_array_equal(D.qw.to_array(ref.qw.shape, np.uint8), ref.qw)
    np.testing.assert_array_equal(D.e8m0.to_array(ref.e8m0.shape, np.uint8), ref.e8m0)


MODES = [dict(), dict(asym=True), dict(scale="signed-max")]


def awkward(rng, n, k):
    """N(0,1) rows at spread magnitudes, plus rows of special groups."""
    w = (rng.standard_normal((n, k)) * np.exp(rng.normal(0, 2, (n, 1)))).astype(np.float32)
    if n >= 8:
        w[0] = 0.0                                  # all-zero row
        w[1] = -0.0
        w[2] = rng.standard_normal(k).astype(np.float32) * np.float32(1e-41)  # subnormal
        w[3] = rng.standard_normal(k).astype(np.float32) * np.float32(1e37)   # huge
        w[4, :] = 1.0
        w[4, ::3] = -1.0                            # equal magnitudes, both signs
        w[5] = np.round(rng.standard_normal(k) * 4) / 2  # halves: rounding ties
        w[5, :min(k, 128)][0] = 7.0                 # s = 1 exactly: w / s lands on .5
        w[6] = np.abs(w[6])                         # one-signed groups (asym)
        w[7] = -np.abs(w[7])
    return w


@pytest.mark.parametrize("kw", MODES)
@pytest.mark.parametrize("n,k", [(8, 128), (13, 200), (64, 896), (9, 4864), (33, 4097)])
def test_int4_matches_host_packer(rng, n, k, kw):
    check_int4(awkward(rng, n, k), **kw)


def test_int4_signed_max_first_of_equal_magnitudes():
    w = np.zeros((2, 128), np.float32)
    w[0, [5, 9]] = [-3.0, 3.0]   # the first (-3) sets the sign: s = -3 / -8 > 0
    w[1, [5, 9]] = [3.0, -3.0]   # s = 3 / -8 < 0
    check_int4(w, scale="signed-max")
    D = lb.quantize_int4_device(w, scale="signed-max")
    s = D.scales.to_array((2, 1), np.float32)
    assert s[0, 0] == np.float32(0.375) and s[1, 0] == np.float32(-0.375)


@pytest.mark.parametrize("n,k", [(8, 32), (7, 48), (16, 128), (64, 896), (5, 4864), (3, 4099)])
def test_mxfp4_matches_host_packer(rng, n, k):
    check_mx(awkward(rng, n, k))


def test_mxfp4_e2m1_decision_points():
    """Every E2M1 decision point (.25 .75 1.25 1.75 2.5 3.5 5) and its neighbours, both
    signs, at a block scale of 1 (amax 4 -> e = 127)."""
    pts = np.array([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0], np.float32)
    vals = np.concatenate([pts, np.nextafter(pts, np.float32(0)), np.nextafter(pts, np.float32(9)),
                           [0.0, 6.0, 5.9, 0.1]]).astype(np.float32)
    rows = []
    for sign in (1.0, -1.0):
        v = np.zeros(32 * 2, np.float32)
        v[:len(vals)] = sign * vals
        v[31] = v[63] = 4.0  # pins the block maximum
        rows.append(v)
    check_mx(np.stack(rows))


def test_mxfp4_maxima_just_below_powers_of_two():
    """Each block's maximum sits n ulps below 2^k (n = 0..399, every k from the
    subnormal range to 2^127): the shared exponent is floor(float32 log2(amax)),
    which rounds up to k for the closest of them."""
    vals = []
    for k in range(-149, 128):
        x = np.ldexp(np.float32(1), k).astype(np.float32)
        for _ in range(400):
            vals.append(x)
            x = np.nextafter(x, np.float32(0))
    vals = np.array(vals, np.float32)
    vals = vals[vals > 0]
    w = np.zeros((len(vals), 32), np.float32)
    w[:, 0] = vals
    w[:, 1] = -vals * np.float32(0.5)
    w[:, 2] = vals * np.float32(0.3)
    ref = lb.quantize_mxfp4(w)
    exact = np.floor(np.log2(vals.astype(np.float64))) - 2 + 127
    assert np.any(ref.e8m0[:, 0].astype(np.float64) > np.clip(exact, 0, 254))  # the round-up cases are in
    check_mx(w)


def test_device_buffer_input_and_errors(rng):
    w = rng.standard_normal((20, 256)).astype(np.float32)
    buf = K.DeviceBuffer.from_array(w)
    D = lb.quantize_int4_device(buf, shape=(20, 256))
    ref = lb.quantize_int4(w)
    np.testing.assert_array_equal(D.qw.to_array(ref.qw.shape, np.uint8), ref.qw)
    with pytest.raises(ValueError):
        lb.quantize_int4_device(buf)  # shape missing
    with pytest.raises(ValueError):
        lb.quantize_int4_device(buf, shape=(40, 256))  # larger than the buffer
    with pytest.raises(ValueError):
        lb.quantize_int4_device(w, asym=True, scale="signed-max")
    # and the handle drives the GEMM like an uploaded host packing
    x = rng.standard_normal((3, 256)).astype(np.float32)
    np.testing.assert_array_equal(lb.gemm_w4a8(x, D), lb.gemm_w4a8(x, lb.to_device(ref)))


def test_qwen_sized_matrices(rng):
    """The largest matrices of the BASELINE config-5 decoder: the 151936 x 896 tied
    embedding / LM head and the 9728 x 896 gate/up projection."""
    for n, k in ((151936, 896), (9728, 896)):
        w = (rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.05))
        check_int4(w)
        check_mx(w)
