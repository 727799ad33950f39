"""Known-answer tests of the packed formats and host quantizers (CPU).

Mirrors the reference's format tests (tests/test_formats.py) against lowbit_amd,
plus cross-checks of the product's packers against the oracle's independent
unpacker.
"""
import numpy as np
import pytest

from lowbit_amd import formats as F
from oracle import reference as O


@pytest.mark.parametrize("block", [32, 128])
def test_nibble_pack_roundtrip(rng, block):
    codes = rng.integers(0, 16, size=(5, 3 * block), dtype=np.uint8)
    packed = F.pack_nibbles(codes, block)
    assert packed.shape == (5, 3 * block // 2)
    np.testing.assert_array_equal(F.unpack_nibbles(packed, block), codes)
    # documented layout: byte j = elem j (low) | elem j + block/2 (high)
    assert packed[0, 0] == codes[0, 0] | (codes[0, block // 2] << 4)
    # the oracle's unpacker (an explicit index map) agrees
    np.testing.assert_array_equal(O.unpack_codes(packed, block), codes)


def test_nibble_layout_byte_positions():
    # element 128g+j -> low nibble of byte 64g+j, element 128g+64+j -> high nibble
    codes = np.zeros((1, 256), np.uint8)
    codes[0, 128 + 5] = 3
    codes[0, 128 + 64 + 5] = 12
    packed = F.pack_nibbles(codes, 128)
    assert packed[0, 64 + 5] == (3 | (12 << 4))
    assert np.count_nonzero(packed) == 1


@pytest.mark.parametrize("asym", [False, True])
@pytest.mark.parametrize("k", [128, 300, 1, 257])
def test_int4_roundtrip_error_bound(rng, asym, k):
    w = rng.standard_normal((7, k)).astype(np.float32) * 3
    q = F.quantize_int4(w, asym=asym)
    assert q.kp % 128 == 0 and q.kp >= k
    wd = q.dequantize()
    assert wd.shape == w.shape
    s = np.repeat(q.scales, 128, axis=1)[:, :k]
    assert np.all(np.abs(wd - w) <= 0.5 * s * (1 + 1e-5) + 1e-7)
    codes = q.codes()
    assert codes.max() <= 15
    zeros = 8 if q.zeros is None else q.zeros[:, -1:]
    np.testing.assert_array_equal(codes[:, k:], np.broadcast_to(zeros, codes[:, k:].shape))


@pytest.mark.parametrize("k", [128, 300, 1])
def test_int4_signed_max_scale(rng, k):
    w = rng.standard_normal((9, k)).astype(np.float32) * 3
    q = F.quantize_int4(w, scale="signed-max")
    wd = q.dequantize()
    s = np.abs(np.repeat(q.scales, 128, axis=1)[:, :k])
    err = np.abs(wd - w)
    g = w[:, :128] if k >= 128 else w
    i = np.abs(g).argmax(axis=1)
    np.testing.assert_allclose(wd[np.arange(9), i], g[np.arange(9), i], rtol=1e-6)
    assert np.all(q.codes()[np.arange(9), i] == 0)
    assert np.all(err <= s * (1 + 1e-5) + 1e-7)
    assert np.mean(err <= 0.5 * s * (1 + 1e-5) + 1e-7) > 0.95
    e0 = np.abs(F.quantize_int4(w).dequantize() - w)
    assert np.mean(err ** 2) <= np.mean(e0 ** 2)
    with pytest.raises(ValueError):
        F.quantize_int4(w, asym=True, scale="signed-max")
    with pytest.raises(ValueError):
        F.quantize_int4(w, scale="bogus")


def test_int4_exact_on_grid(rng):
    s = np.float32(0.25)
    codes = rng.integers(-7, 8, size=(4, 256))
    codes[:, 0] = 7
    codes[:, 128] = -7
    w = (codes * s).astype(np.float32)
    q = F.quantize_int4(w)
    np.testing.assert_array_equal(q.dequantize(), w)
    np.testing.assert_array_equal(q.scales, s)


def test_int4_constant_and_zero_groups():
    w = np.zeros((2, 128), np.float32)
    w[1] = 5.0
    for asym in (False, True):
        q = F.quantize_int4(w, asym=asym)
        np.testing.assert_allclose(q.dequantize(), w, rtol=0, atol=1e-6)
    # the documented special cases: zero rows get s = 1 and code z
    q = F.quantize_int4(w)
    assert q.scales[0, 0] == 1.0 and np.all(q.codes()[0] == 8)
    qa = F.quantize_int4(w, asym=True)
    assert qa.scales[0, 0] == 1.0 and qa.zeros[0, 0] == 0 and np.all(qa.codes()[0] == 0)


def test_int4_asym_closed_form():
    # one group with min -1.5 and max 3: s = 4.5/15 = 0.3, z = rint(1.5/0.3) = 5
    w = np.linspace(-1.5, 3.0, 128, dtype=np.float32)[None]
    q = F.quantize_int4(w, asym=True)
    assert q.scales[0, 0] == np.float32(np.float32(4.5) / np.float32(15))
    assert q.zeros[0, 0] == 5
    c = q.codes()[0]
    assert c[0] == 0 and c[-1] == 15


def test_e2m1_table_and_rounding():
    vals = F.E2M1_VALUES
    c = F.fp32_to_e2m1(vals)
    np.testing.assert_array_equal(vals[c], vals)
    ties = np.array([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0], np.float32)
    expect = np.array([0.0, 1.0, 1.0, 2.0, 2.0, 4.0, 4.0], np.float32)
    np.testing.assert_array_equal(vals[F.fp32_to_e2m1(ties)], expect)
    np.testing.assert_array_equal(vals[F.fp32_to_e2m1(-ties)], -expect)
    np.testing.assert_array_equal(vals[F.fp32_to_e2m1(np.array([7.9, -100.0], np.float32))], [6.0, -6.0])
    # canonical +0: tiny negatives round to code 0, never 8
    assert F.fp32_to_e2m1(np.array([-0.1, -0.0], np.float32)).tolist() == [0, 0]


def test_e8m0_decode():
    e = np.array([0, 1, 126, 127, 128, 254, 255], np.uint8)
    f = F.e8m0_to_float(e)
    np.testing.assert_array_equal(f[:6], np.array([2.0**-127, 2.0**-126, 0.5, 1.0, 2.0, 2.0**127], np.float32))
    assert np.isnan(f[6])
    assert f[0].view(np.uint32) == 0x00400000  # the float32 subnormal 2^-127


@pytest.mark.parametrize("k", [32, 100, 4096])
def test_mxfp4_roundtrip(rng, k):
    w = rng.standard_normal((6, k)).astype(np.float32)
    q = F.quantize_mxfp4(w)
    assert q.kp % 32 == 0
    wd = q.dequantize()
    scale = np.repeat(F.e8m0_to_float(q.e8m0), 32, axis=1)[:, :k]
    assert np.all(np.abs(wd - w) <= 2.0 * scale)
    blk = np.pad(w, ((0, 0), (0, q.kp - k))).reshape(6, -1, 32)
    amax = np.abs(blk).max(axis=2)
    np.testing.assert_array_equal(q.e8m0.astype(int) - 127, np.floor(np.log2(amax)) - 2)


def test_mxfp4_exact_on_grid(rng):
    codes = rng.integers(0, 16, size=(3, 64)).astype(np.uint8)
    codes[:, 0] = 7
    codes[:, 32] = 7
    w = F.E2M1_VALUES[codes] * np.float32(4.0)
    q = F.quantize_mxfp4(w)
    np.testing.assert_array_equal(q.dequantize(), w)
    np.testing.assert_array_equal(q.e8m0, 129)


def test_act_quant(rng):
    x = rng.standard_normal((4, 200)).astype(np.float32)
    a = F.quantize_act_int8(x)
    assert a.xq.shape == (4, 256) and a.gsum.shape == (4, 2)
    assert np.all(np.abs(a.xq) <= 127)
    np.testing.assert_array_equal(a.xq[:, 200:], 0)
    np.testing.assert_array_equal(a.gsum, a.xq.astype(np.int32).reshape(4, 2, 128).sum(-1))
    assert np.all(np.abs(a.dequantize()[:, :200] - x) <= 0.5 * a.scale[:, None] * (1 + 1e-6))


def test_act_quant_matches_oracle(rng):
    x = rng.standard_normal((5, 1000)).astype(np.float32) * 3
    x[2] = 0
    a = F.quantize_act_int8(x)
    xq, xs, asum = O.quant_act_int8(x)
    np.testing.assert_array_equal(a.xq, xq)
    np.testing.assert_array_equal(a.scale, xs)
    np.testing.assert_array_equal(a.gsum, asum)


def test_containers_nbytes():
    w = np.ones((8, 4096), np.float32)
    assert F.quantize_int4(w, asym=True).nbytes == 8 * (2048 + 32 * 4 + 32)
    # the metric's effective weight bytes at the BASELINE shape
    n, k = 11008, 4096
    assert n * k // 2 + n * (k // 128) * 4 + n * (k // 128) == 24_305_664
    assert n * k // 2 + n * (k // 32) == 23_953_408
