"""int4 with groups of 32 on the CPU: the host packer and the oracle (CPU only).

Groups of 32 are this package's extension (the reference ships group 128 and names
groups of 32 as its quality lever, README.md:300-304). They are pinned to the
reference-pinned group-128 path by restriction: a 32-column slab quantized with
group 128 is one group whose zero padding changes neither its max, its min nor its
largest-magnitude element, so its scale, zero point and 32 codes are exactly those
of the same slab as a group of 32. The oracle's group-32 decode and integer sums
are pinned by brute force on tiny inputs and by the same restriction.
"""
import numpy as np
import pytest

from lowbit_amd import formats as F
from oracle import reference as O


def _slabs_match(W32, w, asym, scale):
    n, k = w.shape
    codes32 = W32.codes()
    for i in range(W32.kp // 32):
        slab = w[:, 32 * i:min(k, 32 * i + 32)]
        W128 = F.quantize_int4(slab, asym=asym, scale=scale)  # one group of 128, zero padded
        np.testing.assert_array_equal(W32.scales[:, i], W128.scales[:, 0])
        if asym:
            np.testing.assert_array_equal(W32.zeros[:, i], W128.zeros[:, 0])
        np.testing.assert_array_equal(codes32[:, 32 * i:32 * i + 32], W128.codes()[:, :32])


@pytest.mark.parametrize("asym,scale", [(False, "absmax"), (False, "signed-max"), (True, "absmax")])
@pytest.mark.parametrize("k", [32, 96, 100, 4096 + 17])
def test_group32_is_group128_on_each_slab(rng, asym, scale, k):
    w = (rng.standard_normal((6, k)) * rng.lognormal(0, 1, (6, 1))).astype(np.float32)
    w[0, :40] = 0.0          # zero groups: scale 1
    w[1, 3:9] = 0.75         # repeated maxima
    w[2, 10], w[2, 11] = 5.0, -5.0  # largest magnitude at both signs: signed-max takes the first
    W32 = F.quantize_int4(w, asym=asym, scale=scale, group=32)
    assert W32.group == 32 and W32.kp == F.pad_to(k, 32)
    assert W32.scales.shape == (6, W32.kp // 32) and W32.qw.shape == (6, W32.kp // 2)
    _slabs_match(W32, w, asym, scale)


def test_group32_layout_is_j_and_j_plus_16():
    codes = (np.arange(64) % 16).astype(np.uint8)[None]
    packed = F.pack_nibbles(codes, 32)
    for j in range(32):
        g, b = divmod(j, 16)
        assert packed[0, j] == codes[0, 32 * g + b] | (codes[0, 32 * g + b + 16] << 4)
    np.testing.assert_array_equal(O.unpack_codes(packed, 32), codes)


def test_group32_dequantize_and_oracle_agree(rng):
    w = rng.standard_normal((5, 200)).astype(np.float32)
    for asym in (False, True):
        W = F.quantize_int4(w, asym=asym, group=32)
        d = O.dequant_int4(W.qw, W.scales, W.zeros, W.k, group=32)
        np.testing.assert_array_equal(d, W.dequantize().astype(np.float64))
        # each element within half a step of the weight
        s = np.repeat(W.scales, 32, axis=1)[:, :200]
        assert np.all(np.abs(d - w) <= 0.5 * np.abs(s) * (1 + 1e-6))


def _brute_acc32(xq, qw, zeros):
    n, kp = qw.shape[0], 2 * qw.shape[1]
    out = np.zeros((xq.shape[0], n, kp // 32), np.int64)
    for i in range(xq.shape[0]):
        for r in range(n):
            for b in range(kp // 2):
                g, j = divmod(b, 16)
                z = 8 if zeros is None else int(zeros[r, g])
                lo, hi = int(qw[r, b]) & 15, int(qw[r, b]) >> 4
                out[i, r, g] += (lo - z) * int(xq[i, 32 * g + j]) + (hi - z) * int(xq[i, 32 * g + 16 + j])
    return out


def test_group32_oracle_brute_force(rng):
    xq = rng.integers(-128, 128, size=(2, 96), dtype=np.int8)
    x = rng.standard_normal((2, 96)).astype(np.float32)
    for asym in (False, True):
        W = F.quantize_int4(rng.standard_normal((3, 96)).astype(np.float32), asym=asym, group=32)
        acc = O.w4a8_group_acc_ref(xq, W.qw, W.zeros, group=32)
        np.testing.assert_array_equal(acc, _brute_acc32(xq, W.qw, W.zeros))
        y = O.gemm_w4a8_ref(xq, np.array([0.5, 2.0], np.float32), W.qw, W.scales, W.zeros, group=32)
        want = (acc * W.scales[None].astype(np.float64)).sum(axis=2) * np.array([[0.5], [2.0]])
        np.testing.assert_allclose(y, want, rtol=1e-13)
        # W4A16: linear in x, group by group
        y16 = O.gemm_w4a16_ref(x, W.qw, W.scales, W.zeros, group=32)
        dense = W.dequantize().astype(np.float64)
        np.testing.assert_allclose(y16, x.astype(np.float64) @ dense.T, rtol=1e-12)


def test_group32_rejects_other_groups():
    with pytest.raises(ValueError):
        F.quantize_int4(np.zeros((2, 64), np.float32), group=64)


def test_group32_reference_only_entry_points_refuse():
    from lowbit_amd import kernels as K
    W = F.quantize_int4(np.zeros((2, 64), np.float32), group=32)
    a = F.quantize_act_int8(np.zeros((1, 64), np.float32), 128)
    with pytest.raises(ValueError):
        K.gemm_w4a8_q(a, W)
    with pytest.raises(ValueError):
        K.w4a8_group_acc(a, W)
