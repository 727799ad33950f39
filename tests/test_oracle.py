"""Pins of the CPU oracle (CPU only).

Every oracle function is checked against something that does not share its
code: the reference's own C library (oracle/_ref, when built), golden vectors
that library wrote (tests/golden/ref_vectors.npz), the reference's known-answer
tests, brute force on tiny inputs and closed forms. The last section plants
plausible mistakes in copies of the oracle and shows that the pins catch them.
"""
import ctypes as C
from pathlib import Path

import numpy as np
import pytest

from lowbit_amd import formats as F
from oracle import cref
from oracle import reference as O

class _Gold:
    """The golden vectors, opened on first use (collection alone loads nothing)."""
    _npz = None

    def _open(self):
        if _Gold._npz is None:
            _Gold._npz = np.load(Path(__file__).resolve().parent / "golden" / "ref_vectors.npz")
        return _Gold._npz

    def __getitem__(self, key):
        return self._open()[key]

    @property
    def files(self):
        return self._open().files


GOLD = _Gold()
# The reference's C library is mapped only inside the tests that call it.
needs_ref = pytest.mark.skipif(not cref.ref_path().exists(), reason="oracle/_ref (reference C library) not built")


# ------------------------------------------------------------------ brute force helpers

def brute_codes(qw, block):
    n, nb = qw.shape
    out = np.zeros((n, 2 * nb), np.int64)
    half = block // 2
    for r in range(n):
        for byte in range(nb):
            blk, j = divmod(byte, half)
            out[r, blk * block + j] = int(qw[r, byte]) & 15
            out[r, blk * block + half + j] = int(qw[r, byte]) >> 4
    return out


def brute_w4a16(x, qw, scales, zeros):
    c = brute_codes(qw, 128)
    m, n = x.shape[0], qw.shape[0]
    y = np.zeros((m, n))
    for i in range(m):
        for r in range(n):
            t = 0.0
            for k in range(c.shape[1]):
                g = k // 128
                z = 8 if zeros is None else int(zeros[r, g])
                t += float(x[i, k]) * float(np.float32(np.float32(c[r, k] - z) * scales[r, g]))
            y[i, r] = t
    return y


def brute_groupacc(xq, qw, zeros):
    c = brute_codes(qw, 128)
    m, n, g = xq.shape[0], qw.shape[0], c.shape[1] // 128
    out = np.zeros((m, n, g), np.int64)
    for i in range(m):
        for r in range(n):
            for gi in range(g):
                z = 8 if zeros is None else int(zeros[r, gi])
                out[i, r, gi] = sum((int(c[r, k]) - z) * int(xq[i, k]) for k in range(128 * gi, 128 * gi + 128))
    return out


# ------------------------------------------------------------------ layout / decode pins

def test_unpack_matches_brute_force(rng):
    for block in (32, 128):
        qw = rng.integers(0, 256, size=(3, 2 * block), dtype=np.uint8)
        np.testing.assert_array_equal(O.unpack_codes(qw, block), brute_codes(qw, block))


def test_e8m0_and_e2m1_known_answers():
    # reference KATs: tests/test_formats.py:92-97 and formats.py:23-24
    e = O.e8m0_value(np.array([0, 1, 126, 127, 128, 254, 255]))
    np.testing.assert_array_equal(e[:6], [2.0**-127, 2.0**-126, 0.5, 1.0, 2.0, 2.0**127])
    assert np.isnan(e[6])
    np.testing.assert_array_equal(O.e2m1_value(np.arange(16)),
                                  [0, .5, 1, 1.5, 2, 3, 4, 6, -0.0, -.5, -1, -1.5, -2, -3, -4, -6])


def test_dequant_closed_forms():
    # a row of constant code q with zero-point z and scale s decodes to s*(q-z) everywhere
    qw = np.full((2, 64), 0xB3, np.uint8)  # low nibble 3, high nibble 11
    s = np.array([[0.5], [-2.0]], np.float32)
    z = np.array([[1], [11]], np.uint8)
    w = O.dequant_int4(qw, s, z)
    np.testing.assert_array_equal(w[0, :64], 0.5 * (3 - 1))
    np.testing.assert_array_equal(w[0, 64:], 0.5 * (11 - 1))
    np.testing.assert_array_equal(w[1, :64], -2.0 * (3 - 11))
    np.testing.assert_array_equal(w[1, 64:], 0.0)
    # MXFP4: code 0x7 (6.0) low, 0xA (-1.0) high, e = 128 (x2)
    wm = O.dequant_mxfp4(np.full((1, 16), 0xA7, np.uint8), np.array([[128]], np.uint8))
    np.testing.assert_array_equal(wm[0, :16], 12.0)
    np.testing.assert_array_equal(wm[0, 16:], -2.0)


# ------------------------------------------------------------------ quantizer pins

def test_quantizer_matches_golden_reference_vectors():
    x = GOLD["q_x"]
    xq, xs, asum = O.quant_act_int8(x)
    np.testing.assert_array_equal(xq, GOLD["q_xq"])
    np.testing.assert_array_equal(xs, GOLD["q_xs"])
    np.testing.assert_array_equal(asum, GOLD["q_asum"])
    cq, cs, ca = cref.c_quant_act_int8(F.pad_acts(x, xq.shape[1]))
    np.testing.assert_array_equal(cq, GOLD["q_xq"])
    np.testing.assert_array_equal(cs, GOLD["q_xs"])
    np.testing.assert_array_equal(ca, GOLD["q_asum"])


def test_quantizer_ties_round_to_even():
    # x / sc exactly on .5 steps: 0.5 -> 0, 1.5 -> 2, 2.5 -> 2, -2.5 -> -2; amax 127 gives sc = 1
    x = np.zeros((1, 128), np.float32)
    x[0, :5] = [0.5, 1.5, 2.5, -2.5, 127.0]
    xq, xs, _ = O.quant_act_int8(x)
    assert xs[0] == 1.0
    assert xq[0, :5].tolist() == [0, 2, 2, -2, 127]


@needs_ref
@pytest.mark.parametrize("shape", [(1, 1), (3, 127), (4, 1000), (2, 4096), (5, 11008)])
def test_quantizer_matches_reference_c(rng, shape):
    x = rng.standard_normal(shape).astype(np.float32) * 3
    x[0, 0] = 0.5 * np.abs(x).max() / 127 * 3
    kp = F.pad_to(shape[1], 128)
    xp = F.pad_acts(x, kp)
    m = shape[0]
    rq, rs, ra = np.empty((m, kp), np.int8), np.empty(m, np.float32), np.empty((m, kp // 128), np.int32)
    cref.ref_lib().lb_quant_act_int8(xp, m, kp, rq, rs, ra)
    for xq, xs, asum in (O.quant_act_int8(x), cref.c_quant_act_int8(xp)):
        np.testing.assert_array_equal(xq, rq)
        np.testing.assert_array_equal(xs, rs)
        np.testing.assert_array_equal(asum, ra)


# ------------------------------------------------------------------ integer accumulator pins

@pytest.mark.parametrize("tag", ["sym", "asym"])
def test_group_acc_matches_golden_reference_vectors(tag):
    zeros = GOLD[f"ga_{tag}_zeros"] if f"ga_{tag}_zeros" in GOLD.files else None
    got = O.w4a8_group_acc_ref(GOLD["q_xq"], GOLD[f"ga_{tag}_qw"], zeros)
    np.testing.assert_array_equal(got, GOLD[f"ga_{tag}_out"])
    np.testing.assert_array_equal(cref.c_group_acc(GOLD["q_xq"], GOLD[f"ga_{tag}_qw"], zeros), got)


def test_group_acc_worst_case_fixture():
    got = O.w4a8_group_acc_ref(GOLD["wc_xq"], GOLD["wc_qw"], GOLD["wc_zeros"])
    np.testing.assert_array_equal(got, GOLD["wc_out"])
    # closed form for row 0 (codes 15, z 0) against activations 127: 15 * 127 * 128
    assert got[0, 0, 0] == 15 * 127 * 128
    assert np.abs(got).max() < 2**31


def test_group_acc_brute_force(rng):
    xq = rng.integers(-128, 128, size=(2, 256), dtype=np.int8)
    W = F.quantize_int4(rng.standard_normal((3, 256)).astype(np.float32), asym=True)
    np.testing.assert_array_equal(O.w4a8_group_acc_ref(xq, W.qw, W.zeros), brute_groupacc(xq, W.qw, W.zeros))
    Ws = F.quantize_int4(rng.standard_normal((3, 256)).astype(np.float32))
    np.testing.assert_array_equal(O.w4a8_group_acc_ref(xq, Ws.qw, None), brute_groupacc(xq, Ws.qw, None))


@needs_ref
@pytest.mark.parametrize("asym", [False, True])
@pytest.mark.parametrize("shape", [(1, 1, 1), (3, 5, 127), (7, 33, 129), (17, 70, 1000), (2, 16, 4128)])
def test_group_acc_matches_reference_c(rng, shape, asym):
    m, n, k = shape
    x = rng.standard_normal((m, k)).astype(np.float32)
    W = F.quantize_int4(rng.standard_normal((n, k)).astype(np.float32), asym=asym)
    xq, xs, asum = O.quant_act_int8(x, W.kp)
    want = O.w4a8_group_acc_ref(xq, W.qw, W.zeros)
    for isa in (0, -1):  # reference scalar path and its best SIMD path
        out = np.empty((m, n, W.kp // 128), np.int32)
        assert cref.ref_lib().lb_w4a8_group_acc(xq, asum, m, W.kp, W.qw, cref.zp(W.zeros), n, out, isa) >= 0
        np.testing.assert_array_equal(out, want)
    np.testing.assert_array_equal(cref.c_group_acc(xq, W.qw, W.zeros), want)


# ------------------------------------------------------------------ float GEMM pins

def _bound_int4(x, W):
    return O.fp_bound(x, O.dequant_int4(W.qw, W.scales, W.zeros))


def test_w4a16_brute_force(rng):
    x = rng.standard_normal((2, 256)).astype(np.float32)
    W = F.quantize_int4(rng.standard_normal((3, 256)).astype(np.float32), asym=True)
    np.testing.assert_allclose(O.gemm_w4a16_ref(x, W.qw, W.scales, W.zeros),
                               brute_w4a16(x, W.qw, W.scales, W.zeros), rtol=1e-12, atol=1e-12)


def test_w4a16_closed_form(rng):
    # constant code q with zero-point z and scale s: y = s * (q - z) * sum(x)
    x = rng.standard_normal((3, 128)).astype(np.float32)
    qw = np.full((1, 64), 0x55, np.uint8)
    y = O.gemm_w4a16_ref(x, qw, np.array([[0.25]], np.float32), np.array([[2]], np.uint8))
    np.testing.assert_allclose(y[:, 0], 0.25 * 3 * x.astype(np.float64).sum(axis=1), rtol=1e-13)


@pytest.mark.parametrize("tag", ["sym", "asym"])
def test_gemms_match_golden_reference_vectors(tag):
    zeros = GOLD[f"ga_{tag}_zeros"] if f"ga_{tag}_zeros" in GOLD.files else None
    qw, s = GOLD[f"ga_{tag}_qw"], GOLD[f"ga_{tag}_scales"]
    x = F.pad_acts(GOLD["q_x"], qw.shape[1] * 2)
    ref = O.gemm_w4a16_ref(x, qw, s, zeros)
    O.assert_fp_close(GOLD[f"w4a16_{tag}_y"], ref, O.fp_bound(x, O.dequant_int4(qw, s, zeros)))
    y, bound = cref.c_gemm_w4a8(GOLD["q_xq"], GOLD["q_xs"], GOLD["q_asum"], qw, s, zeros)
    np.testing.assert_allclose(y, O.gemm_w4a8_ref(GOLD["q_xq"], GOLD["q_xs"], qw, s, zeros), rtol=1e-12,
                               atol=1e-12)
    O.assert_fp_close(GOLD[f"w4a8_{tag}_y"], y, bound)
    np.testing.assert_allclose(cref.c_gemm_w4a16(x, qw, s, zeros), ref, rtol=1e-12, atol=1e-12)


def test_mxfp4_matches_golden_reference_vectors():
    x, qw, e = GOLD["mx_x"], GOLD["mx_qw"], GOLD["mx_e8m0"]
    ref = O.gemm_mxfp4_ref(x, qw, e)
    O.assert_fp_close(GOLD["mx_y"], ref, O.fp_bound(x, O.dequant_mxfp4(qw, e)))
    np.testing.assert_allclose(cref.c_gemm_mxfp4(x, qw, e), ref, rtol=1e-12, atol=1e-12)


@needs_ref
@pytest.mark.parametrize("shape", [(1, 64, 128), (3, 5, 127), (5, 37, 300), (2, 16, 4128)])
def test_gemms_match_reference_c(rng, shape):
    m, n, k = shape
    x = rng.standard_normal((m, k)).astype(np.float32)
    w = rng.standard_normal((n, k)).astype(np.float32)
    p = cref.RefParams(-1, 0, 0, 0, 0, 0, 0)
    for asym in (False, True):
        W = F.quantize_int4(w, asym=asym)
        xp = F.pad_acts(x, W.kp)
        y = np.empty((m, n), np.float32)
        assert cref.ref_lib().lb_gemm_w4a16(xp, m, W.kp, W.qw, W.scales, cref.zp(W.zeros), n, y, C.byref(p)) >= 0
        O.assert_fp_close(y, O.gemm_w4a16_ref(xp, W.qw, W.scales, W.zeros), _bound_int4(xp, W))
        assert cref.ref_lib().lb_gemm_w4a8(xp, m, W.kp, W.qw, W.scales, cref.zp(W.zeros), n, y, C.byref(p)) >= 0
        xq, xs, asum = O.quant_act_int8(xp)
        _, bound = cref.c_gemm_w4a8(xq, xs, asum, W.qw, W.scales, W.zeros)
        O.assert_fp_close(y, O.gemm_w4a8_ref(xq, xs, W.qw, W.scales, W.zeros), bound)
    Wm = F.quantize_mxfp4(w)
    xp = F.pad_acts(x, Wm.kp)
    y = np.empty((m, n), np.float32)
    assert cref.ref_lib().lb_gemm_mxfp4(xp, m, Wm.kp, Wm.qw, Wm.e8m0, n, y, C.byref(p)) >= 0
    O.assert_fp_close(y, O.gemm_mxfp4_ref(xp, Wm.qw, Wm.e8m0), O.fp_bound(xp, O.dequant_mxfp4(Wm.qw, Wm.e8m0)))


# ------------------------------------------------------------------ W4A8 bound pins
#
# Every W4A8 GPU test is judged by the `bound` output of the C oracle's
# orc_gemm_w4a8. The reference defines that scale in tests/test_kernels.py:108-116:
# per group the lane magnitude sum_k q|a| + z|sum_k a|, weighted by the group scale
# and multiplied by the token scale. The oracle takes |s| and |xs|, so the bound is
# a magnitude for signed-max weights too (their scales are negative); for positive
# scales the two are the same number.

def _bound_operands(rng, m, n, k, asym, rule="absmax"):
    x = rng.standard_normal((m, k)).astype(np.float32)
    W = F.quantize_int4(rng.standard_normal((n, k)).astype(np.float32), asym=asym, scale=rule)
    xq, xs, asum = O.quant_act_int8(F.pad_acts(x, W.kp))
    return xq, xs, asum, W


@pytest.mark.parametrize("tag", ["sym", "asym"])
def test_w4a8_bound_matches_numpy_restatement_on_golden_vectors(tag):
    zeros = GOLD[f"ga_{tag}_zeros"] if f"ga_{tag}_zeros" in GOLD.files else None
    qw, s = GOLD[f"ga_{tag}_qw"], GOLD[f"ga_{tag}_scales"]
    _, bound = cref.c_gemm_w4a8(GOLD["q_xq"], GOLD["q_xs"], GOLD["q_asum"], qw, s, zeros)
    np.testing.assert_allclose(bound, O.w4a8_lane_bound(GOLD["q_xq"], GOLD["q_xs"], GOLD["q_asum"], qw, s, zeros),
                               rtol=1e-13, atol=0)


@pytest.mark.parametrize("m,n,k,asym,rule", [(1, 7, 128, True, "absmax"), (3, 5, 300, False, "absmax"),
                                             (4, 33, 1000, True, "absmax"), (5, 37, 300, False, "signed-max")])
def test_w4a8_bound_matches_numpy_restatement(rng, m, n, k, asym, rule):
    xq, xs, asum, W = _bound_operands(rng, m, n, k, asym, rule)
    y, bound = cref.c_gemm_w4a8(xq, xs, asum, W.qw, W.scales, W.zeros)
    np.testing.assert_allclose(bound, O.w4a8_lane_bound(xq, xs, asum, W.qw, W.scales, W.zeros), rtol=1e-13, atol=0)
    # |acc_g| = |sum (q - z) a| <= sum q|a| + z|sum a| for every group, so the bound
    # dominates the exact result itself
    assert np.all(np.abs(y) <= bound * (1 + 1e-12))
    if rule == "absmax":
        # positive scales: equal to the reference's expression with signed scales
        # (tests/test_kernels.py:115)
        q = O.unpack_codes(W.qw, 128).astype(np.float64).reshape(n, -1, 128)
        z = np.full(W.scales.shape, 8.0) if W.zeros is None else W.zeros.astype(np.float64)
        mag = (np.einsum("mgk,ngk->mng", np.abs(xq.astype(np.float64)).reshape(m, -1, 128), q)
               + z[None] * np.abs(asum.astype(np.float64))[:, None, :])
        refb = np.einsum("mng,ng->mn", mag, W.scales.astype(np.float64)) * xs.astype(np.float64)[:, None]
        np.testing.assert_allclose(bound, refb, rtol=1e-13, atol=0)


def test_w4a8_bound_closed_forms():
    # one row, one group. Case 1: every code 15, z = 0, every activation -128:
    #   sum q|a| = 128 * 15 * 128, z|sum a| = 0  ->  245760 * |s| * xs
    qw = np.full((1, 64), 0xFF, np.uint8)
    xq = np.full((1, 128), -128, np.int8)
    asum = np.array([[-128 * 128]], np.int32)
    _, b = cref.c_gemm_w4a8(xq, np.array([2.0], np.float32), asum, qw, np.array([[0.5]], np.float32),
                            np.array([[0]], np.uint8))
    assert b[0, 0] == 245760.0
    # Case 2: code 3 everywhere, z = 7, activations alternating +1 / -1 (sum 0):
    #   sum q|a| = 3 * 128 = 384, z|sum a| = 0; a negative scale counts by magnitude
    qw = np.full((1, 64), 0x33, np.uint8)
    xq = np.resize(np.array([1, -1], np.int8), (1, 128))
    y, b = cref.c_gemm_w4a8(xq, np.array([1.0], np.float32), np.array([[0]], np.int32), qw,
                            np.array([[-0.25]], np.float32), np.array([[7]], np.uint8))
    assert b[0, 0] == 384 * 0.25 and y[0, 0] == 0.0
    # Case 3: code 8 = z (symmetric zero row), activations all 5: the exact result is 0
    #   but the magnitude is sum q|a| + z|sum a| = 8 * 640 + 8 * 640
    qw = np.full((1, 64), 0x88, np.uint8)
    xq = np.full((1, 128), 5, np.int8)
    y, b = cref.c_gemm_w4a8(xq, np.array([1.0], np.float32), np.array([[640]], np.int32), qw,
                            np.array([[1.0]], np.float32), None)
    assert y[0, 0] == 0.0 and b[0, 0] == 2 * 8 * 640


def test_w4a8_bound_planted_mistakes(rng):
    """A bound without the zero-point term, or one that measures |acc| instead of the
    lane magnitudes, must fail the pins above."""
    xq, xs, asum, W = _bound_operands(rng, 3, 20, 512, True)
    _, bound = cref.c_gemm_w4a8(xq, xs, asum, W.qw, W.scales, W.zeros)
    s = np.abs(W.scales.astype(np.float64))
    q = O.unpack_codes(W.qw, 128).astype(np.float64).reshape(W.n, -1, 128)
    no_z = np.einsum("mng,ng->mn", np.einsum("mgk,ngk->mng", np.abs(xq.astype(np.float64)).reshape(3, -1, 128), q),
                     s) * xs[:, None]
    assert not np.allclose(no_z, bound, rtol=1e-6)
    acc = O.w4a8_group_acc_ref(xq, W.qw, W.zeros).astype(np.float64)
    abs_acc = np.einsum("mng,ng->mn", np.abs(acc), s) * xs[:, None]
    assert not np.allclose(abs_acc, bound, rtol=1e-6)
    # the |acc| form is never larger: it shrinks wherever a group's sum cancels, the
    # case the reference's lane magnitudes exist for (tests/test_kernels.py:108-110)
    assert np.all(abs_acc <= bound * (1 + 1e-12))


# ------------------------------------------------------------------ planted mistakes

_UNPACK = O.unpack_codes


def _swapped_unpack(qw, block):
    c = _UNPACK(qw, block)
    n, kp = c.shape
    h = block // 2
    return c.reshape(n, kp // block, 2, h)[:, :, ::-1, :].reshape(n, kp)


def test_planted_mistakes_are_caught(monkeypatch):
    """Each mutant of the oracle must fail at least one pin used above."""
    x, xq = GOLD["q_x"], GOLD["q_xq"]
    qw, z = GOLD["ga_asym_qw"], GOLD["ga_asym_zeros"]
    want = GOLD["ga_asym_out"]

    # 1. nibble halves swapped -> group accumulators differ from the reference C
    with monkeypatch.context() as mp:
        mp.setattr(O, "unpack_codes", _swapped_unpack)
        assert not np.array_equal(O.w4a8_group_acc_ref(xq, qw, z), want)

    # 2. zero-point dropped (z treated as 0) -> mismatch
    assert not np.array_equal(O.w4a8_group_acc_ref(xq, qw, np.zeros_like(z)), want)

    # 3. zero-point correction with the wrong sign: sum q*a + z*sum a
    q = O.unpack_codes(qw, 128).astype(np.int64).reshape(qw.shape[0], -1, 128)
    xa = xq.astype(np.int64).reshape(xq.shape[0], -1, 128)
    wrong = np.einsum("mgk,ngk->mng", xa, q) + z.astype(np.int64)[None] * xa.sum(-1)[:, None, :]
    assert not np.array_equal(wrong, want)

    # 4. quantizer rounding half away from zero instead of to even -> the tie KAT fails
    xt = np.zeros((1, 128), np.float32)
    xt[0, :4] = [0.5, 2.5, -2.5, 127.0]
    away = np.trunc(xt / 1.0 + np.copysign(0.5, xt)).astype(np.int8)
    assert away[0, :3].tolist() != O.quant_act_int8(xt)[0][0, :3].tolist()

    # 5. E8M0 bias off by one -> the MXFP4 golden GEMM falls outside the bound
    xm, qm, em = GOLD["mx_x"], GOLD["mx_qw"], GOLD["mx_e8m0"]
    bad = O.gemm_mxfp4_ref(xm, qm, em.astype(np.int64) + 1)
    with pytest.raises(AssertionError):
        O.assert_fp_close(GOLD["mx_y"], bad, O.fp_bound(xm, O.dequant_mxfp4(qm, em)))

    # 6. W4A16 scale applied per row instead of per group -> golden GEMM falls outside the bound
    s = GOLD["ga_asym_scales"]
    xp = F.pad_acts(x, qw.shape[1] * 2)
    bad = O.gemm_w4a16_ref(xp, qw, np.repeat(s[:, :1], s.shape[1], axis=1), z)
    with pytest.raises(AssertionError):
        O.assert_fp_close(GOLD["w4a16_asym_y"], bad, O.fp_bound(xp, O.dequant_int4(qw, s, z)))
