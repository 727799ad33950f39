"""A seeded sweep of shapes (GPU) through every call route, against the oracle.

The fixed-shape tests pin each kernel at chosen shapes; this sweep draws 20 shapes per
format and route with M on and around every regime boundary (the one-row GEMV, the
M <= 4 VALU kernels, 16-row MFMA tiles and their tails, 64-row tiles, wide M), N with
ragged 16-row subtiles and K not a multiple of the group or block (the caller's X is
padded, as the reference pads it, src/lowbit/formats.py:227-233), and activations that
are Gaussian, heavy-tailed with outliers, hold an all-zero row, sit at 1e-30 or 1e15,
spread over many exponents or are mostly zeros; weight rows are Gaussian, spread over
exponents, zero or dominated by one entry. Routes: the
host-pointer ABI (weights uploaded per call), implicit residency (host containers made
resident on their first call) and explicit `to_device` handles. Bar: the reference's
bounds (tests/conftest.py:22-27, tests/test_kernels.py:108-116 of the reference):
1e-5 * (|X| @ |W|^T) for W4A16 / MXFP4 and the W4A8 lane bound on the oracle's codes.
"""
import numpy as np
import pytest

import lowbit_amd as lb
from lowbit_amd import kernels as K
from oracle import cref
from oracle import reference as O

pytestmark = pytest.mark.gpu

M_CHOICES = [1, 1, 2, 3, 4, 5, 8, 15, 16, 17, 31, 32, 33, 47, 48, 63, 64, 65, 80, 130]
ROUTES = ["pointer", "implicit", "handle"]
RTOL = 1e-5


def shapes(seed: int, count: int = 20):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(count):
        m = M_CHOICES[i % len(M_CHOICES)]
        n = int(rng.choice([int(rng.integers(1, 600)), 16 * int(rng.integers(1, 40)) + int(rng.choice([-1, 0, 1]))]))
        k = int(rng.choice([int(rng.integers(1, 2600)), 128 * int(rng.integers(1, 20)), 32 * int(rng.integers(1, 80))]))
        out.append((m, max(n, 1), max(k, 1)))
    return out


ACT_KINDS = 6


def activations(rng, m, k, kind):
    x = rng.standard_normal((m, k)).astype(np.float32)
    if kind == 1:  # heavy tails: a few outliers per row, 1e3 times the rest
        idx = rng.integers(0, k, (m, max(1, k // 200)))
        np.put_along_axis(x, idx, rng.standard_normal(idx.shape).astype(np.float32) * 1e3, axis=1)
    elif kind == 2 and m > 1:
        x[m // 2] = 0.0
    elif kind == 3:  # tiny (1e-30) and huge (1e15) rows, far from 1 in both directions
        x *= np.where(np.arange(m)[:, None] % 2 == 0, 1e-30, 1e15).astype(np.float32)
    elif kind == 4:  # rows of very different scale: LogNormal(0, 3) per row
        x *= np.exp(rng.normal(0.0, 3.0, (m, 1))).astype(np.float32)
    elif kind == 5:  # sparse: about 90 % exact zeros
        x *= (rng.random((m, k)) < 0.1).astype(np.float32)
    return x


def weights(rng, n, k, kind):
    w = rng.standard_normal((n, k)).astype(np.float32)
    if kind == 1:  # rows spread over many exponents (the C4 rows of BASELINE)
        w *= np.exp(rng.normal(0.0, 0.5, (n, 1))).astype(np.float32)
    elif kind == 2 and n > 2:  # a zero row and a row with one dominant entry
        w[0] = 0.0
        w[1, rng.integers(0, k)] = 1e4
    return w


def run(fmt, route, x, W):
    fn = {"w4a16": K.gemm_w4a16, "w4a8": K.gemm_w4a8, "mxfp4": K.gemm_mxfp4}[fmt]
    if route == "handle":
        return fn(x, lb.to_device(W))
    with K.implicit_residency(route == "implicit"):
        y = fn(x, W)
        if route == "implicit":
            y2 = fn(x, W)  # the second call reads the resident copy
            np.testing.assert_array_equal(y2, y)
            lb.release(W)
        return y


@pytest.mark.parametrize("route", ROUTES)
@pytest.mark.parametrize("fmt", ["w4a16", "w4a8", "mxfp4"])
def test_random_shapes(fmt, route):
    seed = 20261202 + 97 * ["w4a16", "w4a8", "mxfp4"].index(fmt) + ROUTES.index(route)
    rng = np.random.default_rng(seed)
    worst = 0.0
    for i, (m, n, k) in enumerate(shapes(seed)):
        kind, wkind = i % ACT_KINDS, (i // 2) % 3
        asym = bool(i % 2) and fmt != "mxfp4"
        print(f"[{fmt} {route}] shape {i}: M={m} N={n} K={k} asym={asym} acts={kind} weights={wkind}", flush=True)
        w = weights(rng, n, k, wkind)
        x = activations(rng, m, k, kind)
        if fmt == "mxfp4":
            W = lb.quantize_mxfp4(w)
            xp = lb.formats.pad_acts(x, W.kp)
            ref, bound = O.gemm_mxfp4_ref(xp, W.qw, W.e8m0), cref.c_gemm_mxfp4(xp, W.qw, W.e8m0, absval=True)
        elif fmt == "w4a16":
            W = lb.quantize_int4(w, asym=asym)
            xp = lb.formats.pad_acts(x, W.kp)
            ref = O.gemm_w4a16_ref(xp, W.qw, W.scales, W.zeros)
            bound = cref.c_gemm_w4a16(xp, W.qw, W.scales, W.zeros, absval=True)
        else:
            W = lb.quantize_int4(w, asym=asym)
            a = lb.quantize_act_int8(x)
            ref, bound = cref.c_gemm_w4a8(a.xq, a.scale, a.gsum, W.qw, W.scales, W.zeros)
        y = run(fmt, route, x, W)
        assert y.shape == (m, n) and y.dtype == np.float32
        worst = max(worst, O.assert_fp_close(y, ref, bound, RTOL))
        if kind == 2 and m > 1:
            assert not y[m // 2].any()  # a zero activation row gives exact zeros
    print(f"[{fmt} {route}] worst err / limit {worst:.3g}")


@pytest.mark.parametrize("fmt", ["w4a16", "mxfp4"])
@pytest.mark.parametrize("m", [1, 3, 16, 64])
@pytest.mark.parametrize("mag", [1e-36, 1e-33, 1e-30, 1e-10, 1e10, 1e30])
def test_activation_magnitudes(fmt, m, mag):
    """Rows of one magnitude far from 1, through the GEMVs (M <= 4) and the matrix
    cores (M >= 5): MXFP4's three bf16 terms keep fp32's 24 bits down to rows of 1e-36
    (below that the matrix cores flush the smallest term); W4A16's two float16 terms
    of each row scaled by its own power of two keep 22 bits at any row magnitude."""
    rng = np.random.default_rng(int(abs(np.log10(mag))) * 10 + m)
    n, k = 96, 1024
    w = rng.standard_normal((n, k)).astype(np.float32)
    x = (rng.standard_normal((m, k)) * mag).astype(np.float32)
    if fmt == "mxfp4":
        W = lb.quantize_mxfp4(w)
        xp = lb.formats.pad_acts(x, W.kp)
        ref, bound = O.gemm_mxfp4_ref(xp, W.qw, W.e8m0), cref.c_gemm_mxfp4(xp, W.qw, W.e8m0, absval=True)
        y = K.gemm_mxfp4(x, lb.to_device(W))
    else:
        W = lb.quantize_int4(w, asym=True)
        xp = lb.formats.pad_acts(x, W.kp)
        ref = O.gemm_w4a16_ref(xp, W.qw, W.scales, W.zeros)
        bound = cref.c_gemm_w4a16(xp, W.qw, W.scales, W.zeros, absval=True)
        y = K.gemm_w4a16(x, lb.to_device(W))
    assert np.isfinite(y).all()
    # assert_fp_close's absolute floor (1e-30) would hide errors at these magnitudes
    err = np.abs(y.astype(np.float64) - ref)
    worst = float((err / (RTOL * bound + 1e-300)).max())
    assert worst <= 1.0, f"max err/limit = {worst:.3g}"


@pytest.mark.parametrize("m", [16, 64])
def test_w4a16_batch_rows_of_mixed_magnitude_and_range(m):
    """The W4A16 matrix-core path scales each activation row by its own power of two
    before the float16 split: rows from 1e-36 to 1e30 in one call, and rows whose
    few huge entries (2^26 times the rest, at the weights' zero-point codes, so the
    reference's bound takes nothing from them) leave the other entries within 2^28
    of the row's largest, where each keeps an absolute error of at most 2^-39 of
    that largest entry."""
    rng = np.random.default_rng(4242 + m)
    n, k = 96, 1024
    mags = np.array([1e-36, 1e-20, 1e-3, 1.0, 1e5, 1e18, 1e30])
    x = rng.standard_normal((m, k)) * mags[np.arange(m) % len(mags)][:, None]
    w = rng.standard_normal((n, k)).astype(np.float32)
    W = lb.quantize_int4(w, asym=True)
    codes = W.codes()
    z = np.repeat(W.zeros, W.group, axis=1)[:, :W.kp]
    for i in range(1, m, 3):  # every third row: outliers at zero-point codes
        cols = rng.choice(k, size=3, replace=False)
        x[i] = rng.standard_normal(k)
        x[i, cols] = 2.0 ** 26 * rng.choice([-1.0, 1.0], size=3)
        codes[:, cols] = z[:, cols]
    W = lb.formats.Int4Weights(lb.formats.pack_nibbles(codes.astype(np.uint8), W.group), W.scales, W.zeros,
                               W.k, W.group)
    x = x.astype(np.float32)
    assert K.gemm_plan("w4a16", m, n, W.kp)["path"] == "gfx950-mfma"
    xp = lb.formats.pad_acts(x, W.kp)
    ref = O.gemm_w4a16_ref(xp, W.qw, W.scales, W.zeros)
    bound = cref.c_gemm_w4a16(xp, W.qw, W.scales, W.zeros, absval=True)
    for y in (K.gemm_w4a16(x, W), K.gemm_w4a16(x, lb.to_device(W))):
        assert np.isfinite(y).all()
        err = np.abs(y.astype(np.float64) - ref)
        worst = float((err / (RTOL * bound + 1e-300)).max())
        assert worst <= 1.0, f"max err/limit = {worst:.3g}"
