"""Small-M GEMVs with more rows per wave than one epilogue window holds (GPU).

`gemv_kernel` reduces each row into one lane of a result register and runs its
epilogue once per window of up to 64 rows, one row per lane. The decoder's shapes
give every wave one window; these shapes (N = 300001 rows of K = 128 elements, over
a persistent grid of at most a few thousand waves) give each wave two or more, with
a ragged last window. Checked against the oracle (the float64 bound for W4A16 /
MXFP4, the W4A8 lane bound on the oracle's codes; tests/conftest.py:22-27 and
tests/test_kernels.py:108-116 of the reference) at one row (two rows per wave
load) and three rows (one row per load), and, for the fused epilogues, bit for
bit against the plain GEMV's output: fp32 `res + (y + bias)` in numpy, the SwiGLU
pairs through lbd_swiglu_pairs, and numpy's argmax. Rows of 32 to 1024 elements
on the two-rows-per-load path (each batch's metadata in one load per array) are
checked at two row counts, with and without zero-points.
"""
import numpy as np
import pytest

import lowbit_amd as lb
from lowbit_amd import kernels as K
from oracle import cref
from oracle import reference as O

# the fused-GEMV helpers, and the autouse fixture that frees their buffers after each test
from test_gpu_fused import FORMATS, _LIVE, _release_buffers, fused, ok, plain, up  # noqa: F401

pytestmark = pytest.mark.gpu

N, KDIM = 300001, 128


def quantized(rng, fmt, n, k):
    w = rng.standard_normal((n, k)).astype(np.float32)
    return lb.quantize_mxfp4(w) if fmt == "mxfp4" else lb.quantize_int4(w, asym=True)


def check_oracle(fmt, x, W, y):
    if fmt == "w4a8":
        a = lb.quantize_act_int8(x)
        ref, bound = cref.c_gemm_w4a8(a.xq, a.scale, a.gsum, W.qw, W.scales, W.zeros)
    elif fmt == "mxfp4":
        ref, bound = O.gemm_mxfp4_ref(x, W.qw, W.e8m0), cref.c_gemm_mxfp4(x, W.qw, W.e8m0, absval=True)
    else:
        ref = O.gemm_w4a16_ref(x, W.qw, W.scales, W.zeros)
        bound = cref.c_gemm_w4a16(x, W.qw, W.scales, W.zeros, absval=True)
    return O.assert_fp_close(y, ref, bound, 1e-5)


@pytest.mark.parametrize("fmt", FORMATS)
@pytest.mark.parametrize("m", [1, 3])
def test_many_rows_within_bound(rng, fmt, m):
    W = quantized(rng, fmt, N, KDIM)
    x = rng.standard_normal((m, KDIM)).astype(np.float32)
    plan = K.gemm_plan(fmt, m, N, KDIM)
    rr = plan["rows_held"]
    window = 64 // (2 * rr) * (2 * rr) if rr % 2 else 64 // rr * rr  # rows per epilogue window
    assert plan["rows_per_wave"] > window, plan  # two windows or more per wave
    fn = {"w4a16": K.gemm_w4a16, "w4a8": K.gemm_w4a8, "mxfp4": K.gemm_mxfp4}[fmt]
    y = fn(x, lb.to_device(W))
    assert y.shape == (m, N)
    check_oracle(fmt, x, W, y)


@pytest.mark.parametrize("fmt", FORMATS)
def test_many_rows_fused_epilogues(rng, fmt):
    W = quantized(rng, fmt, N, KDIM)
    dw = K.to_device(W)
    x = rng.standard_normal(KDIM).astype(np.float32)
    b = rng.standard_normal(N).astype(np.float32)
    r = rng.standard_normal(N).astype(np.float32)
    dx = up(x)
    yp = K.DeviceBuffer(4 * N)
    _LIVE.append(yp)
    plain(fmt, dw, dx.ptr, yp.ptr)
    y0 = yp.to_array((N,), np.float32)
    check_oracle(fmt, x[None], W, y0[None])
    # bias and residual, the residual updated in place
    dr = up(r)
    ok(fused(fmt, dw, dx.ptr, dr.ptr, bias=up(b).ptr, res=dr.ptr))
    np.testing.assert_array_equal(dr.to_array((N,), np.float32), r + (y0 + b))
    # argmax key: numpy's first maximum
    key = up(np.zeros(1024, np.uint64))
    tok, pos, hist = up(np.zeros(1, np.int32)), up(np.array([0], np.int32)), up(np.full(2, -1, np.int32))
    dy = K.DeviceBuffer(4 * N)
    _LIVE.append(dy)
    ok(fused(fmt, dw, dx.ptr, dy.ptr, key=key.ptr))
    np.testing.assert_array_equal(dy.to_array((N,), np.float32), y0)
    ok(K.lib().lbd_argmax_finalize(key.ptr, tok.ptr, pos.ptr, 1, hist.ptr, 2, None))
    assert tok.to_array((1,), np.int32)[0] == int(np.argmax(y0))


@pytest.mark.parametrize("fmt", FORMATS)
def test_many_rows_glu_pairs(rng, fmt):
    n = N + 1  # (gate, up) pairs
    W = quantized(rng, fmt, n, KDIM)
    dw = K.to_device(W)
    dx = up(rng.standard_normal(KDIM).astype(np.float32))
    yp, ref, yg = K.DeviceBuffer(4 * n), K.DeviceBuffer(4 * n // 2), K.DeviceBuffer(4 * n // 2)
    _LIVE.extend([yp, ref, yg])
    plain(fmt, dw, dx.ptr, yp.ptr)
    ok(K.lib().lbd_swiglu_pairs(yp.ptr, 1, n // 2, ref.ptr, None))
    ok(fused(fmt, dw, dx.ptr, yg.ptr, glu=True))
    np.testing.assert_array_equal(yg.to_array((n // 2,), np.float32), ref.to_array((n // 2,), np.float32))


@pytest.mark.parametrize("fmt", FORMATS)
@pytest.mark.parametrize("k", [32, 96, 352, 1000, 1024])
@pytest.mark.parametrize("n", [9000, 20011])
def test_two_rows_per_load_row_lengths(rng, fmt, k, n):
    """One activation row, rows of 1..8 groups (one to 32 chunks), two rows per wave
    load with 1-3 slots per batch: each batch's scales and zero-points come in one
    load each and reach their lanes by cross-lane permute. Symmetric, asymmetric and
    signed-max (negative scales) int4, against the oracle's bounds."""
    for asym, scale in ([(False, "absmax"), (True, "absmax"), (False, "signed-max")] if fmt != "mxfp4"
                        else [(False, None)]):
        w = rng.standard_normal((n, k)).astype(np.float32)
        W = lb.quantize_mxfp4(w) if fmt == "mxfp4" else lb.quantize_int4(w, asym=asym, scale=scale)
        assert K.gemm_plan(fmt, 1, n, W.kp)["two_rows_per_load"] == 1
        x = rng.standard_normal((1, k)).astype(np.float32)
        fn = {"w4a16": K.gemm_w4a16, "w4a8": K.gemm_w4a8, "mxfp4": K.gemm_mxfp4}[fmt]
        y = fn(x, lb.to_device(W))
        check_oracle(fmt, lb.formats.pad_acts(x, W.kp), W, y)


@pytest.mark.parametrize("fmt", ["w4a16", "w4a8"])
@pytest.mark.parametrize("k", [4096, 6000, 11008])
def test_one_row_negative_scales(rng, fmt, k):
    """signed-max int4 (negative group scales, tests/test_kernels.py:44-58 of the
    reference) through the one-row paced GEMVs: unsplit rows, and rows cut into two
    or three slices (W4A16)."""
    n = 3001
    W = lb.quantize_int4(rng.standard_normal((n, k)).astype(np.float32), scale="signed-max")
    assert (W.scales < 0).any()
    x = rng.standard_normal((1, k)).astype(np.float32)
    fn = {"w4a16": K.gemm_w4a16, "w4a8": K.gemm_w4a8}[fmt]
    y = fn(x, lb.to_device(W))
    check_oracle(fmt, lb.formats.pad_acts(x, W.kp), W, y)
