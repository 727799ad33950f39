"""numpy oracle: float64 / int64 ground truth for the fused dequantize+GEMM path.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py). Functions take raw packed
arrays, never the product's containers, and decode the packed layouts with
their own code, so a decoding mistake in the product cannot hide here.

Each function cites the reference it restates (paths relative to the
reference repository root).
"""
from __future__ import annotations

import numpy as np

GROUP = 128
MXBLOCK = 32

# OCP MX E2M1 magnitudes for codes 0..7; codes 8..15 are the negatives
# (src/lowbit/formats.py:23-24, src/lowbit/csrc/kern_scalar.c:6-8).
_E2M1_MAG = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0], np.float64)


def unpack_codes(qw: np.ndarray, block: int) -> np.ndarray:
    """Packed bytes [N, Kp/2] -> codes [N, Kp] (uint8).

    Inside each block, byte j holds element j in its low nibble and element
    j + block/2 in its high nibble (src/lowbit/csrc/lowbit.h:9-19,
    src/lowbit/formats.py:34-51). Written as an explicit index map so that it
    shares no code with the packer it checks.
    """
    qw = np.asarray(qw, np.uint8)
    n, nb = qw.shape
    kp = 2 * nb
    half = block // 2
    k = np.arange(kp)
    blk, pos = k // block, k % block
    byte = blk * half + (pos % half)
    high = pos >= half
    b = qw[:, byte]
    return np.where(high[None, :], b >> 4, b & 15).astype(np.uint8)


def e8m0_value(e: np.ndarray) -> np.ndarray:
    """E8M0 -> float64: 2^(e-127); 255 -> NaN (src/lowbit/csrc/lowbit.h:84-88)."""
    e = np.asarray(e, np.int64)
    out = np.power(2.0, (e - 127).astype(np.float64))
    return np.where(e == 255, np.nan, out)


def e2m1_value(code: np.ndarray) -> np.ndarray:
    code = np.asarray(code, np.int64)
    mag = _E2M1_MAG[code & 7]
    return np.where(code & 8, -mag, mag)


def dequant_int4(qw, scales, zeros, k: int | None = None, group: int = GROUP) -> np.ndarray:
    """[N, K] float64 values of int4 weights with groups of `group` (the reference's
    128; 32 is the product's extension, the same formula), (q - z) * s.

    The product (q - z) * s is rounded to float32 first, as the reference's
    dequantize does (src/lowbit/formats.py:82-87), then widened.
    """
    q = unpack_codes(qw, group).astype(np.float32)
    n, kp = q.shape
    g = kp // group
    q = q.reshape(n, g, group)
    z = np.float32(8.0) if zeros is None else np.asarray(zeros, np.float32)[:, :, None]
    w = ((q - z) * np.asarray(scales, np.float32)[:, :, None]).reshape(n, kp)
    return w[:, : (kp if k is None else k)].astype(np.float64)


def dequant_mxfp4(qw, e8m0, k: int | None = None) -> np.ndarray:
    """[N, K] float64 values of MXFP4 weights, e2m1(q) * 2^(e-127) (exact in float64)
    (src/lowbit/formats.py:169-172)."""
    c = unpack_codes(qw, MXBLOCK)
    n, kp = c.shape
    v = e2m1_value(c).reshape(n, kp // MXBLOCK, MXBLOCK) * e8m0_value(e8m0)[:, :, None]
    return v.reshape(n, kp)[:, : (kp if k is None else k)]


def _xpad(x: np.ndarray, kp: int) -> np.ndarray:
    x = np.atleast_2d(np.asarray(x, np.float64))
    if x.shape[1] < kp:
        x = np.concatenate([x, np.zeros((x.shape[0], kp - x.shape[1]))], axis=1)
    return x


def gemm_w4a16_ref(x, qw, scales, zeros, group: int = GROUP) -> np.ndarray:
    """Y = X @ dequant(W)^T in float64 (src/lowbit/reference.py:9-11)."""
    w = dequant_int4(qw, scales, zeros, group=group)
    return _xpad(x, w.shape[1]) @ w.T


def gemm_mxfp4_ref(x, qw, e8m0) -> np.ndarray:
    """Y = X @ dequant(W)^T in float64 (src/lowbit/reference.py:14-15)."""
    w = dequant_mxfp4(qw, e8m0)
    return _xpad(x, w.shape[1]) @ w.T


def quant_act_int8(x: np.ndarray, kp: int | None = None):
    """Per-token int8 quantizer -> (xq int8 [M,Kp], xs float32 [M], asum int32 [M,G]).

    Restates src/lowbit/csrc/dispatch.c:231-257 and src/lowbit/formats.py:236-248:
    amax = max |x| over the padded row, sc = amax/127 in float32 (1 when amax is
    0), q = clip(rint(x / sc), -127, 127) with float32 division and
    round-half-to-even, asum = per-group sum of q.
    """
    x = np.atleast_2d(np.asarray(x, np.float32))
    m, k = x.shape
    kp = ((k + GROUP - 1) // GROUP) * GROUP if kp is None else kp
    xp = np.zeros((m, kp), np.float32)
    xp[:, :k] = x
    amax = np.max(np.abs(xp), axis=1)
    xs = np.ones(m, np.float32)
    pos = amax > 0
    xs[pos] = amax[pos] / np.float32(127.0)
    v = np.rint(np.divide(xp, xs[:, None], dtype=np.float32))
    xq = np.clip(v, -127.0, 127.0).astype(np.int8)
    asum = xq.astype(np.int64).reshape(m, kp // GROUP, GROUP).sum(axis=2).astype(np.int32)
    return xq, xs, asum


def w4a8_group_acc_ref(xq, qw, zeros, group: int = GROUP) -> np.ndarray:
    """Exact int64 acc[m, n, g] = sum_{k in g} (q[n,k] - z[n,g]) * xq[m,k]
    (src/lowbit/reference.py:18-26; `group` 32 is the product's extension)."""
    xq = np.atleast_2d(np.asarray(xq, np.int64))
    q = unpack_codes(qw, group).astype(np.int64)
    n, kp = q.shape
    m = xq.shape[0]
    g = kp // group
    z = np.full((n, g), 8, np.int64) if zeros is None else np.asarray(zeros, np.int64)
    qc = q.reshape(n, g, group) - z[:, :, None]
    xa = xq.reshape(m, g, group)
    out = np.empty((m, n, g), np.int64)
    for gi in range(g):  # int64 matmul per group: exact, and fast enough for test sizes
        out[:, :, gi] = xa[:, gi, :] @ qc[:, gi, :].T
    return out


def gemm_w4a8_ref(xq, xs, qw, scales, zeros, group: int = GROUP) -> np.ndarray:
    """Y[m,n] = xs[m] * sum_g s[n,g] * acc[m,n,g] in float64 (src/lowbit/reference.py:29-34)."""
    acc = w4a8_group_acc_ref(xq, qw, zeros, group).astype(np.float64)
    y = np.einsum("mng,ng->mn", acc, np.asarray(scales, np.float64))
    return y * np.asarray(xs, np.float64)[:, None]


def w4a8_lane_bound(xq, xs, asum, qw, scales, zeros, group: int = GROUP) -> np.ndarray:
    """Magnitude the W4A8 fp32 rescale error is measured against: per group
    sum_k q|a| + z|sum a|, times |s| and xs (tests/test_kernels.py:108-116).
    `asum` holds the activation sums per group of `group`."""
    xq = np.atleast_2d(np.asarray(xq, np.float64))
    q = unpack_codes(qw, group).astype(np.float64)
    n, kp = q.shape
    g = kp // group
    z = np.full((n, g), 8.0) if zeros is None else np.asarray(zeros, np.float64)
    aa = np.abs(xq).reshape(-1, g, group)
    qq = q.reshape(n, g, group)
    mag = np.einsum("mgk,ngk->mng", aa, qq) + z[None] * np.abs(np.asarray(asum, np.float64))[:, None, :]
    return np.einsum("mng,ng->mn", mag, np.abs(np.asarray(scales, np.float64))) * np.abs(
        np.asarray(xs, np.float64))[:, None]


def fp_bound(x, w_dense: np.ndarray) -> np.ndarray:
    """|X| @ |W|^T in float64: the natural scale of fp32 dot-product error
    (tests/conftest.py:22-27)."""
    return np.abs(_xpad(x, w_dense.shape[1])) @ np.abs(w_dense).T


def assert_fp_close(y, ref, bound, rtol: float = 1e-5) -> float:
    """|y - ref| <= rtol * bound elementwise (tests/conftest.py:22-27). Returns max err/limit."""
    err = np.abs(np.asarray(y, np.float64) - ref)
    lim = rtol * bound + 1e-30
    worst = float(np.max(err / lim)) if err.size else 0.0
    assert worst <= 1.0, f"max err/limit = {worst:.3g} (max abs err {err.max():.3g})"
    return worst
