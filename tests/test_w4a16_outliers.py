"""Why the W4A16 kernels multiply by the dequantized code (q - z), not q then z * sum x.

On activations with a few huge entries where the weight's code equals its zero-point
(tests/problems.py), the reference's bound 1e-5 * (|X| @ |W|^T) takes nothing from
those entries. A float32 emulation of the chunk arithmetic shows that forming
sum q x - z sum x per 32-code chunk misses the bound by a factor of tens to
thousands there, while the dequantized form (the reference's, src/lowbit/csrc/
kern_scalar.c:10-29, and the device kernels') stays far inside it. The device side of
the same problem is tests/test_gpu_kernels.py::test_w4a16_outliers_at_zero_point_codes.
"""
import numpy as np
import pytest

from lowbit_amd import formats as F
from oracle import reference as O
from problems import outlier_int4_problem


def chunk_emulation(x, W, split: bool) -> np.ndarray:
    """float32 emulation of the GEMV's per-chunk arithmetic (32 codes per chunk, each
    step rounded to float32), vectorised over rows of X and W."""
    m, n = x.shape[0], W.n
    xp = F.pad_acts(x, W.kp).astype(np.float32)
    q = W.codes().astype(np.float32)
    z = np.repeat(W.zeros, W.group, axis=1).astype(np.float32)
    s = np.repeat(W.scales, W.group, axis=1).astype(np.float32)
    acc = np.zeros((m, n), np.float32)
    for c0 in range(0, W.kp, 32):
        part = np.zeros((m, n), np.float32)
        xsum = np.zeros((m, 1), np.float32)
        for t in range(c0, c0 + 32):
            xt = xp[:, t:t + 1]
            if split:
                part = (part + (q[None, :, t] * xt).astype(np.float32)).astype(np.float32)
                xsum = (xsum + xt).astype(np.float32)
            else:
                part = (part + ((q[None, :, t] - z[None, :, t]) * xt).astype(np.float32)).astype(np.float32)
        if split:
            part = (part - (z[None, :, c0] * xsum).astype(np.float32)).astype(np.float32)
        acc = (acc + (s[None, :, c0] * part).astype(np.float32)).astype(np.float32)
    return acc


@pytest.mark.parametrize("m,n,k", [(1, 40, 256), (3, 40, 256), (1, 64, 4096)])
def test_split_zero_point_form_misses_the_bound(m, n, k):
    rng = np.random.default_rng(7 + k)
    x, W = outlier_int4_problem(rng, m, n, k)
    xp = F.pad_acts(x, W.kp)
    ref = O.gemm_w4a16_ref(xp, W.qw, W.scales, W.zeros)
    bound = O.fp_bound(xp, W.dequantize())
    assert O.assert_fp_close(chunk_emulation(x, W, split=False), ref, bound) < 0.05
    with pytest.raises(AssertionError):
        O.assert_fp_close(chunk_emulation(x, W, split=True), ref, bound)
