"""bench.py's measurement path computes what it times: every format through the
launch bench.py captures (decode GEMV, and the matrix-core GEMMs on whichever weight
layout the shape takes), checked against the float64 C oracle the benchmark's own
rel_err uses. The timing itself is not checked."""
import numpy as np
import pytest

import bench
import lowbit_amd as lb

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    return bench.Dev()


@pytest.mark.parametrize("fmt", ["w4a8", "w4a16", "mxfp4"])
@pytest.mark.parametrize("m,n,k", [(1, 1024, 1024), (16, 1024, 1024), (64, 1024, 2048)])
def test_measure_computes_the_gemm(dev, fmt, m, n, k):
    rng = np.random.default_rng(7)
    x = rng.standard_normal((m, k)).astype(np.float32)
    w = rng.standard_normal((n, k)).astype(np.float32)
    W = lb.quantize_mxfp4(w) if fmt == "mxfp4" else lb.quantize_int4(w, asym=True)
    r = bench.measure(dev, fmt, (m, n, k), W, x, cold=False, steps=1, warmup=1)
    err = bench.rel_err(fmt, W, x, r["y"])
    # W4A8: the activations' int8 rounding against the float64 reference of the
    # same codes is exact up to fp32 sums (the benchmark reports ~2e-7)
    assert err < 1e-5, (fmt, m, r["weight_layout"], err)
    assert r["us_per_call"] > 0
