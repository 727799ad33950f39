"""GPU parity at the BASELINE configurations' own shapes, against the CPU oracle.

Every shape the benchmark configurations name runs here through the C ABI:
  C1  W4A16 decode, M=1 N=4096 K=4096, asym and sym weights;
  C2  all three formats at M=1 N=11008 K=4096 (the headline shape), through the
      host-pointer ABI (lb_gemm_*), through resident device handles (lbd_gemm_*) and
      through host containers made resident on first use (implicit residency), on the
      small-M kernel configuration bench.py times (asserted via lbd_gemm_plan);
  C3  W4A8 at M=16 and 64, N=11008 and 4096, K=4096, sym and asym, on both weight
      layouts of the matrix-core path, plus worst-case operand tiles (codes 0/15,
      zero-points 0/7/8/15, activations +-127/-128) at 4096 x 4096;
  C4  W4A16 and MXFP4 at M=1, 16, 64, N=4096 K=11008, rows scaled by LogNormal(0, 0.5)
      (which spreads the E8M0 block exponents).
Inputs follow the configurations: X, W ~ N(0, 1) fp32 from a seeded generator.

The bar is the reference's: |y - ref| <= 1e-5 * (|X| @ |W|^T) against float64 for
W4A16 / MXFP4 (tests/conftest.py:22-27), and 1e-5 times the lane magnitudes
sum_k q|a| + z|sum a| for W4A8 (tests/test_kernels.py:108-119); the int32 group
accumulators are compared bit for bit (src/lowbit/reference.py:18-26).
"""
from functools import lru_cache

import numpy as np
import pytest

import lowbit_amd as lb
from lowbit_amd import kernels as K
from oracle import cref
from oracle import reference as O

pytestmark = pytest.mark.gpu

RTOL = 1e-5


@lru_cache(maxsize=None)
def _weights(n, k, seed, lognormal=False):
    rng = np.random.default_rng(seed)
    w = rng.standard_normal((n, k)).astype(np.float32)
    if lognormal:
        w = (w * rng.lognormal(0.0, 0.5, (n, 1))).astype(np.float32)
    return w


@lru_cache(maxsize=None)
def _packed(fmt, n, k, seed, asym=False, lognormal=False):
    w = _weights(n, k, seed, lognormal)
    return lb.quantize_mxfp4(w) if fmt == "mxfp4" else lb.quantize_int4(w, asym=asym)


def _x(m, k, seed):
    return np.random.default_rng(seed + 1).standard_normal((m, k)).astype(np.float32)


def _call(fn, x, W, how):
    """how: "pointer" (the host-pointer ABI lb_gemm_*, weights uploaded per call),
    "handle" (an explicit to_device handle) or "implicit" (the host container, made
    resident on its first GEMM)."""
    if how == "handle":
        return fn(x, lb.to_device(W))
    with K.implicit_residency(how == "implicit"):
        return fn(x, W)


def _check(fmt, x, W, y):
    xp = lb.formats.pad_acts(x, W.kp)
    if fmt == "w4a16":
        ref = cref.c_gemm_w4a16(xp, W.qw, W.scales, W.zeros)
        bound = cref.c_gemm_w4a16(xp, W.qw, W.scales, W.zeros, absval=True)
    elif fmt == "mxfp4":
        ref = cref.c_gemm_mxfp4(xp, W.qw, W.e8m0)
        bound = cref.c_gemm_mxfp4(xp, W.qw, W.e8m0, absval=True)
    else:
        a = lb.quantize_act_int8(x)
        ref, bound = cref.c_gemm_w4a8(a.xq, a.scale, a.gsum, W.qw, W.scales, W.zeros)
    assert y.shape == ref.shape
    return O.assert_fp_close(y, ref, bound, RTOL)


# ------------------------------------------------------------------ C1

@pytest.mark.parametrize("asym", [True, False])
@pytest.mark.parametrize("how", ["pointer", "handle"])
def test_c1_w4a16_decode_4096(asym, how):
    W = _packed("w4a16", 4096, 4096, 0, asym)
    x = _x(1, 4096, 0)
    y = _call(K.gemm_w4a16, x, W, how)
    assert K.last_path() == "gfx950"
    _check("w4a16", x, W, y)


# ------------------------------------------------------------------ C2 (headline shape)

C2 = [("w4a8", True), ("w4a8", False), ("w4a16", True), ("w4a16", False), ("mxfp4", False)]


@pytest.mark.parametrize("fmt,asym", C2)
def test_c2_plan_is_the_benchmarked_kernel(fmt, asym):
    """The small-M configuration at 1 x 11008 x 4096 that bench.py times: the paced
    kernel (the row being computed and the next one in flight), two 16-byte chunks per
    lane (a row of 4096 is 128 chunks), one activation row, several rows per wave."""
    plan = K.gemm_plan(fmt, 1, 11008, 4096)
    assert plan["path"] == "gfx950"
    assert plan["act_rows"] == 1 and plan["chunks_per_lane"] == 2 and plan["two_rows_per_load"] == 0
    assert plan["rows_held"] == 2 and plan["rows_per_wave"] >= 2
    assert plan["workgroups"] * 8 * plan["rows_per_wave"] >= 11008


@pytest.mark.parametrize("how", ["pointer", "handle", "implicit"])
@pytest.mark.parametrize("fmt,asym", C2)
def test_c2_decode_11008x4096(fmt, asym, how):
    W = _packed(fmt, 11008, 4096, 0, asym)
    x = _x(1, 4096, 0)
    fn = K.GEMMS[fmt]
    y = _call(fn, x, W, how)
    assert K.last_path() == "gfx950"
    _check(fmt, x, W, y)
    if fmt == "w4a8":
        a = lb.quantize_act_int8(x)
        ref, bound = cref.c_gemm_w4a8(a.xq, a.scale, a.gsum, W.qw, W.scales, W.zeros)
        with K.implicit_residency(how != "pointer"):
            O.assert_fp_close(K.gemm_w4a8_q(a, W), ref, bound, RTOL)


@pytest.mark.parametrize("case", ["subnormal", "huge", "max", "under"])
@pytest.mark.parametrize("asym", [True, False])
def test_c2_w4a16_activation_range(case, asym):
    """Activations across the float32 range at the headline shape: all subnormal (scales
    raised so that the products and outputs stay normal), and rows scaled to 2^93..2^97
    times N(0, 1). The one-row kernel's sum q x - z sum x stays within the bound."""
    W = _packed("w4a16", 11008, 4096, 0, asym)
    x = _x(1, 4096, 3)
    if case == "subnormal":
        x = (x * np.float32(1e-39)).astype(np.float32)  # every x a float32 subnormal
        # scales times 2^100 (exact) keep the products and outputs normal, so that the
        # relative bound applies
        W = lb.Int4Weights(W.qw, (W.scales * np.float32(2.0 ** 100)).astype(np.float32), W.zeros, W.k)
    elif case == "huge":
        x = (x * np.float32(2.0 ** 97)).astype(np.float32)
    elif case == "max":
        x = (x / np.abs(x).max() * np.float32(2.0 ** 96)).astype(np.float32)
        assert np.abs(x).max() == 2.0 ** 96
    else:
        x = (x * np.float32(2.0 ** 93)).astype(np.float32)
    y = K.gemm_w4a16(x, lb.to_device(W))
    assert K.last_path() == "gfx950"
    assert np.isfinite(y).all()
    _check("w4a16", x, W, y)


# ------------------------------------------------------------------ C3 (W4A8 batches)

C3 = [(m, n, asym) for m in (16, 64) for n in (11008, 4096) for asym in (True, False)]


@pytest.mark.parametrize("how", ["handle", "pointer"])
@pytest.mark.parametrize("m,n,asym", C3)
def test_c3_w4a8_batches(m, n, asym, how):
    """Resident handles run on the t16 tile layout, the pointer ABI on the row-major
    layout; both are the int8 matrix-core path."""
    W = _packed("w4a8", n, 4096, 1, asym)
    x = _x(m, 4096, 1)
    y = _call(K.gemm_w4a8, x, W, how)
    assert K.last_path() == "gfx950-mfma"
    _check("w4a8", x, W, y)


def _adversarial_4096(rng, asym):
    n = k = 4096
    g = k // 128
    codes = rng.choice(np.array([0, 15], np.uint8), size=(n, k))
    codes[: n // 4] = 15  # whole rows at the top code
    zeros = rng.choice(np.array([0, 7, 8, 15], np.uint8), size=(n, g)) if asym else None
    W = lb.Int4Weights(lb.formats.pack_nibbles(codes, 128),
                       (rng.standard_normal((n, g)) * 0.01).astype(np.float32), zeros, k)
    xq = rng.choice(np.array([127, -128, -127], np.int8), size=(64, k))
    xq[0] = -128
    xq[1] = 127
    a = lb.Int8Acts(xq, np.abs(rng.standard_normal(64)).astype(np.float32) + 0.01,
                    xq.astype(np.int32).reshape(64, g, 128).sum(axis=2).astype(np.int32))
    return W, a


@pytest.mark.parametrize("isa", ["gfx950", "gfx950-mfma"])
@pytest.mark.parametrize("asym", [True, False])
def test_c3_worst_case_tiles_bit_exact(rng, isa, asym):
    """64 x 4096 x 4096 of worst-case operands: exact int32 group accumulators on both
    integer paths, and the fp32 rescale within the bound."""
    W, a = _adversarial_4096(rng, asym)
    want = cref.c_group_acc(a.xq, W.qw, W.zeros)
    assert np.abs(want).max() < 2 ** 31
    np.testing.assert_array_equal(K.w4a8_group_acc(a, W, isa=isa), want)
    ref, bound = cref.c_gemm_w4a8(a.xq, a.scale, a.gsum, W.qw, W.scales, W.zeros)
    O.assert_fp_close(K.gemm_w4a8_q(a, W, isa=isa), ref, bound, RTOL)


# ------------------------------------------------------------------ C4 (down-projection shape)

@pytest.mark.parametrize("how", ["handle", "pointer"])
@pytest.mark.parametrize("m", [1, 16, 64])
@pytest.mark.parametrize("fmt,asym", [("mxfp4", False), ("w4a16", True), ("w4a16", False)])
def test_c4_down_projection_lognormal_rows(fmt, asym, m, how):
    W = _packed(fmt, 4096, 11008, 2, asym, lognormal=True)
    if fmt == "mxfp4":
        assert len(np.unique(W.e8m0)) >= 6  # the row scaling spreads the block exponents
    x = _x(m, 11008, 2)
    y = _call(K.GEMMS[fmt], x, W, how)
    assert K.last_path() == ("gfx950" if m == 1 else "gfx950-mfma")
    _check(fmt, x, W, y)


# ------------------------------------------------------------------ rows past 4096 elements

def test_c4_plan_splits_rows_over_waves():
    """At M=1 the down-projection's W4A16 and MXFP4 rows (11008 elements, 344 chunks)
    are cut into three slices of at most 128 chunks, one wave each, two chunks per
    lane; W4A8 rows and the headline shape's rows are not split."""
    for fmt in ("w4a16", "mxfp4"):
        plan = K.gemm_plan(fmt, 1, 4096, 11008)
        assert plan["path"] == "gfx950" and plan["k_slices"] == 3 and plan["chunks_per_lane"] == 2
        assert plan["rows_held"] == 2 and plan["act_rows"] == 1
    assert K.gemm_plan("w4a8", 1, 4096, 11008)["k_slices"] == 1
    for fmt in ("w4a16", "mxfp4", "w4a8"):
        assert K.gemm_plan(fmt, 1, 11008, 4096)["k_slices"] == 1


# (format, asym, rows, row length, slices): fp32 rows split up to 12288 elements (the
# planes of whole slices within the 60 KB LDS budget); a 13312-element row (416
# chunks: four slices would need 64 KB) and every W4A8 row keep the unsplit kernel
SPLIT = [("w4a16", True, 4097, 4224, 2), ("w4a16", False, 1000, 12288, 3), ("mxfp4", False, 4097, 8224, 3),
         ("mxfp4", False, 3000, 12288, 3), ("w4a16", True, 1500, 13312, 1), ("w4a8", True, 4096, 11008, 1),
         ("w4a8", False, 1000, 16384, 1),
         # fewer rows than the CUs' workgroups of full size: one to a few row-slices
         # per wave, some waves without rows
         ("w4a16", True, 1, 11008, 3), ("mxfp4", False, 7, 5000, 2), ("w4a16", False, 896, 4864, 2),
         ("mxfp4", False, 1023, 11008, 3), ("w4a16", True, 2047, 8192, 2)]


@pytest.mark.parametrize("fmt,asym,n,k,slices", SPLIT)
def test_split_rows_against_oracle(fmt, asym, n, k, slices):
    """One activation row against rows of 4224..16384 elements: two or three slices,
    the last one mostly past the row's end (4224: 4 of 128 chunks) or partial (8224:
    257 chunks), odd row counts; the rows that stay unsplit checked alongside."""
    W = _packed(fmt, n, k, 5, asym)
    x = _x(1, k, 5)
    plan = K.gemm_plan(fmt, 1, n, W.kp)
    assert plan["path"] == "gfx950" and plan["k_slices"] == slices
    y = K.GEMMS[fmt](x, lb.to_device(W))
    assert K.last_path() == "gfx950"
    _check(fmt, x, W, y)


def test_split_rows_few_rows_fill_the_cus():
    """With fewer rows than workgroups of full size would give every CU, the split
    GEMV spreads them over more workgroups (at most one per CU) to reach the fewest
    row-slices per wave, and no more workgroups than that takes (row lengths padded
    to whole groups, as `gemm_plan` takes them)."""
    cus = K.gemm_plan("w4a16", 1, 4096, 11008)["workgroups"]  # one per CU at this shape
    for fmt, n, k, wg, rpw in [("w4a16", 1024, 11008, cus, 1), ("mxfp4", 1024, 11008, cus, 1),
                               ("w4a16", 896, 4864, 224, 1), ("mxfp4", 896, 4864, 112, 1),
                               ("w4a16", 1536, 5120, 192, 2), ("mxfp4", 1, 11008, 1, 1)]:
        plan = K.gemm_plan(fmt, 1, n, k)
        assert plan["k_slices"] > 1 and plan["workgroups"] == wg and plan["rows_per_wave"] == rpw, (fmt, n, k, plan)


def test_split_rows_zero_rows_exact():
    """Rows whose codes all equal the zero-point give exactly 0 in every slice, so
    exactly 0 after the slices are added (symmetric int4 of zero rows: q = z = 8)."""
    rng = np.random.default_rng(9)
    w = rng.standard_normal((512, 12288)).astype(np.float32)
    w[::7] = 0.0
    W = lb.quantize_int4(w)
    x = rng.standard_normal((1, 12288)).astype(np.float32)
    for fn in (K.gemm_w4a16, K.gemm_w4a8):
        y = fn(x, lb.to_device(W))
        assert np.all(y[:, ::7] == 0)
        _check("w4a16" if fn is K.gemm_w4a16 else "w4a8", x, W, y)
