"""The fused decode entry points against the unfused ones and the oracle.

* lbd_gemv_*_fused: the RMSNorm and SwiGLU prologues and the bias / residual
  epilogue. Where the prologue's result is exactly representable (constructed
  rows: power-of-two magnitudes for the norm, silu(g) == g for large g), the fused
  GEMV must equal the plain GEMV on the host-computed activations bit for bit,
  for every format (W4A8 included: its int8 codes then come from the same fp32
  values). On random rows W4A16 / MXFP4 are held to the float64 oracle's bound
  1e-5 * (|act| @ |W|^T) (tests/conftest.py:22-27 of the reference), with the
  activations computed in float64 from the reference's formulas
  (src/lowbit/model.py:190-192, 213). The epilogue is fp32 `res + (y + bias)`,
  checked bit for bit against numpy on the plain GEMV's y.
* the argmax key: numpy's argmax of the fused GEMV's output (first maximum among
  ties, first NaN), via lbd_argmax_finalize, with pos / hist bookkeeping.
* lbd_attention_decode against a float64 restatement of one-token attention
  (src/lowbit/model.py:201-210, 353-378) and, for the cache write, against
  lbd_qkv_rope on the same row.
"""
import ctypes as C

import numpy as np
import pytest

from lowbit_amd import formats as F
from lowbit_amd import kernels as K
from lowbit_amd import model as DM
from oracle import model_ref as MR
from oracle import reference as O

pytestmark = pytest.mark.gpu

FORMATS = ["w4a16", "mxfp4", "w4a8"]
_LIVE: list = []


@pytest.fixture(autouse=True)
def _release_buffers():
    yield
    _LIVE.clear()


def up(a):
    b = K.DeviceBuffer.from_array(np.ascontiguousarray(a))
    _LIVE.append(b)
    return b


def ok(rc):
    assert rc >= 0, K.lib().lb_last_error().decode()


def weights(rng, fmt, n, k, asym=False):
    w = rng.standard_normal((n, k)).astype(np.float32)
    hw = F.quantize_mxfp4(w) if fmt == "mxfp4" else F.quantize_int4(w, asym=asym)
    return hw, K.to_device(hw)


def plain(fmt, dw, x_dev, y_dev, m=1):
    """y = x . w^T through the unfused small-M entry points."""
    L, prm = K.lib(), K._Params(K.ISA_GFX950, 0, 0, 0, 0, 0, 0)
    if fmt == "mxfp4":
        rc = L.lbd_gemm_mxfp4(x_dev, m, dw.kp, dw.qw.ptr, dw.e8m0.ptr, dw.n, y_dev, C.byref(prm), None)
    else:
        zp = None if dw.zeros is None else dw.zeros.ptr
        if fmt == "w4a16":
            rc = L.lbd_gemm_w4a16(x_dev, m, dw.kp, dw.qw.ptr, dw.scales.ptr, zp, dw.n, y_dev, C.byref(prm), None)
        else:
            rc = L.lbd_gemm_w4a8(x_dev, m, dw.kp, dw.qw.ptr, dw.scales.ptr, zp, dw.n, y_dev, C.byref(prm), None,
                                 0, None)
    assert rc == K.ISA_GFX950, K.lib().lb_last_error().decode()


def fused(fmt, dw, x_dev, y_dev, m=1, norm=None, eps=0.0, swiglu=False, bias=None, res=None, key=None,
          glu=False):
    L = K.lib()
    f = K.LbdFusion(norm, eps, int(swiglu), bias, res, key, int(glu))
    if fmt == "mxfp4":
        return L.lbd_gemv_mxfp4_fused(x_dev, m, dw.kp, dw.qw.ptr, dw.e8m0.ptr, dw.n, y_dev, C.byref(f), None)
    zp = None if dw.zeros is None else dw.zeros.ptr
    fn = L.lbd_gemv_w4a16_fused if fmt == "w4a16" else L.lbd_gemv_w4a8_fused
    return fn(x_dev, m, dw.kp, dw.qw.ptr, dw.scales.ptr, zp, dw.n, y_dev, C.byref(f), None)


def dense(hw):
    if isinstance(hw, F.MXFP4Weights):
        return O.dequant_mxfp4(hw.qw, hw.e8m0)
    return O.dequant_int4(hw.qw, hw.scales, hw.zeros)


def run_plain(fmt, dw, act, n):
    """The unfused GEMV of `act`. W4A16 / MXFP4 rows past 4096 elements take the
    split one-row kernel there, which adds its slices' sums in another order than
    the fused kernels sum a row, so for them the same small-M kernel runs without
    the prologue (a zero bias keeps the launch off the one-row kernels; adding +0
    changes no value)."""
    y = K.DeviceBuffer(4 * n)
    _LIVE.append(y)
    x_dev = up(act.astype(np.float32)).ptr
    if fmt != "w4a8" and dw.kp > 4096:
        ok(fused(fmt, dw, x_dev, y.ptr, bias=up(np.zeros(n, np.float32)).ptr))
    else:
        plain(fmt, dw, x_dev, y.ptr)
    return y.to_array((n,), np.float32)


# ---------------------------------------------------------------- prologues

@pytest.mark.parametrize("fmt", FORMATS)
@pytest.mark.parametrize("n,k", [(1152, 896), (300, 4864), (77, 128), (4096, 4096), (9, 11008)])
def test_norm_prologue_exact_rows(rng, fmt, n, k):
    """|x| = 2^e everywhere and eps = 0: the norm is exactly sign(x) * norm_w."""
    hw, dw = weights(rng, fmt, n, k, asym=(fmt == "w4a8"))
    x = (np.sign(rng.standard_normal(k)) * 2.0 ** rng.integers(-6, 6)).astype(np.float32)
    nw = rng.standard_normal(k).astype(np.float32)
    y = K.DeviceBuffer(4 * n)
    ok(fused(fmt, dw, up(x).ptr, y.ptr, norm=up(nw).ptr, eps=0.0))
    np.testing.assert_array_equal(y.to_array((n,), np.float32), run_plain(fmt, dw, np.sign(x) * nw, n))


@pytest.mark.parametrize("fmt", FORMATS)
@pytest.mark.parametrize("n,k", [(896, 4864), (64, 384), (33, 11008)])
def test_swiglu_prologue_exact_rows(rng, fmt, n, k):
    """gate in {0, 64, 100, 2^20}: silu(gate) == gate in float32; up = j / 64."""
    hw, dw = weights(rng, fmt, n, k)
    g = rng.choice(np.array([0.0, 64.0, 100.0, 2.0 ** 20], np.float32), k)
    u = (rng.integers(-64, 64, k) / 64.0).astype(np.float32)
    y = K.DeviceBuffer(4 * n)
    ok(fused(fmt, dw, up(np.concatenate([g, u])).ptr, y.ptr, swiglu=True))
    np.testing.assert_array_equal(y.to_array((n,), np.float32), run_plain(fmt, dw, g * u, n))


@pytest.mark.parametrize("fmt", ["w4a16", "mxfp4"])
@pytest.mark.parametrize("n,k", [(1152, 896), (151, 4864)])
def test_prologues_random_rows_within_bound(rng, fmt, n, k):
    hw, dw = weights(rng, fmt, n, k)
    W = dense(hw)
    x = (rng.standard_normal(k) * 7).astype(np.float32)
    nw = (1 + 0.05 * rng.standard_normal(k)).astype(np.float32)
    y = K.DeviceBuffer(4 * n)
    ok(fused(fmt, dw, up(x).ptr, y.ptr, norm=up(nw).ptr, eps=1e-6))
    act = MR.rms_norm(x[None].astype(np.float64), nw.astype(np.float64), 1e-6)
    O.assert_fp_close(y.to_array((1, n), np.float32), act @ W.T, O.fp_bound(act, W))
    gu = (rng.standard_normal(2 * k) * 4).astype(np.float32)
    ok(fused(fmt, dw, up(gu).ptr, y.ptr, swiglu=True))
    g, u = gu[:k].astype(np.float64), gu[k:].astype(np.float64)
    act = (g / (1 + np.exp(-g)) * u)[None]
    O.assert_fp_close(y.to_array((1, n), np.float32), act @ W.T, O.fp_bound(act, W))


# ---------------------------------------------------------------- epilogue

@pytest.mark.parametrize("fmt", FORMATS)
@pytest.mark.parametrize("m", [1, 3])
def test_bias_and_residual_in_place(rng, fmt, m):
    n, k = 700, 896
    hw, dw = weights(rng, fmt, n, k, asym=True)
    x = rng.standard_normal((m, k)).astype(np.float32)
    b = rng.standard_normal(n).astype(np.float32)
    r = rng.standard_normal((m, n)).astype(np.float32)
    dx = up(x)
    yp = K.DeviceBuffer(4 * m * n)
    plain(fmt, dw, dx.ptr, yp.ptr, m)
    y0 = yp.to_array((m, n), np.float32)
    dr = up(r)  # residual and output are the same buffer
    ok(fused(fmt, dw, dx.ptr, dr.ptr, m, bias=up(b).ptr, res=dr.ptr))
    np.testing.assert_array_equal(dr.to_array((m, n), np.float32), r + (y0 + b))
    dy = K.DeviceBuffer(4 * m * n)
    ok(fused(fmt, dw, dx.ptr, dy.ptr, m, res=up(r).ptr))
    np.testing.assert_array_equal(dy.to_array((m, n), np.float32), r + y0)


@pytest.mark.parametrize("fmt", FORMATS)
@pytest.mark.parametrize("m,n,k", [(1, 9728, 896), (1, 600, 4864), (2, 600, 4864), (1, 154, 11008),
                                   (4, 2000, 128), (1, 2, 256), (3, 9728, 896)])
def test_glu_epilogue(rng, fmt, m, n, k):
    """(gate, up) row pairs: the glu epilogue equals the plain fused GEMV followed by
    lbd_swiglu_pairs bit for bit (same rows, same sums, the SwiGLU kernel's
    expression), with the RMSNorm prologue and a bias too; shapes cover one, two
    and four rows per batch (one row: the gate is carried across batches) and the
    2-8 pair shares of the persistent grid. W4A16 / MXFP4 also held to the float64
    oracle's bound on silu(g) * u."""
    hw, dw = weights(rng, fmt, n, k, asym=(fmt == "w4a8"))
    x = (rng.standard_normal((m, k)) * 3).astype(np.float32)
    b = rng.standard_normal(n).astype(np.float32)
    dx, db = up(x), up(b)
    L = K.lib()
    yp, ref, yg = K.DeviceBuffer(4 * m * n), K.DeviceBuffer(4 * m * n // 2), K.DeviceBuffer(4 * m * n // 2)
    _LIVE.extend([yp, ref, yg])
    # a plain one-row launch of W4A16 / MXFP4 rows past 4096 elements takes the split
    # kernel (its slices' sums added in another order), so a zero bias stands in for
    # "no fusion" there (see run_plain)
    split = m == 1 and fmt != "w4a8" and dw.kp > 4096
    cases = [dict(bias=up(np.zeros(n, np.float32)).ptr) if split else dict(), dict(bias=db.ptr)]
    if m == 1:
        nw = up((1 + 0.05 * rng.standard_normal(k)).astype(np.float32))
        cases.append(dict(norm=nw.ptr, eps=1e-6, bias=db.ptr))
    for kw in cases:
        ok(fused(fmt, dw, dx.ptr, yp.ptr, m, **kw))
        ok(L.lbd_swiglu_pairs(yp.ptr, m, n // 2, ref.ptr, None))
        ok(fused(fmt, dw, dx.ptr, yg.ptr, m, glu=True, **kw))
        np.testing.assert_array_equal(yg.to_array((m, n // 2), np.float32), ref.to_array((m, n // 2), np.float32))
    if fmt != "w4a8":
        ok(fused(fmt, dw, dx.ptr, yg.ptr, m, glu=True))
        t = x.astype(np.float64) @ dense(hw).T
        g, u = t[:, 0::2], t[:, 1::2]
        with np.errstate(over="ignore"):  # exp(-g) = inf for very negative g: s = 0
            s = 1 / (1 + np.exp(-g))
        # |d(silu(g) u)| <= |u| (|s| + |g| s (1 - s)) |dg| + |silu(g)| |du|, dg and du
        # within the GEMM bound of their rows; plus the float32 rounding of the product
        bnd = 1e-5 * O.fp_bound(x.astype(np.float64), dense(hw))
        tol = np.abs(u) * (s + np.abs(g) * s * (1 - s)) * bnd[:, 0::2] + np.abs(g * s) * bnd[:, 1::2]
        want = g * s * u
        got = yg.to_array((m, n // 2), np.float32).astype(np.float64)
        assert np.all(np.abs(got - want) <= tol + 4 * np.finfo(np.float32).eps * np.abs(want) + 1e-30)


def test_fused_argument_checks(rng):
    hw, dw = weights(rng, "w4a16", 64, 256)
    x, y, nw = up(np.zeros(512, np.float32)), K.DeviceBuffer(4 * 64 * 4), up(np.ones(256, np.float32))
    assert fused("w4a16", dw, x.ptr, y.ptr, norm=nw.ptr, swiglu=True) == -6   # two prologues
    assert fused("w4a16", dw, x.ptr, y.ptr, m=2, norm=nw.ptr) == -6           # prologue needs M == 1
    key = up(np.zeros(1024, np.uint64))
    assert fused("w4a16", dw, x.ptr, y.ptr, m=2, key=key.ptr) == -6           # argmax needs M == 1
    assert fused("w4a16", dw, x.ptr, y.ptr, m=5) == -1                        # small-M kernels only
    assert fused("w4a16", dw, x.ptr, y.ptr, glu=True, res=y.ptr) == -6         # glu excludes the residual
    assert fused("w4a16", dw, x.ptr, y.ptr, glu=True, key=key.ptr) == -6       # ... and the argmax key
    hw3, dw3 = weights(rng, "w4a16", 63, 256)
    assert fused("w4a16", dw3, x.ptr, y.ptr, glu=True) == -1                   # glu takes row pairs
    assert fused("w4a16", dw, x.ptr, y.ptr, m=2, glu=True) == K.ISA_GFX950
    assert fused("w4a16", dw, x.ptr, y.ptr, m=1) == K.ISA_GFX950


# ---------------------------------------------------------------- argmax key

@pytest.mark.parametrize("fmt", FORMATS)
def test_argmax_key_matches_numpy(rng, fmt):
    n, k = 50000, 896
    w = rng.standard_normal((n, k)).astype(np.float32)
    x = rng.standard_normal(k).astype(np.float32)
    # identical rows along x: identical logits far above the others; the first wins
    w[[30000, 777, 45000]] = x * 0.5
    hw = F.quantize_mxfp4(w) if fmt == "mxfp4" else F.quantize_int4(w)
    dw = K.to_device(hw)
    y = K.DeviceBuffer(4 * n)
    key = up(np.zeros(1024, np.uint64))
    tok, pos, hist = up(np.zeros(1, np.int32)), up(np.array([6], np.int32)), up(np.full(10, -1, np.int32))
    L = K.lib()
    for trial in range(2):  # the finalize clears the key, so a second step starts clean
        ok(fused(fmt, dw, up(x).ptr, y.ptr, key=key.ptr))
        yv = y.to_array((n,), np.float32)
        ok(L.lbd_argmax_finalize(key.ptr, tok.ptr, pos.ptr, 1, hist.ptr, 10, None))
        assert tok.to_array((1,), np.int32)[0] == int(np.argmax(yv))
        assert not key.to_array((1024,), np.uint64).any()
    assert int(np.argmax(yv)) == 777 and yv[777] == yv[30000] == yv[45000]
    assert pos.to_array((1,), np.int32)[0] == 8
    np.testing.assert_array_equal(hist.to_array((10,), np.int32)[6:9], [-1, np.argmax(yv), np.argmax(yv)])


def test_argmax_key_nan_and_negative_logits(rng):
    n, k = 3000, 256
    w = rng.standard_normal((n, k)).astype(np.float32)
    hw = F.quantize_int4(w)
    hw.scales[[2100, 1500]] = np.nan  # NaN logits: numpy's argmax returns the first NaN
    dw = K.to_device(hw)
    x = rng.standard_normal(k).astype(np.float32)
    y, key, tok = K.DeviceBuffer(4 * n), up(np.zeros(1024, np.uint64)), up(np.zeros(1, np.int32))
    L = K.lib()
    ok(fused("w4a16", dw, up(x).ptr, y.ptr, key=key.ptr))
    ok(L.lbd_argmax_finalize(key.ptr, tok.ptr, None, 1, None, 0, None))
    yv = y.to_array((n,), np.float32)
    assert np.isnan(yv[1500]) and tok.to_array((1,), np.int32)[0] == 1500 == int(np.argmax(yv))
    # all logits negative (bias far below zero): the largest still wins
    hw2 = F.quantize_int4(w)
    dw2 = K.to_device(hw2)
    b = np.full(n, -1e6, np.float32)
    ok(fused("w4a16", dw2, up(x).ptr, y.ptr, bias=up(b).ptr, key=key.ptr))
    ok(L.lbd_argmax_finalize(key.ptr, tok.ptr, None, 1, None, 0, None))
    yv = y.to_array((n,), np.float32)
    assert yv.max() < 0 and tok.to_array((1,), np.int32)[0] == int(np.argmax(yv))


# ---------------------------------------------------------------- one-token attention

def attention_one(qkv, kc, vc, p, H, KV, D, cos, sin):
    """float64: rotate q and k at position p, attend over cache keys 0..p-1 plus the
    new key (keys 0..cap-1 from the cache when p >= cap)."""
    cap = kc.shape[1]
    x = qkv.astype(np.float64)
    pc = min(p, cos.shape[0] - 1)
    c, s = cos[pc:pc + 1].astype(np.float64), sin[pc:pc + 1].astype(np.float64)
    q = MR.rotate(x[:H * D].reshape(1, H, D), c, s)[0]
    k = MR.rotate(x[H * D:(H + KV) * D].reshape(1, KV, D), c, s)[0]
    v = x[(H + KV) * D:].reshape(KV, D)
    K_, V_ = kc.astype(np.float64).copy(), vc.astype(np.float64).copy()
    if p < cap:
        K_[:, p], V_[:, p] = k, v
    S = min(p + 1, cap)
    out = np.zeros((H, D))
    for h in range(H):
        g = h // (H // KV)
        sc = K_[g, :S] @ q[h] / np.sqrt(D)
        e = np.exp(sc - sc.max())
        out[h] = (e / e.sum()) @ V_[g, :S]
    return out.reshape(-1), k, v


# one round, several, a small position in a large cache, p >= cap; from cap = 1024
# the workspace entry point takes key slices (one, several, several rounds each at
# p = 15999: 250 rounds over 32 slices)
@pytest.mark.parametrize("D,H,KV,p,cap", [(64, 14, 2, 0, 8), (64, 14, 2, 191, 192), (64, 14, 2, 255, 300),
                                          (64, 14, 2, 256, 300), (32, 8, 1, 37, 64), (128, 4, 4, 700, 1000),
                                          (64, 16, 1, 5, 16), (64, 2, 2, 20, 20), (64, 14, 2, 15999, 16000),
                                          (64, 14, 2, 70, 16000), (32, 8, 2, 300, 301), (128, 8, 8, 4000, 4000),
                                          (64, 14, 2, 1023, 1024), (64, 14, 2, 40, 1024), (32, 16, 4, 5000, 5000),
                                          (128, 14, 2, 2100, 3000)])
@pytest.mark.parametrize("ws", [False, True])
def test_attention_decode(rng, D, H, KV, p, cap, ws):
    """ws: lbd_attention_decode_ws with a workspace, i.e. key slices on many
    workgroups and a merge launch for caches of 1024 positions and more."""
    L = K.lib()
    width = (H + 2 * KV) * D
    qkv = rng.standard_normal(width).astype(np.float32)
    kc0 = rng.standard_normal((KV, cap, D)).astype(np.float32)
    vc0 = rng.standard_normal((KV, cap, D)).astype(np.float32)
    max_pos = 16384
    cos, sin = DM.rope_tables(D, max_pos, 10000.0)
    dk, dv, out = up(kc0), up(vc0), K.DeviceBuffer(4 * H * D)
    dcos, dsin, dpos = up(cos), up(sin), up(np.array([p], np.int32))
    if ws:
        work = K.DeviceBuffer(L.lbd_attention_decode_work_bytes(H, D, cap))
        _LIVE.append(work)
        ok(L.lbd_attention_decode_ws(up(qkv).ptr, H, KV, D, dcos.ptr, dsin.ptr, dpos.ptr, max_pos, dk.ptr, dv.ptr,
                                     cap, out.ptr, work.ptr, work.nbytes, None))
    else:
        ok(L.lbd_attention_decode(up(qkv).ptr, H, KV, D, dcos.ptr, dsin.ptr, dpos.ptr, max_pos, dk.ptr, dv.ptr, cap,
                                  out.ptr, None))
    ref, k, v = attention_one(qkv, kc0, vc0, p, H, KV, D, cos, sin)
    got = out.to_array((H * D,), np.float32)
    assert np.abs(got - ref).max() <= 2e-5 * max(np.abs(vc0).max(), np.abs(v).max())
    kc, vc = dk.to_array(kc0.shape, np.float32), dv.to_array(vc0.shape, np.float32)
    if p < cap:
        # the cache row is what lbd_qkv_rope writes for the same q / k / v row (both
        # round each product of the rotation, as numpy's float32 does)
        rk, rv = up(kc0), up(vc0)
        ok(L.lbd_qkv_rope(up(qkv[None]).ptr, None, 1, H, KV, D, dcos.ptr, dsin.ptr, dpos.ptr, max_pos, rk.ptr,
                          rv.ptr, cap, None))
        np.testing.assert_array_equal(kc[:, p], rk.to_array(kc0.shape, np.float32)[:, p])
        np.testing.assert_array_equal(vc[:, p], rv.to_array(vc0.shape, np.float32)[:, p])
        np.testing.assert_allclose(kc[:, p], k, rtol=0, atol=1e-5)
    others = np.ones(cap, bool)
    if p < cap:
        others[p] = False
    np.testing.assert_array_equal(kc[:, others], kc0[:, others])
    np.testing.assert_array_equal(vc[:, others], vc0[:, others])


@pytest.mark.parametrize("cap", [600, 2000])
def test_attention_decode_consecutive_positions(rng, cap):
    """A run of decode positions on one cache (as the decoder's graph replays it),
    through the workspace entry point (key slices from cap = 1024): every step
    matches the float64 attention, and each step's cache row is there for the next."""
    L = K.lib()
    D, H, KV = 64, 14, 2
    max_pos = 2048
    work = K.DeviceBuffer(L.lbd_attention_decode_work_bytes(H, D, cap))
    _LIVE.append(work)
    cos, sin = DM.rope_tables(D, max_pos, 10000.0)
    kc = rng.standard_normal((KV, cap, D)).astype(np.float32)
    vc = rng.standard_normal((KV, cap, D)).astype(np.float32)
    dk, dv, out = up(kc), up(vc), K.DeviceBuffer(4 * H * D)
    _LIVE.append(out)
    dcos, dsin = up(cos), up(sin)
    for p in (0, 1, 63, 64, 65, 255, 256, 300, 599, cap - 1, cap + 5):
        qkv = rng.standard_normal((H + 2 * KV) * D).astype(np.float32)
        ok(L.lbd_attention_decode_ws(up(qkv).ptr, H, KV, D, dcos.ptr, dsin.ptr, up(np.array([p], np.int32)).ptr,
                                     max_pos, dk.ptr, dv.ptr, cap, out.ptr, work.ptr, work.nbytes, None))
        ref, k, v = attention_one(qkv, kc, vc, p, H, KV, D, cos, sin)
        got = out.to_array((H * D,), np.float32)
        assert np.abs(got - ref).max() <= 2e-5 * max(np.abs(vc).max(), np.abs(v).max()), p
        kc, vc = dk.to_array(kc.shape, np.float32), dv.to_array(vc.shape, np.float32)


# slices 1, 3, 4 (all active), 8 with 2 active, 8 with p >= cap, 7 at D = 128, 2 at D = 32
@pytest.mark.parametrize("D,H,KV,p,cap", [(64, 14, 2, 30, 64), (64, 14, 2, 150, 193), (64, 14, 2, 255, 256),
                                          (64, 14, 2, 100, 512), (64, 14, 2, 600, 512), (128, 8, 2, 200, 224),
                                          (32, 16, 4, 200, 256)])
def test_attention_slices_merge_and_fused_prologue(rng, D, H, KV, p, cap):
    """lbd_attention_slices + lbd_attention_merge against the float64 attention, and
    the fused o projection whose prologue merges the same partials equal to the
    merge kernel's output followed by the plain fused GEMV, bit for bit."""
    L = K.lib()
    qkv = rng.standard_normal((H + 2 * KV) * D).astype(np.float32)
    kc0 = rng.standard_normal((KV, cap, D)).astype(np.float32)
    vc0 = rng.standard_normal((KV, cap, D)).astype(np.float32)
    max_pos = 1024
    cos, sin = DM.rope_tables(D, max_pos, 10000.0)
    dk, dv = up(kc0), up(vc0)
    dcos, dsin, dpos = up(cos), up(sin), up(np.array([p], np.int32))
    part = K.DeviceBuffer(L.lbd_attention_decode_work_bytes(H, D, cap))
    out = K.DeviceBuffer(4 * H * D)
    _LIVE.extend([part, out])
    ok(L.lbd_attention_slices(up(qkv).ptr, H, KV, D, dcos.ptr, dsin.ptr, dpos.ptr, max_pos, dk.ptr, dv.ptr, cap,
                              part.ptr, part.nbytes, None))
    ok(L.lbd_attention_merge(part.ptr, part.nbytes, H, D, dpos.ptr, cap, out.ptr, None))
    assert L.lbd_attention_merge(part.ptr, part.nbytes - 16, H, D, dpos.ptr, cap, out.ptr, None) == -6
    ref, k, v = attention_one(qkv, kc0, vc0, p, H, KV, D, cos, sin)
    att = out.to_array((H * D,), np.float32)
    assert np.abs(att - ref).max() <= 2e-5 * max(np.abs(vc0).max(), np.abs(v).max())
    if p < cap:
        np.testing.assert_allclose(dk.to_array(kc0.shape, np.float32)[:, p], k, rtol=0, atol=1e-5)
    n = 300
    r = rng.standard_normal(n).astype(np.float32)
    for fmt in FORMATS:
        hw, dw = weights(rng, fmt, n, H * D, asym=(fmt == "w4a8"))
        y_ref, y_fz = up(r), up(r)
        ok(fused(fmt, dw, out.ptr, y_ref.ptr, res=y_ref.ptr))
        f = K.LbdFusion(None, 0.0, 0, None, y_fz.ptr, None, 0, part.ptr, cap, D)
        if fmt == "mxfp4":
            ok(L.lbd_gemv_mxfp4_fused(None, 1, dw.kp, dw.qw.ptr, dw.e8m0.ptr, n, y_fz.ptr, C.byref(f), None))
        else:
            fn = L.lbd_gemv_w4a16_fused if fmt == "w4a16" else L.lbd_gemv_w4a8_fused
            zp = None if dw.zeros is None else dw.zeros.ptr
            ok(fn(None, 1, dw.kp, dw.qw.ptr, dw.scales.ptr, zp, n, y_fz.ptr, C.byref(f), None))
        np.testing.assert_array_equal(y_fz.to_array((n,), np.float32), y_ref.to_array((n,), np.float32))


def test_attention_merge_prologue_argument_checks(rng):
    L = K.lib()
    hw, dw = weights(rng, "w4a16", 64, 896)
    part, y = up(np.zeros(1 << 16, np.float32)), K.DeviceBuffer(4 * 64 * 2)
    _LIVE.append(y)
    nw = up(np.ones(896, np.float32))

    def call(m=1, cap=193, d=64, norm=None):
        f = K.LbdFusion(norm, 0.0, 0, None, None, None, 0, part.ptr, cap, d)
        return L.lbd_gemv_w4a16_fused(None, m, dw.kp, dw.qw.ptr, dw.scales.ptr, None, 64, y.ptr, C.byref(f), None)
    assert call() == K.ISA_GFX950
    assert call(m=2) == -6                 # one activation row
    assert call(norm=nw.ptr) == -6         # one prologue
    assert call(cap=513) == -1             # nine slices of 64 keys
    assert call(d=48) == -1                # head_dim
    assert call(d=128, cap=257) == -1      # nine slices of 32 keys


def test_attention_decode_argument_checks():
    L = K.lib()
    b = up(np.zeros(4096, np.float32))
    pos = up(np.zeros(1, np.int32))
    args = lambda H, KV, D, cap: (b.ptr, H, KV, D, b.ptr, b.ptr, pos.ptr, 8, b.ptr, b.ptr, cap, b.ptr, None)  # noqa
    assert L.lbd_attention_decode(*args(34, 2, 64, 8)) == -1   # 17 query heads per KV head
    assert L.lbd_attention_decode(*args(14, 3, 64, 8)) == -1   # H % KV
    assert L.lbd_attention_decode(*args(14, 2, 48, 8)) == -1   # head_dim
    assert L.lbd_attention_decode(*args(14, 2, 64, 16001)) == -1
    assert L.lbd_attention_decode(*args(14, 2, 64, 8)) == 0
    wb = L.lbd_attention_decode_work_bytes(14, 64, 2048)
    w = up(np.zeros(wb // 4, np.float32))
    assert L.lbd_attention_decode_ws(b.ptr, 14, 2, 64, b.ptr, b.ptr, pos.ptr, 8, w.ptr, w.ptr, 2048, b.ptr, w.ptr,
                                     wb - 16, None) == -6   # workspace too small


# ---------------------------------------------------------------- the model: fused = unfused

@pytest.mark.parametrize("backend", ["w4a8", "mxfp4"])
def test_fused_decode_long_prompt(backend):
    """Decode steps after a 200-token prompt (cache of 210: four key slices merged in
    the o projection's prologue, three of them in use) against the unfused step."""
    cfg = DM.qwen2_config(num_layers=2, vocab_size=4096, max_position=512)
    W = DM.random_weights(cfg, seed=3)
    toks = np.random.default_rng(9).integers(0, cfg.vocab_size, 205)
    out = {}
    for fz in (True, False):
        m = DM.Model(cfg, W, backend, fused=fz)
        c = m.new_cache(210)
        assert c.fused_merge
        m.forward(toks[:200], c)
        out[fz] = np.stack([m.forward([t], c) for t in toks[200:]])
    scale = np.abs(out[False]).max()
    assert np.abs(out[True] - out[False]).max() <= 1e-4 * scale
    assert (out[True].argmax(-1) == out[False].argmax(-1)).all()


@pytest.mark.parametrize("backend", ["w4a16", "w4a8", "mxfp4"])
def test_fused_decode_matches_unfused_and_oracle(backend):
    cfg = DM.qwen2_config(num_layers=2, vocab_size=4096, max_position=512)
    W = DM.random_weights(cfg, seed=11)
    toks = np.random.default_rng(5).integers(0, cfg.vocab_size, 24)
    ref_model = MR.RefModel(cfg, W, backend, F.quantize_mxfp4 if backend == "mxfp4" else F.quantize_int4)
    out = {}
    for fz in (True, False):
        m = DM.Model(cfg, W, backend, fused=fz)
        assert m.fused == fz
        c = m.new_cache(32)
        m.forward(toks[:16], c)
        out[fz] = np.stack([m.forward([t], c) for t in toks[16:]])
        r, flips = MR.rel_with_flips(ref_model, toks, out[fz], slice(16, None), 1e-5)
        print(f"[{backend} fused={fz}] rel {r:.3g} flips {flips}")
        assert r < 1e-5
    g = {fz: DM.Model(cfg, W, backend, fused=fz).generate(toks[:8], 6) for fz in (True, False)}
    assert g[True] == g[False] == ref_model.generate(list(toks[:8]), 6)
