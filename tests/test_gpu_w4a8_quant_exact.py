"""Bit-exact pins of the int8 activation quantizers that run inside W4A8 calls.

The reference quantizes every W4A8 call's activations with one function,
lb_quant_act_int8 (src/lowbit/csrc/dispatch.c:231-257, called at :281), and pins
it bit for bit against numpy (tests/test_kernels.py:122-131). This build runs
that quantizer in several places, each of which must give the same bytes:

* M = 1, the paced one-row GEMV: the quantizer fused into the kernel, with the
  token scale from lbk::div127 instead of an IEEE division;
* M = 2..4 and the decoder's fused GEMVs (RMSNorm, SwiGLU and attention-merge
  prologues, residual epilogue): the quantizer fused into gemv_kernel;
* M >= 5: quant_rows_kernel writing the tiled layout of the int8 MFMA GEMM.

The one-row and small-M kernels have a twin that takes codes, token scales and
group sums from memory (W4A8Q) and then runs the same arithmetic. So
gemm_w4a8(x) must equal gemm_w4a8_q(oracle codes of x) bit for bit there; a single
activation code off by one changes the exact int32 group accumulator of every
weight row whose code at that position differs from its zero-point, and so that
row's output (test_planted_code_error_is_seen shows the comparison sees one). For
M >= 5 the tiled codes, scales and group sums the quantizer left in the caller's
workspace are read back and compared with the oracle's directly.

The activation rows are built to land exactly on, and 1-3 ulps beside, the .5 ties
of x / scale at row maxima from 2^-140 (scales below the float32 normal range, where
1 / scale overflows) to 2^125, plus zero rows. The oracle is oracle/reference.py's
quant_act_int8, itself pinned against the reference's C library and its golden
vectors (tests/test_oracle.py).
"""
import ctypes as C

import numpy as np
import pytest

from lowbit_amd import formats as F
from lowbit_amd import kernels as K
from lowbit_amd import model as DM
from oracle import reference as O

pytestmark = pytest.mark.gpu

MANTS = np.array([1.0, 1.5, 1.25, 1.9375, 1.0 + 1.0 / 64], np.float64)
EXPS = [-140, -135, -129, -127, -126, -100, -60, -20, -8, -1, 0, 3, 10, 40, 90, 117]
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


def tie_row(rng, k, e, mant=None):
    """One row of k float32 values whose amax is 127 * mant * 2^e, so that the token
    scale amax / 127 is exactly mant * 2^e. About half the elements are exact ties
    (j + 1/2) * scale, a quarter sit 1-3 ulps beside one, the rest are exact
    multiples of the scale or uniform in [-amax, amax]."""
    mant = float(rng.choice(MANTS)) if mant is None else mant
    sc = np.ldexp(mant, e)
    amax = np.float32(127.0 * sc)
    assert float(amax) == 127.0 * sc and np.float32(amax / np.float32(127.0)) == np.float32(sc)
    t = rng.integers(-127, 127, k) + 0.5                     # ties -126.5 .. 126.5
    x = (t * sc).astype(np.float32)
    assert np.all(x.astype(np.float64) == t * sc)           # exactly representable
    kind = rng.random(k)
    near = (kind >= 0.5) & (kind < 0.75)
    steps = rng.integers(1, 4, k) * rng.choice([-1, 1], k)
    xn = x.copy()
    for s in (1, 2, 3):
        sel = near & (np.abs(steps) >= s)
        xn[sel] = np.nextafter(xn[sel], np.where(steps[sel] > 0, np.inf, -np.inf).astype(np.float32))
    x = np.where(near, xn, x)
    mult = (kind >= 0.75) & (kind < 0.87)
    x = np.where(mult, (rng.integers(-127, 128, k) * sc).astype(np.float32), x)
    unif = kind >= 0.87
    x = np.where(unif, (rng.uniform(-1, 1, k) * float(amax)).astype(np.float32), x)
    x = np.clip(x, -amax, amax)
    x[rng.integers(k)] = amax if rng.random() < 0.5 else -amax
    return x.astype(np.float32)


def random_scale_row(rng, k, e):
    """A row with a random amax in [2^e, 2^(e+1)) (a scale with a full mantissa):
    candidates fl((j + 1/2) * scale) and their neighbours within 3 ulps, some of
    which are exact ties of fl(x / scale)."""
    amax = np.float32(np.ldexp(1.0 + rng.random(), e))
    sc = np.float32(amax / np.float32(127.0))
    t = (rng.integers(-127, 127, k) + 0.5).astype(np.float32)
    x = t * sc
    for _ in range(3):
        move = rng.random(k) < 0.4
        x = np.where(move, np.nextafter(x, np.where(rng.random(k) < 0.5, np.inf, -np.inf).astype(np.float32)), x)
    x = np.clip(x, -amax, amax).astype(np.float32)
    x[rng.integers(k)] = amax
    return x


def exact_ties(x):
    """How many elements of the rows are exact .5 ties of fl(x / scale)."""
    x = np.atleast_2d(x)
    _, xs, _ = O.quant_act_int8(x)
    v = np.divide(x, xs[:, None], dtype=np.float32)
    return int(np.count_nonzero(v - np.floor(v) == 0.5))


def rows(rng, m, k, exps):
    out = []
    for i in range(m):
        e = exps[i % len(exps)]
        if i % 7 == 3:
            out.append(np.zeros(k, np.float32))
        elif i % 5 == 4 and -120 < e < 120:
            out.append(random_scale_row(rng, k, e))
        else:
            out.append(tie_row(rng, k, e))
    return np.stack(out)


def int4(rng, n, k, asym):
    w = rng.standard_normal((n, k)).astype(np.float32)
    return F.quantize_int4(w, asym=asym)


def q_call(W, xq, xs, asum, m, dW=None):
    """gemm_w4a8_q on device copies of the oracle's codes (lbd_gemm_w4a8_q)."""
    dW = dW or K.to_device(W)
    L = K.lib()
    y = K.DeviceBuffer(4 * m * W.n)
    _LIVE.append(y)
    prm = K._Params(0, 0, 0, 0, 0, 0, 0)
    zp = None if dW.zeros is None else dW.zeros.ptr
    ok(L.lbd_gemm_w4a8_q(up(xq).ptr, up(xs).ptr, up(asum.astype(np.int32)).ptr, m, W.kp, dW.qw.ptr, dW.scales.ptr,
                         zp, W.n, y.ptr, C.byref(prm), None))
    ok(L.lb_stream_synchronize(None))
    return y.to_array((m, W.n), np.float32)


def x_call(W, x, dW, ws=True):
    """gemm_w4a8 on fp32 activations (lbd_gemm_w4a8, row-major weights)."""
    L = K.lib()
    m = x.shape[0]
    y = K.DeviceBuffer(4 * m * W.n)
    _LIVE.append(y)
    prm = K._Params(0, 0, 0, 0, 0, 0, 0)
    zp = None if dW.zeros is None else dW.zeros.ptr
    wsb = K.DeviceBuffer(L.lbd_w4a8_workspace_bytes(m, W.kp)) if ws else None
    if wsb:
        _LIVE.append(wsb)
    ok(L.lbd_gemm_w4a8(up(F.pad_acts(x, W.kp)).ptr, m, W.kp, dW.qw.ptr, dW.scales.ptr, zp, W.n, y.ptr,
                       C.byref(prm), wsb.ptr if wsb else None, wsb.nbytes if wsb else 0, None))
    ok(L.lb_stream_synchronize(None))
    return y.to_array((m, W.n), np.float32), wsb


# ---------------------------------------------------------------- the division by 127

def test_div127_on_device_equals_ieee_division_for_every_input():
    """The paced kernel's token scale amax / 127 (lbk::div127) as this GPU computes
    it, against this GPU's IEEE division, for all 2^31 - 2^23 + 1 non-negative finite
    float32 values and +inf (the host twin is tests/test_div127.py)."""
    out = K.DeviceBuffer(8)
    _LIVE.append(out)
    ok(K.lib().lbd_probe_div127(out.ptr, None))
    ok(K.lib().lb_stream_synchronize(None))
    bad, first = out.to_array((2,), np.uint32)
    assert bad == 0, f"{bad} inputs differ, first bit pattern {first:#010x}"
    assert first == 0xFFFFFFFF


# ---------------------------------------------------------------- M = 1: the paced kernel

@pytest.mark.parametrize("n,k,asym", [(11008, 4096, True), (11008, 4096, False), (4096, 11008, True),
                                      (4096, 4096, True), (1000, 4000, True)])
def test_paced_one_row_quantizer_bit_exact(rng, n, k, asym):
    W = int4(rng, n, k, asym)
    dW = K.to_device(W)
    plan = K.gemm_plan("w4a8", 1, n, W.kp)
    assert plan["path"] == "gfx950" and plan["act_rows"] == 1
    ties = 0
    for e in EXPS:
        for maker in (tie_row, random_scale_row):
            if maker is random_scale_row and not -120 < e < 120:
                continue
            x = maker(rng, k, e)[None]
            ties += exact_ties(x)
            xq, xs, asum = O.quant_act_int8(x, W.kp)
            y, _ = x_call(W, x, dW)
            np.testing.assert_array_equal(y, q_call(W, xq, xs, asum, 1, dW), err_msg=f"row amax 2^{e}")
    x = np.zeros((1, k), np.float32)
    xq, xs, asum = O.quant_act_int8(x, W.kp)
    y, _ = x_call(W, x, dW)
    np.testing.assert_array_equal(y, q_call(W, xq, xs, asum, 1, dW))
    assert np.all(y == 0)
    assert ties > 5 * k  # the rows really are full of exact ties


def test_planted_code_error_is_seen(rng):
    """One oracle code moved by one (and its group sum with it) changes the output:
    the bitwise comparison above would see a quantizer that rounds one tie the wrong
    way."""
    W = int4(rng, 11008, 4096, True)
    dW = K.to_device(W)
    x = tie_row(rng, 4096, -8)[None]
    xq, xs, asum = O.quant_act_int8(x, W.kp)
    y, _ = x_call(W, x, dW)
    base = q_call(W, xq, xs, asum, 1, dW)
    np.testing.assert_array_equal(y, base)
    v = np.divide(x, xs[:, None], dtype=np.float32)
    tie = np.flatnonzero((v[0] - np.floor(v[0]) == 0.5) & (np.abs(v[0]) < 126))
    j = int(tie[0])
    bad = xq.copy()
    v0 = float(v[0, j])
    bad[0, j] = int(np.floor(v0)) if int(xq[0, j]) == int(np.ceil(v0)) else int(np.ceil(v0))  # the other rounding
    basum = asum.copy()
    basum[0, j // 128] += int(bad[0, j]) - int(xq[0, j])
    moved = q_call(W, bad, xs, basum, 1, dW)
    codes = O.unpack_codes(W.qw, 128)[:, j].astype(np.int64)
    seen = codes != W.zeros[:, j // 128]
    assert np.count_nonzero(moved[0] != y[0]) >= 0.9 * np.count_nonzero(seen)
    assert np.all(moved[0][~seen] == y[0][~seen])


# ---------------------------------------------------------------- M = 2..4: gemv_kernel

@pytest.mark.parametrize("m", [2, 3, 4])
@pytest.mark.parametrize("n,k", [(11008, 4096), (4096, 11008), (896, 4864)])
def test_small_m_quantizer_bit_exact(rng, m, n, k):
    W = int4(rng, n, k, True)
    dW = K.to_device(W)
    plan = K.gemm_plan("w4a8", m, n, W.kp)
    assert plan["path"] == "gfx950" and plan["act_rows"] == m
    ties = 0
    for start in range(0, len(EXPS), m):
        x = rows(rng, m, k, EXPS[start:start + m] + EXPS[:max(0, start + m - len(EXPS))])
        ties += exact_ties(x)
        xq, xs, asum = O.quant_act_int8(x, W.kp)
        y, _ = x_call(W, x, dW)
        np.testing.assert_array_equal(y, q_call(W, xq, xs, asum, m, dW), err_msg=f"rows from {start}")
    assert ties > 3 * k


# ---------------------------------------------------------------- decoder GEMVs with prologues

def fused_w4a8(dW, n, kp, x_dev, f):
    L = K.lib()
    y = K.DeviceBuffer(4 * n)
    _LIVE.append(y)
    zp = None if dW.zeros is None else dW.zeros.ptr
    ok(L.lbd_gemv_w4a8_fused(x_dev, 1, kp, dW.qw.ptr, dW.scales.ptr, zp, n, y.ptr, C.byref(f), None))
    ok(L.lb_stream_synchronize(None))
    return y.to_array((1, n), np.float32)


# config 5's linear shapes: qkv 1152 x 896 and gate_up 9728 x 896 behind the RMSNorm,
# the LM head's 896 columns at 4096 rows, down 896 x 4864 behind the SwiGLU
@pytest.mark.parametrize("n,k", [(1152, 896), (9728, 896), (4096, 896)])
def test_rmsnorm_prologue_quantizer_bit_exact(rng, n, k):
    """x = all ones and eps = 0: the RMSNorm is exactly 1 * norm_w, so the quantizer
    sees norm_w, which carries the ties."""
    W = int4(rng, n, k, True)
    dW = K.to_device(W)
    ones = up(np.ones(k, np.float32))
    for e in EXPS:
        act = tie_row(rng, k, e)[None]
        f = K.LbdFusion(up(act[0]).ptr, 0.0, 0, None, None, None, 0, None, 0, 0)
        y = fused_w4a8(dW, n, k, ones.ptr, f)
        xq, xs, asum = O.quant_act_int8(act, W.kp)
        np.testing.assert_array_equal(y, q_call(W, xq, xs, asum, 1, dW), err_msg=f"row amax 2^{e}")


@pytest.mark.parametrize("n,k", [(896, 4864), (300, 11008)])
def test_swiglu_prologue_quantizer_bit_exact(rng, n, k):
    """gate = 64 everywhere (silu(64) == 64 in float32) and up = act / 64: the
    prologue's product is exactly act."""
    W = int4(rng, n, k, True)
    dW = K.to_device(W)
    for e in [e for e in EXPS if -100 <= e <= 110]:
        act = tie_row(rng, k, e)[None]
        u = (act[0] / np.float32(64.0)).astype(np.float32)
        assert np.array_equal(np.float32(64.0) * u, act[0])
        f = K.LbdFusion(None, 0.0, 1, None, None, None, 0, None, 0, 0)
        y = fused_w4a8(dW, n, k, up(np.concatenate([np.full(k, 64.0, np.float32), u])).ptr, f)
        xq, xs, asum = O.quant_act_int8(act, W.kp)
        np.testing.assert_array_equal(y, q_call(W, xq, xs, asum, 1, dW), err_msg=f"row amax 2^{e}")


@pytest.mark.parametrize("n,k", [(896, 4864), (11008, 4096)])
def test_residual_epilogue_gemv_quantizer_bit_exact(rng, n, k):
    """The down projection's launch: no prologue, a residual epilogue (zero here, so
    y = 0 + x . w^T), which keeps M = 1 on gemv_kernel instead of the paced kernel."""
    W = int4(rng, n, k, True)
    dW = K.to_device(W)
    for e in EXPS:
        act = tie_row(rng, k, e)[None]
        f = K.LbdFusion(None, 0.0, 0, None, up(np.zeros(n, np.float32)).ptr, None, 0, None, 0, 0)
        y = fused_w4a8(dW, n, k, up(act[0]).ptr, f)
        xq, xs, asum = O.quant_act_int8(act, W.kp)
        np.testing.assert_array_equal(y, q_call(W, xq, xs, asum, 1, dW), err_msg=f"row amax 2^{e}")


@pytest.mark.parametrize("D,H,KV,p,cap", [(64, 14, 2, 150, 193), (64, 14, 2, 100, 512), (128, 8, 2, 200, 224)])
def test_attention_merge_prologue_quantizer_bit_exact(rng, D, H, KV, p, cap):
    """The o projection: its prologue merges the attention partials (bit for bit
    lbd_attention_merge's row, tests/test_gpu_fused.py), then quantizes that row."""
    L = K.lib()
    max_pos = 1024
    cos, sin = DM.rope_tables(D, max_pos, 10000.0)
    n = 896
    W = int4(rng, n, H * D, True)
    dW = K.to_device(W)
    for scale in (1.0, 2.0 ** -30, 2.0 ** 40):
        qkv = (rng.standard_normal((H + 2 * KV) * D) * scale).astype(np.float32)
        kc = (rng.standard_normal((KV, cap, D)) * scale).astype(np.float32)
        vc = (rng.standard_normal((KV, cap, D)) * scale).astype(np.float32)
        dk, dv = up(kc), up(vc)
        dpos = up(np.array([p], np.int32))
        part = K.DeviceBuffer(L.lbd_attention_decode_work_bytes(H, D, cap))
        out = K.DeviceBuffer(4 * H * D)
        _LIVE.extend([part, out])
        ok(L.lbd_attention_slices(up(qkv).ptr, H, KV, D, up(cos).ptr, up(sin).ptr, dpos.ptr, max_pos, dk.ptr,
                                  dv.ptr, cap, part.ptr, part.nbytes, None))
        ok(L.lbd_attention_merge(part.ptr, part.nbytes, H, D, dpos.ptr, cap, out.ptr, None))
        ok(L.lb_stream_synchronize(None))
        act = out.to_array((1, H * D), np.float32)
        f = K.LbdFusion(None, 0.0, 0, None, None, None, 0, part.ptr, cap, D)
        y = fused_w4a8(dW, n, H * D, None, f)
        xq, xs, asum = O.quant_act_int8(act, W.kp)
        np.testing.assert_array_equal(y, q_call(W, xq, xs, asum, 1, dW), err_msg=f"scale {scale}")


# ---------------------------------------------------------------- M >= 5: the tiled quantizer

def detile(ws, m, kp):
    """The tiled codes, token scales and group sums of the int8 MFMA path, read back
    from the workspace into the reference's row-major [M, Kp] / [M] / [M, G] layout.
    Element e of row r sits at byte (((r / 16 G + g) 2 + h) 64 + 16 q + r % 16) 16 + e % 16
    (g = e / 128, h = e % 128 / 64, q = e % 64 / 16); sums at [r / 16][g][r % 16]."""
    g = kp // 128
    mb = (m + 15) // 16
    xq_bytes = mb * 16 * kp
    a256 = lambda v: (v + 255) // 256 * 256
    raw = ws.to_array((ws.nbytes,), np.uint8)
    t = raw[:xq_bytes].view(np.int8).reshape(mb, g, 2, 4, 16, 16)   # [rb][g][h][q][row][16 B]
    xq = t.transpose(0, 4, 1, 2, 3, 5).reshape(mb * 16, kp)
    xs = raw[a256(xq_bytes):a256(xq_bytes) + 4 * m].view(np.float32)
    off = a256(xq_bytes) + a256(4 * m)
    asum = raw[off:off + mb * g * 16 * 4].view(np.int32).reshape(mb, g, 16).transpose(0, 2, 1).reshape(mb * 16, g)
    return xq, xs, asum


@pytest.mark.parametrize("m", [5, 16, 17, 64])
@pytest.mark.parametrize("n,k", [(11008, 4096), (4096, 11008)])
@pytest.mark.parametrize("layout", ["rowmajor", "t16"])
def test_tiled_quantizer_bit_exact(rng, m, n, k, layout):
    W = int4(rng, n, k, True)
    dW = K.to_device(W)
    L = K.lib()
    assert K.gemm_plan("w4a8", m, n, W.kp)["path"] == "gfx950-mfma"
    x = rows(rng, m, k, EXPS[::-1])
    xq, xs, asum = O.quant_act_int8(x, W.kp)
    assert exact_ties(x) > k
    if layout == "rowmajor":
        y, ws = x_call(W, x, dW)
    else:
        qwt, st, zt = dW.tiles()
        ws = K.DeviceBuffer(L.lbd_w4a8_workspace_bytes(m, W.kp))
        yb = K.DeviceBuffer(4 * m * n)
        _LIVE.extend([ws, yb])
        prm = K._Params(0, 0, 0, 0, 0, 0, 0)
        ok(L.lbd_gemm_w4a8_t16(up(x).ptr, m, W.kp, qwt.ptr, st.ptr, zt.ptr, n, yb.ptr, C.byref(prm), ws.ptr,
                               ws.nbytes, None))
        ok(L.lb_stream_synchronize(None))
        y = yb.to_array((m, n), np.float32)
    gq, gs, ga = detile(ws, m, W.kp)
    np.testing.assert_array_equal(gq[:m], xq)
    np.testing.assert_array_equal(gs, xs)
    np.testing.assert_array_equal(ga[:m], asum)
    assert not gq[m:].any() and not ga[m:].any()  # the last row block's padding rows
    # and the output is within the reference's bound of the oracle on those codes
    # (rows whose exact result lies beyond the float32 range overflow to +-inf, as the
    # reference's fp32 result does)
    ref = O.gemm_w4a8_ref(xq, xs, W.qw, W.scales, W.zeros)
    bound = O.w4a8_lane_bound(xq, xs, asum, W.qw, W.scales, W.zeros)
    fits = np.all(np.abs(ref) < 3.0e38, axis=1)
    assert fits.sum() >= (3 * m) // 4
    O.assert_fp_close(y[fits], ref[fits], bound[fits])
    big = np.abs(ref) > 3.5e38
    assert np.all(np.isinf(y[big]) & (np.sign(y[big]) == np.sign(ref[big])))
