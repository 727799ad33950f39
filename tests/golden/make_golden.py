"""Writes tests/golden/ref_vectors.npz: input/output vectors of the reference's own C library.

The library is oracle/_ref/liblowbit_ref.so, the reference's unmodified C sources
(src/lowbit/csrc/*.c) compiled in place by oracle/Makefile. Inputs are seeded;
the packed weights are stored in the file, so the vectors do not depend on any
quantizer. Outputs come from the reference's scalar path (isa 0), the one with a
fixed summation order, and for the integer results also from its best SIMD
path (which must agree bit for bit).

    make -C oracle && python tests/golden/make_golden.py
"""
from __future__ import annotations

import ctypes as C
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from lowbit_amd import formats as F  # noqa: E402  (inputs only: packing seeded weights)
from oracle.cref import RefParams, ref_lib, zp  # noqa: E402

OUT = Path(__file__).resolve().parent / "ref_vectors.npz"


def main() -> None:
    L = ref_lib()
    if L is None:
        raise SystemExit("oracle/_ref/liblowbit_ref.so is not built (make -C oracle)")
    rng = np.random.default_rng(20261201)
    v: dict[str, np.ndarray] = {}

    # ---- per-token int8 quantizer: random rows, a zero row, a constructed .5 tie
    m, k = 4, 300
    kp = F.pad_to(k, 128)
    x = (rng.standard_normal((m, k)) * 3).astype(np.float32)
    x[1] = 0.0
    amax = np.float32(np.abs(x[2]).max())
    sc = np.float32(amax / np.float32(127))
    x[2, 5] = np.float32(np.float32(2.5) * sc)  # lands on (or next to) a tie at 2.5
    xp = F.pad_acts(x, kp)
    xq = np.empty((m, kp), np.int8)
    xs = np.empty(m, np.float32)
    asum = np.empty((m, kp // 128), np.int32)
    L.lb_quant_act_int8(xp, m, kp, xq, xs, asum)
    v.update(q_x=x, q_xq=xq, q_xs=xs, q_asum=asum)

    # ---- exact group accumulators, sym and asym weights, scalar and SIMD paths
    n = 37
    w = rng.standard_normal((n, k)).astype(np.float32)
    for tag, asym in (("sym", False), ("asym", True)):
        W = F.quantize_int4(w, asym=asym)
        out = np.empty((m, n, kp // 128), np.int32)
        assert L.lb_w4a8_group_acc(xq, asum, m, kp, W.qw, zp(W.zeros), n, out, 0) == 0
        out2 = np.empty_like(out)
        L.lb_w4a8_group_acc(xq, asum, m, kp, W.qw, zp(W.zeros), n, out2, -1)
        assert np.array_equal(out, out2), "reference scalar and SIMD accumulators disagree"
        v[f"ga_{tag}_qw"] = W.qw
        v[f"ga_{tag}_scales"] = W.scales
        if W.zeros is not None:
            v[f"ga_{tag}_zeros"] = W.zeros
        v[f"ga_{tag}_out"] = out
        # fp32 GEMMs of the reference (scalar path: fixed summation order)
        p = RefParams(0, 0, 0, 0, 0, 0, 1)
        y = np.empty((m, n), np.float32)
        assert L.lb_gemm_w4a16(xp, m, kp, W.qw, W.scales, zp(W.zeros), n, y, C.byref(p)) == 0
        v[f"w4a16_{tag}_y"] = y.copy()
        assert L.lb_gemm_w4a8(xp, m, kp, W.qw, W.scales, zp(W.zeros), n, y, C.byref(p)) == 0
        v[f"w4a8_{tag}_y"] = y.copy()

    # ---- worst-case accumulator operands (tests/test_kernels.py:108-124 of the reference)
    mw, nw, kw = 3, 4, 512
    codes = np.zeros((nw, kw), np.uint8)
    codes[0] = 15
    codes[1, ::2] = 15
    codes[2] = np.arange(kw) % 16
    qw = F.pack_nibbles(codes, 128)
    zeros = np.repeat(np.array([0, 15, 7, 8], np.uint8)[:, None], kw // 128, axis=1)
    xqw = np.full((mw, kw), 127, np.int8)
    xqw[1] = -128
    xqw[2, ::2] = -128
    asw = xqw.astype(np.int32).reshape(mw, -1, 128).sum(-1).astype(np.int32)
    outw = np.empty((mw, nw, kw // 128), np.int32)
    assert L.lb_w4a8_group_acc(xqw, asw, mw, kw, qw, zp(zeros), nw, outw, 0) == 0
    v.update(wc_qw=qw, wc_zeros=zeros, wc_xq=xqw, wc_asum=asw, wc_out=outw)

    # ---- MXFP4 GEMM, K not a multiple of 128 (tail block)
    km = 100
    wm = rng.standard_normal((n, km)).astype(np.float32)
    Wm = F.quantize_mxfp4(wm)
    xm = F.pad_acts(x[:, :km], Wm.kp)
    ym = np.empty((m, n), np.float32)
    p = RefParams(0, 0, 0, 0, 0, 0, 1)
    assert L.lb_gemm_mxfp4(xm, m, Wm.kp, Wm.qw, Wm.e8m0, n, ym, C.byref(p)) == 0
    v.update(mx_x=xm, mx_qw=Wm.qw, mx_e8m0=Wm.e8m0, mx_y=ym)

    np.savez_compressed(OUT, **v)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes, {len(v)} arrays)")


if __name__ == "__main__":
    main()
