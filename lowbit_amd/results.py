"""Results pipeline: GPU benchmark rows in the reference's bench.json schema and a
RESULTS.md-style report that puts them beside the reference's published CPU numbers.

`run` follows the reference's benchmark driver (src/lowbit/bench.py:140-330): the
same shapes (plus the down-projection batch shapes and two prefill-sized M), the
same synthetic data (seed 0, W ~ N(0, 1) * 0.02, symmetric int4 g128 and MXFP4 of
the same W, X ~ N(0, 1)), one row per (shape, method, cache) with the reference's
fields (`phase`, `M`, `N`, `K`, `threads`, `cache`, `method`, `format`, `isa`,
`params`, `reps`, `t_median_s`, `t_min_s`, `gflops`, `weight_bytes`,
`weight_gbps`, `speedup_vs_numpy_fp32`, `max_rel_err`) and GPU fields added
(`device`, `weight_layout`, `roofline`, `roofline_frac`). Decode shapes run hot and
cold (cold: every launch reads another copy of the weights from a pool larger than
2 x (256 MB Infinity Cache + 32 MB L2), the GPU form of src/lowbit/bench.py:169-178).

Timing: the launches of one repetition are captured as a HIP graph and replayed
between HIP events on the launch stream; a repetition's time per launch is one
sample, t_median_s / t_min_s are the median / minimum over the samples (the
reference's "median of >= 3 reps", src/lowbit/bench.py:116-124, per launch).

`report` renders the headline decode table and the all-shapes table in the layout
of src/lowbit/report.py:44-101, with roofline columns and the reference's best
published 4-thread CPU row for each cell (results/bench.json of the reference,
its RESULTS.md tables) beside it.

    python -m lowbit_amd.results run [--out results] [--quick]
    python -m lowbit_amd.results report results/bench.json > results/RESULTS.md
"""
from __future__ import annotations

import argparse
import ctypes as C
import datetime as _dt
import json
import math
import platform
import statistics
import sys
import time
from pathlib import Path

import numpy as np

from . import formats as F
from . import kernels as K

DECODE_SHAPES = [(1, 4096, 4096), (1, 11008, 4096), (1, 4096, 11008)]
BATCH_SHAPES = [(16, 4096, 4096), (64, 4096, 4096), (16, 11008, 4096), (64, 11008, 4096),
                (16, 4096, 11008), (64, 4096, 11008)]
PREFILL_SHAPES = [(512, 4096, 4096), (2048, 4096, 4096)]
QUICK_SHAPES = [(1, 4096, 4096), (16, 4096, 4096)]
FORMATS = ["w4a16", "w4a8", "mxfp4"]
G32_FORMATS = ["w4a16", "w4a8"]  # int4 with groups of 32 (decode shapes only)
HEADLINE_SHAPE = (1, 11008, 4096)

# MI355X published peaks (dense)
HBM_GBS = 8000.0
PEAK_TFLOPS = {"int8": 5000.0, "bf16": 2500.0, "fp32": 157.3}
COLD_POOL_BYTES = 1280 << 20

# The reference's best published 4-thread row per (M, N, K, format, cache): (method,
# t_median_s, GFLOP/s, weight GB/s), from its results/bench.json (rendered in its
# results/RESULTS.md:77-395; Xeon @ 2.10 GHz, 4 vCPU, AVX-512 VNNI + AMX).
REFERENCE_4T = {
    (1, 4096, 4096, "w4a16", "cold"): ("w4a16 avx512", 474e-6, 70.7, 18.8),
    (1, 4096, 4096, "w4a16", "hot"): ("w4a16 avx512", 237e-6, 141.7, 37.6),
    (1, 4096, 4096, "w4a8", "cold"): ("w4a8 avx512-vnni", 265e-6, 126.8, 33.7),
    (1, 4096, 4096, "w4a8", "hot"): ("w4a8 avx512-vnni", 136e-6, 246.4, 65.4),
    (1, 4096, 4096, "mxfp4", "cold"): ("mxfp4 avx512", 425e-6, 78.9, 21.0),
    (1, 4096, 4096, "mxfp4", "hot"): ("mxfp4 avx512", 259e-6, 129.7, 34.4),
    (1, 11008, 4096, "w4a16", "cold"): ("w4a16 avx512", 1070e-6, 84.2, 22.4),
    (1, 11008, 4096, "w4a16", "hot"): ("w4a16 avx512", 529e-6, 170.5, 45.3),
    (1, 11008, 4096, "w4a8", "cold"): ("w4a8 avx512-vnni", 621e-6, 145.2, 38.6),
    (1, 11008, 4096, "w4a8", "hot"): ("w4a8 avx2-maddubs", 324e-6, 278.2, 73.9),
    (1, 11008, 4096, "mxfp4", "cold"): ("mxfp4 avx512", 866e-6, 104.1, 27.6),
    (1, 11008, 4096, "mxfp4", "hot"): ("mxfp4 avx512", 611e-6, 147.6, 39.2),
    (1, 4096, 11008, "w4a16", "cold"): ("w4a16 avx512", 806e-6, 111.9, 29.7),
    (1, 4096, 11008, "w4a16", "hot"): ("w4a16 avx512", 524e-6, 172.0, 45.7),
    (1, 4096, 11008, "w4a8", "cold"): ("w4a8 avx512-vnni", 568e-6, 158.6, 42.1),
    (1, 4096, 11008, "w4a8", "hot"): ("w4a8 avx512-vnni", 326e-6, 276.7, 73.5),
    (1, 4096, 11008, "mxfp4", "cold"): ("mxfp4 avx512", 839e-6, 107.5, 28.6),
    (1, 4096, 11008, "mxfp4", "hot"): ("mxfp4 avx512", 594e-6, 151.8, 40.3),
    (16, 4096, 4096, "w4a16", "hot"): ("w4a16 avx512", 1444e-6, 371.7, 6.2),
    (16, 4096, 4096, "w4a8", "hot"): ("w4a8 amx", 400e-6, 1341.0, 23.6),
    (16, 4096, 4096, "mxfp4", "hot"): ("mxfp4 avx512", 1634e-6, 328.7, 5.5),
    (64, 4096, 4096, "w4a16", "hot"): ("w4a16 avx512", 7655e-6, 280.5, 1.2),
    (64, 4096, 4096, "w4a8", "hot"): ("w4a8 amx", 1410e-6, 1523.2, 6.7),
    (64, 4096, 4096, "mxfp4", "hot"): ("mxfp4 avx512", 6693e-6, 320.9, 1.3),
    (16, 11008, 4096, "w4a16", "hot"): ("w4a16 avx512", 3524e-6, 409.5, 6.8),
    (16, 11008, 4096, "w4a8", "hot"): ("w4a8 amx", 874e-6, 1651.7, 29.0),
    (16, 11008, 4096, "mxfp4", "hot"): ("mxfp4 avx512", 4284e-6, 336.8, 5.6),
    (64, 11008, 4096, "w4a16", "hot"): ("w4a16 avx512", 17984e-6, 320.9, 1.3),
    (64, 11008, 4096, "w4a8", "hot"): ("w4a8 amx", 2666e-6, 2164.8, 9.5),
    (64, 11008, 4096, "mxfp4", "hot"): ("mxfp4 avx512", 17940e-6, 321.7, 1.3),
}

_KIND = {"w4a16": 0, "mxfp4": 1, "w4a8": 2}


def _check(rc: int, what: str) -> int:
    if rc < 0:
        K._err(rc, what)
    return rc


def _rel_err(y: np.ndarray, ref: np.ndarray) -> float:
    """max |y - ref| / max |ref| (the reference's max_rel_err)."""
    return float(np.abs(y.astype(np.float64) - ref).max() / max(np.abs(ref).max(), 1e-300))


class _Timer:
    """Graph-replayed launches timed with HIP events on one stream."""

    def __init__(self):
        self.L = K.lib()
        s = C.c_void_p()
        _check(self.L.lb_stream_create(C.byref(s)), "stream")
        self.stream = s.value

    def _event(self):
        e = C.c_void_p()
        _check(self.L.lb_event_create(C.byref(e)), "event")
        return e.value

    WARM_MS = 10.0  # untimed replays first, at least this long (an idle GPU's clocks ramp up)

    def samples(self, launch, n_launch: int, reps: int) -> list[float]:
        """Seconds per launch, one sample per replay of a graph of n_launch launches,
        after untimed replays of the same graph for at least WARM_MS."""
        L, s = self.L, self.stream
        _check(L.lb_stream_synchronize(s), "sync")
        _check(L.lb_stream_begin_capture(s), "begin capture")
        try:
            for i in range(n_launch):
                launch(i)
        finally:
            ex = C.c_void_p()
            _check(L.lb_stream_end_capture(s, C.byref(ex)), "end capture")
        e0, e1 = self._event(), self._event()
        out = []
        try:
            _check(L.lb_event_record(e0, s), "record")
            _check(L.lb_graph_launch(ex.value, s), "graph warm-up")
            _check(L.lb_event_record(e1, s), "record")
            _check(L.lb_event_synchronize(e1), "sync")
            ms = C.c_float()
            _check(L.lb_event_elapsed_ms(e0, e1, C.byref(ms)), "elapsed")
            for _ in range(min(1000, max(0, math.ceil(self.WARM_MS / max(1e-3, ms.value)) - 1))):
                _check(L.lb_graph_launch(ex.value, s), "graph warm-up")
            for _ in range(reps):
                _check(L.lb_stream_synchronize(s), "sync")
                _check(L.lb_event_record(e0, s), "record")
                _check(L.lb_graph_launch(ex.value, s), "graph launch")
                _check(L.lb_event_record(e1, s), "record")
                _check(L.lb_event_synchronize(e1), "sync")
                ms = C.c_float()
                _check(L.lb_event_elapsed_ms(e0, e1, C.byref(ms)), "elapsed")
                out.append(ms.value * 1e-3 / n_launch)
        finally:
            L.lb_graph_destroy(ex.value)
            L.lb_event_destroy(e0)
            L.lb_event_destroy(e1)
        return out


def _gemm_case(timer: _Timer, fmt: str, shape, W, x: np.ndarray, cold: bool):
    """(launch(i), y of the first launch, path name, layout, pool size) for one GEMM."""
    L, s = timer.L, timer.stream
    m, n, _ = shape
    prm = K._Params(-1, 0, 0, 0, 0, 0, 0)
    g32 = getattr(W, "group", F.GROUP) == 32
    mfma = not g32 and _check(L.lbd_gemm_path(_KIND[fmt], m, W.kp, C.byref(prm)), "path") == K.ISA_GFX950_MFMA
    copies = max(1, -(-COLD_POOL_BYTES // W.nbytes)) if cold else 1
    first = K.to_device(W)
    pool = [first] + [K.to_device(W) for _ in range(copies - 1)]
    dx = K.DeviceBuffer.from_array(F.pad_acts(x, W.kp))
    dy = K.DeviceBuffer(4 * m * n)
    if mfma:
        for d in pool:
            if fmt == "w4a16" and K.w4a16_uses_t16f8(d, m):
                d.tiles_f8()
            else:
                d.tiles()
        ws_bytes = (L.lbd_w4a8_workspace_bytes(m, W.kp) if fmt == "w4a8"
                    else L.lbd_bf16x3_workspace_bytes_split(_KIND[fmt], m, n, W.kp))
    else:
        ws_bytes = L.lbd_w4a8_workspace_bytes(m, W.kp)
    ws = K.DeviceBuffer(ws_bytes)

    def launch(i):
        d = pool[i % len(pool)]
        if g32:
            fn = L.lbd_gemm_w4a16_g32 if fmt == "w4a16" else L.lbd_gemm_w4a8_g32
            return _check(fn(dx.ptr, m, W.kp, d.qw.ptr, d.scales.ptr, None if d.zeros is None else d.zeros.ptr, n,
                             dy.ptr, s), f"{fmt} g32 GEMM")
        if mfma:
            if fmt == "mxfp4":
                qwt, et = d.tiles()
                rc = L.lbd_gemm_mxfp4_t16(dx.ptr, m, W.kp, qwt.ptr, et.ptr, n, dy.ptr, C.byref(prm), ws.ptr,
                                          ws_bytes, s)
            elif fmt == "w4a16":
                rc = K.gemm_w4a16_tiles(d, dx.ptr, m, dy.ptr, prm, ws.ptr, ws_bytes, s)
            else:
                qwt, st, zt = d.tiles()
                rc = L.lbd_gemm_w4a8_t16(dx.ptr, m, W.kp, qwt.ptr, st.ptr, None if zt is None else zt.ptr, n,
                                         dy.ptr, C.byref(prm), ws.ptr, ws_bytes, s)
        elif fmt == "mxfp4":
            rc = L.lbd_gemm_mxfp4(dx.ptr, m, W.kp, d.qw.ptr, d.e8m0.ptr, n, dy.ptr, C.byref(prm), s)
        elif fmt == "w4a16":
            rc = L.lbd_gemm_w4a16(dx.ptr, m, W.kp, d.qw.ptr, d.scales.ptr, None if d.zeros is None else d.zeros.ptr,
                                  n, dy.ptr, C.byref(prm), s)
        else:
            rc = L.lbd_gemm_w4a8(dx.ptr, m, W.kp, d.qw.ptr, d.scales.ptr, None if d.zeros is None else d.zeros.ptr,
                                 n, dy.ptr, C.byref(prm), ws.ptr, ws_bytes, s)
        return _check(rc, f"{fmt} GEMM")

    path = launch(0)
    _check(L.lb_stream_synchronize(s), "sync")
    y = dy.to_array((m, n), np.float32)
    keep = (pool, dx, dy, ws)  # alive while the caller times `launch`
    layout = ("t16f8" if fmt == "w4a16" and K.w4a16_uses_t16f8(first, m) else "t16") if mfma else "row-major"
    return launch, y, K.ISA_NAMES.get(path, "?"), layout, len(pool), keep


def _roofline(fmt: str, layout: str, m: int, n: int, k: int, t: float, wbytes: int) -> tuple[str, float]:
    """(roofline name, fraction) of one row: HBM for the decode kernels, the matrix
    cores' dense peak otherwise (three bf16 products per fp32 product on MXFP4's
    bf16x3, two float16 products per product on W4A16's f16x2; one dense peak)."""
    if layout == "row-major":
        return "hbm", (wbytes + 4 * m * (k + n)) / t / 1e9 / HBM_GBS
    if fmt == "w4a8":
        return "int8 mfma", 2.0 * m * n * k / t / 1e12 / PEAK_TFLOPS["int8"]
    if fmt == "w4a16":
        return "f16x2 mfma", 2 * 2.0 * m * n * k / t / 1e12 / PEAK_TFLOPS["bf16"]
    return "bf16x3 mfma", 3 * 2.0 * m * n * k / t / 1e12 / PEAK_TFLOPS["bf16"]


def run(shapes=None, cold: bool = True, seed: int = 0, n_launch: int = 50, reps: int = 7, log=print) -> dict:
    """Benchmark rows for every shape and format (src/lowbit/bench.py:140-307)."""
    shapes = shapes or DECODE_SHAPES + BATCH_SHAPES + PREFILL_SHAPES
    info = K.cpu_info()
    timer = _Timer()
    rng = np.random.default_rng(seed)
    rows = []
    t_start = time.time()
    for (m, n, k) in shapes:
        log(f"== shape M={m} N={n} K={k}")
        w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
        x = rng.standard_normal((m, k)).astype(np.float32)
        wq = {"w4a16": F.quantize_int4(w), "mxfp4": F.quantize_mxfp4(w)}
        wq["w4a8"] = wq["w4a16"]
        w32 = w if m == 1 else None
        del w
        ref = {f: x.astype(np.float64) @ wq[f].dequantize().T.astype(np.float64) for f in ("w4a16", "mxfp4")}
        ref["w4a8"] = ref["w4a16"]
        phase = "decode" if m == 1 else ("batch" if m <= 64 else "prefill")
        modes = ["hot", "cold"] if (cold and m == 1) else ["hot"]
        for mode in modes:
            for fmt in FORMATS:
                W = wq[fmt]
                launch, y, path, layout, copies, keep = _gemm_case(timer, fmt, (m, n, k), W, x, mode == "cold")
                nl = max(n_launch, 2 * copies) if mode == "cold" else n_launch
                ts = timer.samples(launch, nl, reps)
                del keep
                med, mn = statistics.median(ts), min(ts)
                roof, frac = _roofline(fmt, layout, m, n, k, med, W.nbytes)
                row = {
                    "phase": phase, "M": m, "N": n, "K": k, "threads": None, "cache": mode,
                    "method": f"{fmt} {path}", "format": fmt, "isa": path, "params": None,
                    "reps": len(ts), "t_median_s": med, "t_min_s": mn,
                    "gflops": 2.0 * m * n * k / med / 1e9, "weight_bytes": int(W.nbytes),
                    "weight_gbps": W.nbytes / med / 1e9, "speedup_vs_numpy_fp32": None,
                    "max_rel_err": _rel_err(y, ref[fmt]),
                    "device": info.get("arch"), "weight_layout": layout, "pool_copies": copies,
                    "launches_per_rep": nl, "roofline": roof, "roofline_frac": frac,
                }
                rows.append(row)
                log(f"  [{mode}] {row['method']:<18} {med * 1e6:9.2f} us  {row['gflops']:10.1f} GFLOP/s  "
                    f"{row['weight_gbps']:7.1f} GB/s  {100 * frac:5.1f}% of {roof}  rel err {row['max_rel_err']:.2g}")
            if m > 1:
                continue
            # int4 with groups of 32 (this package's extension): decode shapes
            for fmt in G32_FORMATS:
                W = W32 = wq.setdefault("g32", F.quantize_int4(w32, group=32))
                ref32 = ref.setdefault("g32", x.astype(np.float64) @ W32.dequantize().T.astype(np.float64))
                launch, y, path, layout, copies, keep = _gemm_case(timer, fmt, (m, n, k), W, x, mode == "cold")
                nl = max(n_launch, 2 * copies) if mode == "cold" else n_launch
                ts = timer.samples(launch, nl, reps)
                del keep
                med, mn = statistics.median(ts), min(ts)
                roof, frac = _roofline(fmt, layout, m, n, k, med, W.nbytes)
                rows.append({
                    "phase": phase, "M": m, "N": n, "K": k, "threads": None, "cache": mode,
                    "method": f"{fmt}-g32 {path}", "format": f"{fmt}-g32", "isa": path, "params": None,
                    "reps": len(ts), "t_median_s": med, "t_min_s": mn,
                    "gflops": 2.0 * m * n * k / med / 1e9, "weight_bytes": int(W.nbytes),
                    "weight_gbps": W.nbytes / med / 1e9, "speedup_vs_numpy_fp32": None,
                    "max_rel_err": _rel_err(y, ref32), "device": info.get("arch"), "weight_layout": layout,
                    "pool_copies": copies, "launches_per_rep": nl, "roofline": roof, "roofline_frac": frac,
                })
                r = rows[-1]
                log(f"  [{mode}] {r['method']:<18} {med * 1e6:9.2f} us  {r['weight_gbps']:7.1f} GB/s  "
                    f"{100 * frac:5.1f}% of {roof}  rel err {r['max_rel_err']:.2g}")
    meta = {
        "date": _dt.datetime.now(_dt.timezone.utc).isoformat(timespec="seconds"),
        "device": f"{info.get('arch')} ({info.get('compute_units')} CUs)",
        "lowbit": {k_: v for k_, v in info.items() if k_ in ("cpu_isa", "active_isa")},
        "host": platform.processor() or platform.machine(), "numpy": np.__version__,
        "python": platform.python_version(), "wall_s": round(time.time() - t_start, 1),
        "timing": (f"per launch, median (and min) over {reps} replays of a HIP graph of {n_launch}+ launches, "
                   "HIP events on the launch stream; cold = weights rotated over copies > 1.28 GB"),
        "peaks": {"hbm_gbs": HBM_GBS, **{f"{k_}_tflops": v for k_, v in PEAK_TFLOPS.items()}},
    }
    return {"meta": meta, "rows": rows}


def save(result: dict, out_dir) -> Path:
    """results/bench.json (src/lowbit/bench.py:321-326)."""
    out = Path(out_dir)
    out.mkdir(parents=True, exist_ok=True)
    p = out / "bench.json"
    p.write_text(json.dumps(result, indent=1))
    return p


# ---------------------------------------------------------------- report

def _t(s: float) -> str:
    return f"{s * 1e6:.1f} µs" if s < 1e-3 else f"{s * 1e3:.2f} ms"


def _row(rows, **kv):
    for r in rows:
        if all(r.get(k_) == v for k_, v in kv.items()):
            return r
    return None


def report(res: dict) -> str:
    """Markdown tables in the layout of src/lowbit/report.py:44-101, GPU beside CPU."""
    rows, meta = res["rows"], res["meta"]
    out = []
    m, n, k = HEADLINE_SHAPE
    sel = [r for r in rows if (r["M"], r["N"], r["K"]) == HEADLINE_SHAPE]
    if sel:
        cache = "cold" if any(r["cache"] == "cold" for r in sel) else "hot"
        out += [f"**Decode, M={m}, N={n}, K={k} (LLaMA-7B MLP up-projection), {cache} cache** — weights "
                "streamed from HBM every call; the reference's best 4-thread CPU row beside each:\n",
                "| method | weight bytes | MI355X time | weight GB/s | % of HBM roofline | reference (4T) | "
                "reference time | reference GB/s | speedup |", "|---|---|---|---|---|---|---|---|---|"]
        for fmt in FORMATS:
            r = _row(sel, format=fmt, cache=cache)
            if r is None:
                continue
            ref = REFERENCE_4T.get((m, n, k, fmt, cache))
            refc = (f"{ref[0]} | {_t(ref[1])} | {ref[3]:.1f} | {ref[1] / r['t_median_s']:.0f}×" if ref
                    else "— | — | — | —")
            out.append(f"| {r['method']} | {r['weight_bytes'] / 2**20:.1f} MiB | {_t(r['t_median_s'])} | "
                       f"{r['weight_gbps']:.0f} | {100 * r['roofline_frac']:.1f} % | {refc} |")
        out.append("")
    out += ["**All shapes, hot cache** — MI355X GFLOP/s (fraction of the roofline that bounds the kernel: HBM "
            "for the decode kernels, the dense int8 / bf16x3 (MXFP4) / f16x2 (W4A16) matrix-core peak otherwise), and the reference's "
            "best 4-thread CPU GFLOP/s:\n",
            "| M | N | K | W4A16 | W4A8 | MXFP4 | ref W4A16 (4T) | ref W4A8 (4T) | ref MXFP4 (4T) |",
            "|---|---|---|---|---|---|---|---|---|"]
    shapes = []
    for r in rows:
        sh = (r["M"], r["N"], r["K"])
        if sh not in shapes:
            shapes.append(sh)
    for sh in shapes:
        cells, refs = [], []
        for fmt in FORMATS:
            r = _row(rows, M=sh[0], N=sh[1], K=sh[2], format=fmt, cache="hot")
            cells.append(f"{r['gflops']:.0f} ({100 * r['roofline_frac']:.0f} % {r['roofline']})" if r else "—")
            ref = REFERENCE_4T.get((*sh, fmt, "hot"))
            refs.append(f"{ref[2]:.1f}" if ref else "—")
        out.append(f"| {sh[0]} | {sh[1]} | {sh[2]} | " + " | ".join(cells + refs) + " |")
    out.append("")
    g32 = [r for r in rows if r["format"].endswith("-g32")]
    if g32:
        out += ["**int4 with groups of 32** (this package's extension; the reference ships group 128) — decode "
                "shapes, the same weights as above with 4x the scales:\n",
                "| M | N | K | cache | method | weight bytes | time | weight GB/s | % of HBM roofline | rel err |",
                "|---|---|---|---|---|---|---|---|---|---|"]
        for r in g32:
            out.append(f"| {r['M']} | {r['N']} | {r['K']} | {r['cache']} | {r['method']} | "
                       f"{r['weight_bytes'] / 2**20:.1f} MiB | {_t(r['t_median_s'])} | {r['weight_gbps']:.0f} | "
                       f"{100 * r['roofline_frac']:.1f} % | {r['max_rel_err']:.2g} |")
        out.append("")
    out.append(f"Measured {meta['date']} on {meta['device']}; {meta['timing']}. Maximum relative error against "
               f"float64 over every row: {max(r['max_rel_err'] for r in rows):.2g}. Reference rows: its "
               "results/bench.json (Xeon @ 2.10 GHz, 4 vCPU, AVX-512 VNNI + AMX).")
    return "\n".join(out)


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description="GPU results pipeline (bench.json rows and RESULTS.md tables)")
    sub = ap.add_subparsers(dest="cmd", required=True)
    r = sub.add_parser("run")
    r.add_argument("--out", default="results")
    r.add_argument("--quick", action="store_true", help="two small shapes only")
    r.add_argument("--no-cold", action="store_true")
    p = sub.add_parser("report")
    p.add_argument("json")
    a = ap.parse_args(argv)
    if a.cmd == "run":
        res = run(QUICK_SHAPES if a.quick else None, cold=not a.no_cold,
                  log=lambda *s: print(*s, file=sys.stderr, flush=True))
        path = save(res, a.out)
        (Path(a.out) / "RESULTS.md").write_text(report(res) + "\n")
        print(path)
    else:
        print(report(json.loads(Path(a.json).read_text())))
    return 0


if __name__ == "__main__":
    sys.exit(main())
