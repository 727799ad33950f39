#!/usr/bin/env python3
"""Benchmark of the fused dequantize+GEMM hot path on one MI355X.

Metric: weight GB/s (and % of HBM peak) at M=1, N=11008, K=4096,
and GFLOP/s at M=64, per format. The headline `value` is the W4A8 decode GEMV
(int4 g128 asymmetric weights, int8 per-token activations quantized inside the
call) with weights cold: every call reads a different copy from a pool of more
than 2 x (256 MB Infinity Cache + 8 x 4 MB L2), so each call streams its
weights from HBM (the cold rule of src/lowbit/bench.py:169-178, sized for the GPU).

One step = one GEMM call on device-resident inputs. The timed launches are
captured in a HIP graph and replayed, so host launch overhead is not counted;
HIP events on the launch stream bracket the timed replay (after W warm-up
steps, a device synchronisation, and untimed replays of the same graph for at
least 10 ms queued right before it, so that the GPU's clocks have risen as in
steady use; a device synchronisation after it). The metric definitions
follow src/lowbit/bench.py:213-214: weight GB/s = packed weight bytes / time,
GFLOP/s = 2*M*N*K / time with the logical K.

The CPU baseline times the reference's own C library (oracle/_ref, built from
the reference sources) on this host's cores on a bounded sample of the same
workload; it is a reported baseline only.

The config-5 decoder (a Qwen2.5-0.5B-shaped model with random weights, every
linear layer W4A8 or MXFP4) is timed as tokens/s of greedy decoding under
"decoder", beside the reference's published CPU tokens/s.

    python bench.py [--gpus 1] [--steps 200] [--warmup 20] [--no-cpu] [--no-decoder]
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import math
import os
import platform
import subprocess
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0        # MI355X HBM3E, published
INT8_PEAK_TOPS = 5000.0      # dense int8 MFMA, published (POP/s -> TOP/s here)
FP32_PEAK_TFLOPS = 157.3     # dense fp32 matrix, published
BF16_PEAK_TFLOPS = 2500.0    # dense bf16 MFMA, published
BF16X3_TERMS = 3             # bf16 products per fp32 product on the bf16x3 path (MXFP4)
F16X2_TERMS = 2              # float16 products per product on the W4A16 two-term path
COLD_POOL_BYTES = 1280 << 20  # > 2 x (256 MB MALL + 32 MB L2)
DECODE = (1, 11008, 4096)
BATCH = (64, 11008, 4096)
TRAFFIC_FILE = ROOT / "profiles" / "traffic_w4a8_gemv_1x11008x4096.txt"
TRACE_FILE = ROOT / "profiles" / "kernel_trace_headline_w4a8_1x11008x4096.md"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


# ------------------------------------------------------------------ device helpers

class Dev:
    """Thin wrapper over the library's device plumbing."""

    def __init__(self):
        from lowbit_amd import kernels as K
        self.K = K
        self.L = K.lib()
        s = C.c_void_p()
        self.check(self.L.lb_stream_create(C.byref(s)), "stream")
        self.stream = s.value

    def check(self, rc, what):
        if rc < 0:
            raise RuntimeError(f"{what}: rc={rc} {self.L.lb_last_error().decode()}")
        return rc

    def upload(self, a: np.ndarray):
        return self.K.DeviceBuffer.from_array(a)

    def event(self):
        e = C.c_void_p()
        self.check(self.L.lb_event_create(C.byref(e)), "event")
        return e.value

    def elapsed_ms(self, e0, e1) -> float:
        ms = C.c_float()
        self.check(self.L.lb_event_elapsed_ms(e0, e1, C.byref(ms)), "elapsed")
        return ms.value

    GATE_WGS = 256

    def gate(self, us: float):
        """Enqueue a busy kernel (the fmac issue-rate probe) of about `us` microseconds on
        the stream: launches enqueued behind it start back to back when it ends, however
        slowly the host (or a tracer intercepting every launch) enqueues them."""
        L = self.L
        if not hasattr(self, "_gate_out"):
            # calibrate on the last of several runs: the first ones run while the clocks
            # of an idle GPU ramp up (2000 iterations took 1.6 ms cold, ~0.3 ms warm)
            self._gate_out = self.K.DeviceBuffer(self.GATE_WGS * 512 * 4)
            iters = 20000
            e0, e1 = self.event(), self.event()
            for _ in range(4):
                self.check(L.lb_dev_synchronize(), "sync")
                self.check(L.lb_event_record(e0, self.stream), "record")
                self.check(L.lbd_probe_valu(0, iters, self.GATE_WGS, self._gate_out.ptr, self.stream), "gate")
                self.check(L.lb_event_record(e1, self.stream), "record")
                self.check(L.lb_event_synchronize(e1), "sync")
            self._gate_iters_per_us = iters / max(1e-3, self.elapsed_ms(e0, e1) * 1e3)
            L.lb_event_destroy(e0)
            L.lb_event_destroy(e1)
        iters = max(1, int(us * self._gate_iters_per_us))
        self.check(L.lbd_probe_valu(0, iters, self.GATE_WGS, self._gate_out.ptr, self.stream), "gate")

    GATE_US_PER_LAUNCH = 40.0  # host time per queued launch the gate covers (tracer included)

    WARM_MS = 10.0  # replays of the captured graph before the timed one, at least this long

    def time_launches(self, launch, n_launch: int, warmup: int, graph: bool = True) -> float:
        """ms per launch of `launch(i)` over n_launch launches (HIP events on the stream):
        a replayed graph, or (graph=False) plain launches queued behind a busy kernel so
        that they run back to back as the graph's do. The graph is replayed untimed for
        at least WARM_MS first, the timed replay queued right behind those replays: an
        idle GPU's clocks take milliseconds to rise, and the arithmetic-heavy W4A16
        decode GEMV measured 0.3-0.7 us slower after a single warm-up replay."""
        L = self.L
        if not graph:
            self.gate(self.GATE_US_PER_LAUNCH * warmup)
        for i in range(warmup):
            launch(i)
        self.check(L.lb_stream_synchronize(self.stream), "sync")
        e0, e1 = self.event(), self.event()
        if graph:
            self.check(L.lb_stream_begin_capture(self.stream), "begin capture")
            for i in range(n_launch):
                launch(i)
            ex = C.c_void_p()
            self.check(L.lb_stream_end_capture(self.stream, C.byref(ex)), "end capture")
            # one warm-up replay, timed, then as many more as fill WARM_MS, with the
            # timed replay queued behind them (no idle gap before it)
            self.check(L.lb_event_record(e0, self.stream), "record")
            self.check(L.lb_graph_launch(ex.value, self.stream), "graph warm-up")
            self.check(L.lb_event_record(e1, self.stream), "record")
            self.check(L.lb_event_synchronize(e1), "sync")
            more = min(1000, max(0, math.ceil(self.WARM_MS / max(1e-3, self.elapsed_ms(e0, e1))) - 1))
            for _ in range(more):
                self.check(L.lb_graph_launch(ex.value, self.stream), "graph warm-up")
            self.check(L.lb_event_record(e0, self.stream), "record")
            self.check(L.lb_graph_launch(ex.value, self.stream), "graph launch")
            self.check(L.lb_event_record(e1, self.stream), "record")
            self.check(L.lb_event_synchronize(e1), "sync")
            L.lb_graph_destroy(ex.value)
        else:
            self.check(L.lb_dev_synchronize(), "sync")
            self.gate(self.GATE_US_PER_LAUNCH * n_launch)
            self.check(L.lb_event_record(e0, self.stream), "record")
            for i in range(n_launch):
                launch(i)
            self.check(L.lb_event_record(e1, self.stream), "record")
            self.check(L.lb_event_synchronize(e1), "sync")
        self.check(L.lb_dev_synchronize(), "sync")
        ms = self.elapsed_ms(e0, e1)
        L.lb_event_destroy(e0)
        L.lb_event_destroy(e1)
        return ms / n_launch


MIN_LAUNCHES = 100  # timed launches per measurement, at least (BASELINE: >= 100 launches)


def timed_launches(steps: int, pool: int) -> int:
    """Launches in one timed graph: the requested steps, but never fewer than one pass
    over the weight pool (so a cold measurement reads every copy) or MIN_LAUNCHES."""
    return max(steps, pool, MIN_LAUNCHES)


def weight_pool(dev: Dev, arrays: list[np.ndarray], nbytes: int, cold: bool):
    """Device copies of the packed weight arrays; > COLD_POOL_BYTES in total when cold."""
    copies = max(1, math.ceil(COLD_POOL_BYTES / nbytes)) if cold else 1
    first = [dev.upload(a) for a in arrays]
    pool = [first]
    for _ in range(copies - 1):
        cp = []
        for a, src in zip(arrays, first):
            b = dev.K.DeviceBuffer(a.nbytes)
            dev.check(dev.L.lb_memcpy_d2d(b.ptr, src.ptr, a.nbytes), "d2d")
            cp.append(b)
        pool.append(cp)
    return pool


# ------------------------------------------------------------------ one GPU measurement

def measure(dev: Dev, fmt: str, shape, W, x: np.ndarray, cold: bool, steps: int, warmup: int,
            graph: bool = True, eager_too: bool = False, call: bool = True) -> dict:
    """One GEMM configuration: device time per launch over >= MIN_LAUNCHES launches
    (HIP events around a replayed graph, or around plain launches with graph=False;
    eager_too adds the plain-launch time beside the graph's), and the wall time of
    one synchronous Python call (call=False skips it, for kernel traces)."""
    from lowbit_amd import formats as F
    K = dev.K
    L = dev.L
    m, n, k = shape
    xp = F.pad_acts(x, W.kp)
    if fmt == "mxfp4":
        arrays = [W.qw, W.e8m0]
    else:
        arrays = [W.qw, W.scales] + ([W.zeros] if W.zeros is not None else [])
    pool = weight_pool(dev, arrays, W.nbytes, cold)
    dx = dev.upload(xp)
    dy = K.DeviceBuffer(m * n * 4)
    prm = K._Params(-1, 0, 0, 0, 0, 0, 0)
    ws_bytes = L.lbd_w4a8_workspace_bytes(m, W.kp)
    ws = K.DeviceBuffer(ws_bytes)
    s = dev.stream
    # the matrix-core regime reads the t16 tile layout (a one-time device repack of
    # each resident copy, as lowbit_amd.to_device handles do; not timed)
    layout = "row-major"
    if L.lbd_gemm_path({"w4a16": 0, "mxfp4": 1, "w4a8": 2}[fmt], m, W.kp, C.byref(prm)) == K.ISA_GFX950_MFMA:
        layout = "t16"
        tiled = []
        if fmt == "mxfp4":
            bq, be = C.c_size_t(0), C.c_size_t(0)
            dev.check(L.lbd_mxfp4_t16_bytes(n, W.kp, C.byref(bq), C.byref(be)), "t16 sizes")
            for b in pool:
                qwt, et = K.DeviceBuffer(bq.value), K.DeviceBuffer(be.value)
                dev.check(L.lbd_repack_mxfp4_t16(b[0].ptr, b[1].ptr, n, W.kp, qwt.ptr, et.ptr, s), "t16 repack")
                tiled.append((qwt, et))
        elif fmt == "w4a16" and L.lbd_w4a16_prefers_t16f8(m, n, W.kp) == 1 and \
                (W.zeros is None or int(W.zeros.max(initial=0)) <= 15):
            # the t16f8 copy (zero-points folded in), where lowbit_amd handles read it
            layout = "t16f8"
            bq, bs = C.c_size_t(0), C.c_size_t(0)
            dev.check(L.lbd_int4_t16f8_bytes(n, W.kp, C.byref(bq), C.byref(bs)), "t16f8 sizes")
            for b in pool:
                qwt8, st = K.DeviceBuffer(bq.value), K.DeviceBuffer(bs.value)
                dev.check(L.lbd_repack_int4_t16f8(b[0].ptr, b[1].ptr, b[2].ptr if len(b) > 2 else None, n, W.kp,
                                                  qwt8.ptr, st.ptr, s), "t16f8 repack")
                tiled.append((qwt8, st))
        else:
            bq, bs, bz = C.c_size_t(0), C.c_size_t(0), C.c_size_t(0)
            dev.check(L.lbd_int4_t16_bytes(n, W.kp, C.byref(bq), C.byref(bs), C.byref(bz)), "t16 sizes")
            for b in pool:
                qwt, st = K.DeviceBuffer(bq.value), K.DeviceBuffer(bs.value)
                zt = K.DeviceBuffer(bz.value) if len(b) > 2 else None
                dev.check(L.lbd_repack_int4_t16(b[0].ptr, b[1].ptr, b[2].ptr if len(b) > 2 else None, n, W.kp,
                                                qwt.ptr, st.ptr, zt.ptr if zt else None, s), "t16 repack")
                tiled.append((qwt, st, zt))
        dev.check(L.lb_stream_synchronize(s), "sync")
        pool = tiled
        if fmt != "w4a8":
            ws_bytes = L.lbd_bf16x3_workspace_bytes_split(0 if fmt == "w4a16" else 1, m, n, W.kp)
            ws = K.DeviceBuffer(ws_bytes)

    def launch(i):
        b = pool[i % len(pool)]
        if layout == "t16f8":
            rc = L.lbd_gemm_w4a16_t16f8(dx.ptr, m, W.kp, b[0].ptr, b[1].ptr, n, dy.ptr, C.byref(prm), ws.ptr,
                                        ws_bytes, s)
        elif layout == "t16":
            if fmt == "w4a8":
                rc = L.lbd_gemm_w4a8_t16(dx.ptr, m, W.kp, b[0].ptr, b[1].ptr, b[2].ptr if b[2] else None, n,
                                         dy.ptr, C.byref(prm), ws.ptr, ws_bytes, s)
            elif fmt == "w4a16":
                rc = L.lbd_gemm_w4a16_t16(dx.ptr, m, W.kp, b[0].ptr, b[1].ptr, b[2].ptr if b[2] else None, n,
                                          dy.ptr, C.byref(prm), ws.ptr, ws_bytes, s)
            else:
                rc = L.lbd_gemm_mxfp4_t16(dx.ptr, m, W.kp, b[0].ptr, b[1].ptr, n, dy.ptr, C.byref(prm), ws.ptr,
                                          ws_bytes, s)
        elif fmt == "w4a16":
            rc = L.lbd_gemm_w4a16(dx.ptr, m, W.kp, b[0].ptr, b[1].ptr, b[2].ptr if len(b) > 2 else None,
                                  n, dy.ptr, C.byref(prm), s)
        elif fmt == "mxfp4":
            rc = L.lbd_gemm_mxfp4(dx.ptr, m, W.kp, b[0].ptr, b[1].ptr, n, dy.ptr, C.byref(prm), s)
        else:
            rc = L.lbd_gemm_w4a8(dx.ptr, m, W.kp, b[0].ptr, b[1].ptr, b[2].ptr if len(b) > 2 else None,
                                 n, dy.ptr, C.byref(prm), ws.ptr, ws_bytes, s)
        dev.check(rc, f"lbd_gemm_{fmt}")
        return rc

    path = launch(0)
    dev.check(L.lb_stream_synchronize(s), "sync")
    y = dy.to_array((m, n), np.float32)
    # every timed graph covers the whole pool at least once and at least MIN_LAUNCHES
    # launches, whatever --steps asks for
    n_launch = timed_launches(steps, len(pool))
    ms = dev.time_launches(launch, n_launch, warmup, graph=graph)
    ms_eager = dev.time_launches(launch, n_launch, warmup, graph=False) if (eager_too and graph) else None
    t = ms * 1e-3
    call_us = call_time(dev, fmt, W, x, pool, layout, n_launch, warmup) if call else None
    return {
        "format": fmt, "M": m, "N": n, "K": k, "cache": "cold" if cold else "hot",
        "path": K.ISA_NAMES.get(path, "?"), "weight_layout": layout, "pool_copies": len(pool),
        "timed_launches": n_launch, "bytes_rotated": int(min(n_launch, len(pool)) * W.nbytes),
        "us_per_call": round(ms * 1e3, 3),
        "us_per_call_eager": None if ms_eager is None else round(ms_eager * 1e3, 3),
        "call_us": call_us, "weight_bytes": int(W.nbytes),
        "weight_gbps": round(W.nbytes / t / 1e9, 1),
        "gflops": round(2.0 * m * n * k / t / 1e9, 1),
        "y": y,
    }


# Configurations of the plain-read sweep: (workgroups, threads, 16-byte loads in flight per thread)
FLOOR_CONFIGS = [(wg, th, ld) for wg in (256, 512, 1024, 2048) for th in (256, 512) for ld in (1, 2, 4, 8)]


def read_floor(dev: Dev, nbytes: int, steps: int, warmup: int, graph: bool = True) -> dict:
    """The fastest plain streaming read (lbd_read_kernel) of `nbytes` over the sweep
    FLOOR_CONFIGS, timed like the GEMMs: cold (one copy of a pool larger than
    COLD_POOL_BYTES per launch) and hot (one buffer), HIP events over a replayed graph."""
    K, L = dev.K, dev.L
    nbytes = (nbytes + 15) // 16 * 16
    copies = max(1, math.ceil(COLD_POOL_BYTES / nbytes))
    pool = [K.DeviceBuffer(nbytes) for _ in range(copies)]
    for i, b in enumerate(pool):
        dev.check(L.lb_memset_d(b.ptr, 0x11 + i % 200, nbytes), "memset")
    sink = K.DeviceBuffer(16)
    rows = []
    for wg, th, ld in FLOOR_CONFIGS:
        row = {"workgroups": wg, "threads": th, "loads": ld}
        for cache in ("cold", "hot"):
            def launch(i, cache=cache):
                b = pool[i % copies] if cache == "cold" else pool[0]
                return dev.check(L.lbd_read_kernel(b.ptr, nbytes, wg, th, ld, sink.ptr, dev.stream), "read kernel")

            n_launch = timed_launches(steps, copies)
            row[f"{cache}_us"] = round(dev.time_launches(launch, n_launch, warmup, graph=graph) * 1e3, 3)
        rows.append(row)
    best = {c: min(rows, key=lambda r: r[f"{c}_us"]) for c in ("cold", "hot")}
    out = {"bytes": nbytes, "pool_copies": copies, "timed_launches": timed_launches(steps, copies), "sweep": rows}
    for c in ("cold", "hot"):
        b = best[c]
        out[c] = {"us": b[f"{c}_us"], "gbps": round(nbytes / (b[f"{c}_us"] * 1e-6) / 1e9, 1),
                  "config": {k: b[k] for k in ("workgroups", "threads", "loads")}}
    log(f"read floor {nbytes} B: cold {out['cold']['us']:.2f} us ({out['cold']['gbps']:.0f} GB/s) "
        f"{out['cold']['config']}, hot {out['hot']['us']:.2f} us ({out['hot']['gbps']:.0f} GB/s) {out['hot']['config']}")
    return out


# The plain read at sizes from the headline's 24.3 MB to 1 GiB (cold), to separate the
# fixed cost of a launch from the streaming rate: t(S) = t0 + S / B, least squares.
FLOOR_SIZE_FACTORS = (1, 2, 4, 8, 16, 32)
FLOOR_SIZE_CONFIGS = [(wg, 512, ld) for wg in (512, 1024, 2048) for ld in (2, 4, 8)]


def read_floor_sizes(dev: Dev, base_bytes: int, steps: int, warmup: int, graph: bool = True) -> dict:
    """The fastest cold plain read (over FLOOR_SIZE_CONFIGS) at base_bytes x
    FLOOR_SIZE_FACTORS and at 1 GiB, and the fit t = t0 + S / B over those sizes."""
    K, L = dev.K, dev.L
    sizes = [(base_bytes * f + 15) // 16 * 16 for f in FLOOR_SIZE_FACTORS] + [1 << 30]
    sink = K.DeviceBuffer(16)
    rows = []
    for nbytes in sizes:
        copies = max(2, math.ceil(COLD_POOL_BYTES / nbytes))
        pool = [K.DeviceBuffer(nbytes) for _ in range(copies)]
        for i, b in enumerate(pool):
            dev.check(L.lb_memset_d(b.ptr, 0x21 + i % 200, nbytes), "memset")
        best = None
        for wg, th, ld in FLOOR_SIZE_CONFIGS:
            def launch(i, wg=wg, th=th, ld=ld):
                b = pool[i % copies]
                return dev.check(L.lbd_read_kernel(b.ptr, nbytes, wg, th, ld, sink.ptr, dev.stream), "read kernel")

            us = dev.time_launches(launch, timed_launches(steps, copies), warmup, graph=graph) * 1e3
            if best is None or us < best[0]:
                best = (us, {"workgroups": wg, "threads": th, "loads": ld})
        rows.append({"bytes": nbytes, "us": round(best[0], 3), "gbps": round(nbytes / (best[0] * 1e-6) / 1e9, 1),
                     "config": best[1], "pool_copies": copies})
        del pool
        log(f"read floor {nbytes / 2**20:8.1f} MiB cold: {best[0]:8.2f} us ({rows[-1]['gbps']:.0f} GB/s) {best[1]}")
    S = np.array([r["bytes"] for r in rows], np.float64)
    T = np.array([r["us"] for r in rows], np.float64) * 1e-6
    slope, t0 = np.polyfit(S, T, 1)  # T = t0 + slope * S
    bw = 1.0 / slope / 1e9
    return {"sizes": rows, "fit": {"t0_us": round(t0 * 1e6, 3), "asymptotic_gbps": round(bw, 1),
                                   "asymptotic_frac_of_peak": round(bw / HBM_PEAK_GBS, 4),
                                   "max_resid_us": round(float(np.max(np.abs(T - (t0 + slope * S)))) * 1e6, 3)}}


PROBE_FORMS = ["v_fmac_f32", "v_fma_f32", "v_add_f32", "v_mul_f32", "v_and_b32", "v_lshrrev_b32",
               "v_cvt_f32_ubyte1", "v_cvt_f32_u32", "v_bfe_u32", "v_perm_b32", "v_and_or_b32", "v_fma_mix_f32",
               "v_dot4_i32_i8", "v_pk_add_f16", "v_cvt_scalef32_pk_f32_fp4", "v_dot2_f32_f16", "v_dot2c_f32_f16",
               "v_cvt_f32_f16"]


BARRIER_MODES = ("atomic counter", "flag per workgroup", "flags + agent release/acquire fences")


def grid_barrier_costs(dev: Dev, cus: int, rounds: int = 200, reps: int = 5) -> dict:
    """Cost of one device-wide barrier inside a launch (lbd_probe_grid_barrier): HIP
    events around one eager launch of `rounds` barriers and around one of none (the
    launch and the clearing of the sync words), median over `reps`, the difference
    divided by `rounds`. A grid whose waits timed out (not every workgroup resident)
    is reported as such instead of a time."""
    L = dev.L
    sync = dev.K.DeviceBuffer((64 + 1024) * 4)
    status = dev.K.DeviceBuffer(4)

    def launch_ms(g, r, mode):
        e0, e1 = dev.event(), dev.event()
        dev.check(L.lb_event_record(e0, dev.stream), "record")
        dev.check(L.lbd_probe_grid_barrier(g, r, mode, sync.ptr, sync.nbytes, status.ptr, dev.stream),
                  "barrier probe")
        dev.check(L.lb_event_record(e1, dev.stream), "record")
        dev.check(L.lb_event_synchronize(e1), "sync")
        ms = dev.elapsed_ms(e0, e1)
        L.lb_event_destroy(e0)
        L.lb_event_destroy(e1)
        return ms, int(status.to_array((1,), np.uint32)[0])

    out = {}
    for g, modes in ((cus, (0, 1, 2)), (cus // 4, (0, 1)), (4 * cus, (0,))):
        for mode in modes:
            base, full, timed_out = [], [], 0
            for _ in range(reps):
                ms0, t0 = launch_ms(g, 0, mode)
                ms1, t1 = launch_ms(g, rounds, mode)
                base.append(ms0)
                full.append(ms1)
                timed_out |= t0 | t1
            key = f"{g} workgroups, {BARRIER_MODES[mode]}"
            if timed_out:
                out[key] = "timed out"
                log(f"grid barrier, {key}: a wait timed out")
                continue
            us = (float(np.median(full)) - float(np.median(base))) * 1e3 / rounds
            out[key] = round(us, 3)
            log(f"grid barrier, {key}: {us:.2f} us per barrier")
    return out


MFMA_VALU_VARIANTS = ["mfma", "valu", "interleaved", "blocks"]


def mfma_valu_sharing(dev: Dev, cus: int, warmup: int) -> dict:
    """Whether one SIMD overlaps int8 MFMA with independent VALU work
    (lbd_probe_mfma_valu): ns per loop iteration (per wave: 8 v_mfma_i32_16x16x64_i8,
    64 v_fmac_f32, or both) at one workgroup per CU of 256 or 512 threads, i.e. one or
    two waves per SIMD. Overlap shows as both near the larger alone; sharing as both
    near the sum."""
    K, L = dev.K, dev.L
    iters = 1024
    out = K.DeviceBuffer(cus * 512 * 4)
    res = {}
    for threads in (256, 512):
        row = {}
        for v, name in enumerate(MFMA_VALU_VARIANTS):
            ms = dev.time_launches(lambda i, v=v, t=threads: dev.check(
                L.lbd_probe_mfma_valu(v, iters, cus, t, out.ptr, dev.stream), "probe"), 5, max(2, warmup // 10))
            row[name] = round(ms * 1e6 / iters, 2)
        key = f"{threads // 256}_wave_per_simd"
        res[key] = row
        log(f"MFMA / VALU on one SIMD, {key}: " + ", ".join(f"{k} {v:.1f}" for k, v in row.items()) +
            f" ns per iteration (sum of the two alone {row['mfma'] + row['valu']:.1f})")
    return res


def machine_facts(dev: Dev, warmup: int) -> dict:
    """The device facts the kernel designs rest on, measured by the library's probe
    kernels (lb_probe.hip): the issue cost of single VALU instruction forms (16 waves
    per CU, eight independent registers, 32 instructions per loop iteration) and the
    fixed cost of a launch (an
    empty kernel over the same grid, graph replay)."""
    K, L = dev.K, dev.L
    cus = K.device_info()["compute_units"]
    wgs, iters, waves_per_cu = 2 * cus, 1024, 16  # 32 instructions per iteration
    assert L.lbd_probe_forms() == len(PROBE_FORMS)
    out = K.DeviceBuffer(wgs * 512 * 4)
    rates = {}
    for op, name in enumerate(PROBE_FORMS):
        ms = dev.time_launches(lambda i, op=op: dev.check(L.lbd_probe_valu(op, iters, wgs, out.ptr, dev.stream),
                                                          "probe"), 5, max(2, warmup // 10))
        rates[name] = round(ms * 1e6 / (waves_per_cu * iters * 32), 4)
        log(f"{name:28s} {rates[name]:.3f} ns per wave64 instruction per CU")
    empty = {}
    for g in (cus, 2 * cus):
        ms = dev.time_launches(lambda i, g=g: dev.check(L.lbd_empty_kernel(g, dev.stream), "empty"), 200, warmup)
        empty[f"{g}x512"] = round(ms * 1e3, 3)
        log(f"empty kernel {g} x 512 threads: {empty[f'{g}x512']:.2f} us per graph-replayed launch")
    barrier = grid_barrier_costs(dev, cus)
    sharing = mfma_valu_sharing(dev, cus, warmup)
    return {"valu_ns_per_wave_instruction_per_cu": rates, "empty_launch_us": empty, "grid_barrier_us": barrier,
            "mfma_valu_ns_per_iteration": sharing,
            "probe": {"workgroups": wgs, "threads": 512, "iters": iters, "instructions_per_iter": 32,
                      "independent_registers": 8}}


def call_time(dev: Dev, fmt: str, W, x: np.ndarray, pool, layout: str, n_calls: int, warmup: int) -> float:
    """Median wall time (us) of one Python call lowbit_amd.gemm_<fmt>(x, handle) on
    resident weights, rotating over the same pool of copies as the kernel timing: the
    whole synchronous call through ctypes (pad X, X to the device, the GEMM, Y back),
    as the reference times its calls (src/lowbit/bench.py:116-124)."""
    K = dev.K
    handles = []
    for b in pool:
        if fmt == "mxfp4":
            h = K.DeviceMXFP4Weights(None, None, W.n, W.kp, W.k, W.nbytes)
            if layout == "t16":
                h.t16 = (b[0], b[1])
            else:
                h.qw, h.e8m0 = b[0], b[1]
        else:
            h = K.DeviceInt4Weights(None, None, None, W.n, W.kp, W.k, W.nbytes)
            if layout == "t16f8":
                h.t16f8, h.zmax = (b[0], b[1]), 8 if W.zeros is None else int(W.zeros.max(initial=0))
            elif layout == "t16":
                h.t16 = (b[0], b[1], b[2])
            else:
                h.qw, h.scales, h.zeros = b[0], b[1], (b[2] if len(b) > 2 else None)
        handles.append(h)
    fn = K.GEMMS[fmt]
    # warm-up by time as well as by count: the first format timed in a process ran
    # ~23 us slower per call after a 20-call warm-up (host and device clocks ramping)
    i, t_end = 0, time.perf_counter() + 0.3
    while i < max(3, warmup) or time.perf_counter() < t_end:
        fn(x, handles[i % len(handles)])
        i += 1
    ts = []
    for i in range(n_calls):
        h = handles[i % len(handles)]
        t0 = time.perf_counter()
        fn(x, h)
        ts.append(time.perf_counter() - t0)
    return round(float(np.median(ts)) * 1e6, 2)


def call_time_host(dev: Dev, fmt: str, W, x: np.ndarray, n_calls: int, implicit: bool) -> float:
    """Median wall time (us) of lowbit_amd.gemm_<fmt>(x, W) on the host container W, the
    call the reference's linear layers make (src/lowbit/model.py:139-141): with implicit
    residency (the container's device copy, made on its first call, reused), or through
    the host-pointer ABI (lb_gemm_*: the weights cross PCIe on every call, as a binary
    drop-in of the reference's library behaves)."""
    K = dev.K
    fn = K.GEMMS[fmt]
    with K.implicit_residency(implicit):
        i, t_end = 0, time.perf_counter() + 0.3
        while i < 3 or time.perf_counter() < t_end:
            fn(x, W)
            i += 1
        ts = []
        for _ in range(n_calls):
            t0 = time.perf_counter()
            fn(x, W)
            ts.append(time.perf_counter() - t0)
    return round(float(np.median(ts)) * 1e6, 2)


def rel_err(fmt: str, W, x, y) -> float:
    """max|y - ref| / max|ref| against the float64 C oracle (the reference's bench check)."""
    from lowbit_amd import formats as F
    from oracle import cref
    xp = F.pad_acts(x, W.kp)
    if fmt == "w4a16":
        ref = cref.c_gemm_w4a16(xp, W.qw, W.scales, W.zeros)
    elif fmt == "mxfp4":
        ref = cref.c_gemm_mxfp4(xp, W.qw, W.e8m0)
    else:
        a = F.quantize_act_int8(xp)
        ref, _ = cref.c_gemm_w4a8(a.xq, a.scale, a.gsum, W.qw, W.scales, W.zeros)
    return float(np.max(np.abs(y - ref)) / (np.max(np.abs(ref)) + 1e-30))


# ------------------------------------------------------------------ CPU baseline

def host_llc_bytes() -> int:
    best = 0
    for idx in Path("/sys/devices/system/cpu/cpu0/cache").glob("index*"):
        try:
            txt = (idx / "size").read_text().strip()
        except OSError:
            continue
        mult = {"K": 1 << 10, "M": 1 << 20, "G": 1 << 30}.get(txt[-1], 1)
        best = max(best, (int(txt[:-1]) if txt[-1] in "KMG" else int(txt)) * mult)
    return best or 32 << 20


def cpu_model() -> str:
    try:
        for ln in Path("/proc/cpuinfo").read_text().splitlines():
            if ln.startswith("model name"):
                return ln.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def host_cpu() -> dict:
    """nproc, the CPUs this process may use, the lscpu model name, sockets and cores
    per socket (the run metadata the reference's bench records, src/lowbit/bench.py:280-291)."""
    info = {"nproc": os.cpu_count(), "affinity": len(os.sched_getaffinity(0)), "model": cpu_model(),
            "sockets": None, "cores_per_socket": None}
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for ln in out.splitlines():
            key, _, val = ln.partition(":")
            if key.strip() == "Socket(s)":
                info["sockets"] = int(val.strip())
            elif key.strip() == "Core(s) per socket":
                info["cores_per_socket"] = int(val.strip())
            elif key.strip() == "Model name":
                info["model"] = val.strip()
    except (OSError, ValueError, subprocess.SubprocessError):
        pass
    info["avx512_vnni"] = "avx512_vnni" in Path("/proc/cpuinfo").read_text() if Path("/proc/cpuinfo").exists() else None
    return info


# The CPU share a one-GPU job may use on the GPU boxes (their worker pools are sized
# to it): the baseline never runs more threads than this.
CPU_SHARE = 16


def cpu_threads(info: dict) -> int:
    """Threads for the multi-thread leg: the cores of one socket, capped by the CPUs
    this process may use and by the job's CPU share."""
    one_socket = info.get("cores_per_socket") or info["affinity"]
    return max(1, min(one_socket, info["affinity"], CPU_SHARE))


def _busy_s() -> float:
    """CPU-seconds every tenant of this host has spent non-idle (Linux /proc/stat)."""
    v = [int(t) for t in Path("/proc/stat").read_text().splitlines()[0].split()[1:]]
    return (sum(v) - v[3] - v[4]) / os.sysconf("SC_CLK_TCK")


def _self_s() -> float:
    t = os.times()
    return t.user + t.system  # every thread of this process


def timed_uncontended(run, max_other: float = 1.0, attempts: int = 3):
    """Call run() (which returns a list of call times) up to `attempts` times until the
    other processes on the host used at most `max_other` cores meanwhile, waiting a
    second between attempts; keep the least contended attempt. Returns (times, other
    tenants' cores during it, attempts made). The reference guards its CPU timings the
    same way (src/lowbit/bench.py:88-113)."""
    best = None
    for a in range(1, attempts + 1):
        try:
            b0, s0, w0 = _busy_s(), _self_s(), time.perf_counter()
        except (OSError, ValueError, IndexError):
            return run(), None, a
        ts = run()
        b1, s1, w1 = _busy_s(), _self_s(), time.perf_counter()
        other = max(0.0, ((b1 - b0) - (s1 - s0)) / max(1e-9, w1 - w0))
        if best is None or other < best[1]:
            best = (ts, other, a)
        if other <= max_other:
            break
        time.sleep(1.0)
    return best[0], round(best[1], 3), best[2]


def cpu_baseline_run(budget_s: float, info: dict) -> dict | None:
    """Every decode format of the reference's own C library (oracle/_ref) at M=1
    11008x4096, at 1 thread and at cpu_threads(info) threads, weights rotated past 2x
    the host LLC, median of >= 3 calls after a warm-up (src/lowbit/bench.py:116-124).
    Runs in a child process started with OMP_PROC_BIND=close, OMP_PLACES=cores;
    `info` is the parent's host_cpu(): once the OpenMP runtime has bound the child's
    first thread to one core, the child's own affinity mask holds that core alone."""
    from dataclasses import replace

    import lowbit_amd as lb
    from lowbit_amd import formats as F
    from oracle import cref
    L = cref.ref_lib()
    if L is None:
        return None
    threads = cpu_threads(info)
    rng = np.random.default_rng(0)
    m, n, k = DECODE
    w = rng.standard_normal((n, k)).astype(np.float32)
    x = rng.standard_normal((m, k)).astype(np.float32)
    w4 = lb.quantize_int4(w, asym=True)
    weights = {"w4a8": w4, "w4a16": w4, "mxfp4": lb.quantize_mxfp4(w)}
    llc = host_llc_bytes()
    legs = {}
    kind_id = {"w4a16": 0, "mxfp4": 1, "w4a8": 2}
    isa_names = {0: "scalar", 1: "avx2", 2: "avx512"}
    for fmt, W in weights.items():
        copies = min(max(1, math.ceil(max(2 * llc, 512 << 20) / W.nbytes)), max(1, (3 << 30) // W.nbytes))
        if fmt == "mxfp4":
            pool = [W] + [replace(W, qw=W.qw.copy(), e8m0=W.e8m0.copy()) for _ in range(copies - 1)]
        else:
            pool = [W] + [replace(W, qw=W.qw.copy(), scales=W.scales.copy(),
                                  zeros=None if W.zeros is None else W.zeros.copy()) for _ in range(copies - 1)]
        xp = F.pad_acts(x, W.kp)
        y = np.empty((m, n), np.float32)
        for nt in sorted({1, threads}):
            p = cref.RefParams(-1, 0, 0, 0, 0, 0, nt)

            def call(i):
                wi = pool[i % len(pool)]
                if fmt == "w4a8":
                    rc = L.lb_gemm_w4a8(xp, m, wi.kp, wi.qw, wi.scales, cref.zp(wi.zeros), n, y, C.byref(p))
                elif fmt == "w4a16":
                    rc = L.lb_gemm_w4a16(xp, m, wi.kp, wi.qw, wi.scales, cref.zp(wi.zeros), n, y, C.byref(p))
                else:
                    rc = L.lb_gemm_mxfp4(xp, m, wi.kp, wi.qw, wi.e8m0, n, y, C.byref(p))
                assert rc >= 0, rc

            call(0)

            def run(call=call):
                ts, i, t_end = [], 1, time.perf_counter() + budget_s / (2 * (len(weights) + 1))
                while len(ts) < 3 or (time.perf_counter() < t_end and len(ts) < 2000):
                    t0 = time.perf_counter()
                    call(i)
                    ts.append(time.perf_counter() - t0)
                    i += 1
                return ts

            ts, other, att = timed_uncontended(run)
            med = float(np.median(ts))
            isa = L.lb_effective_isa(kind_id[fmt], -1)
            legs[f"{fmt}_{nt}t"] = {"us": round(med * 1e6, 1), "weight_gbps": round(W.nbytes / med / 1e9, 2),
                                    "reps": len(ts), "threads": nt,
                                    "isa": isa_names.get(isa, isa) + ("-vnni" if fmt == "w4a8" and isa == 2 else ""),
                                    "pool_copies": copies, "other_tenant_cores": other, "attempts": att}
    # the memory floor the reference publishes beside its kernels: numpy fp32 X @ W^T on
    # the dense weights (src/lowbit/bench.py numpy fp32 rows, README.md:85), same rotation
    legs.update(numpy_fp32_floor(w, x, llc, threads, budget_s / (len(weights) + 1)))
    return {"legs": legs, "threads": threads, "host": info, "llc_bytes": llc,
            "omp_proc_bind": os.environ.get("OMP_PROC_BIND"), "omp_places": os.environ.get("OMP_PLACES")}


def numpy_fp32_floor(w: np.ndarray, x: np.ndarray, llc: int, threads: int, budget_s: float) -> dict:
    """numpy fp32 y = x @ w.T (BLAS sgemv) at 1 thread and `threads` threads, the dense
    fp32 weights rotated past 2x the host LLC; fp32 weight bytes per second."""
    try:
        from threadpoolctl import threadpool_limits
    except ImportError:
        return {}
    copies = min(max(1, math.ceil(max(2 * llc, 512 << 20) / w.nbytes)), max(1, (3 << 30) // w.nbytes))
    pool = [w] + [w.copy() for _ in range(copies - 1)]
    out = {}
    for nt in sorted({1, threads}):
        with threadpool_limits(limits=nt, user_api="blas"):
            _ = x @ pool[0].T

            def run():
                ts, i, t_end = [], 1, time.perf_counter() + budget_s / 2
                while len(ts) < 3 or (time.perf_counter() < t_end and len(ts) < 2000):
                    t0 = time.perf_counter()
                    _ = x @ pool[i % copies].T
                    ts.append(time.perf_counter() - t0)
                    i += 1
                return ts

            ts, other, att = timed_uncontended(run)
        med = float(np.median(ts))
        out[f"numpy_fp32_{nt}t"] = {"us": round(med * 1e6, 1), "weight_gbps": round(w.nbytes / med / 1e9, 2),
                                    "reps": len(ts), "threads": nt, "isa": "numpy fp32 (BLAS sgemv)",
                                    "pool_copies": copies, "other_tenant_cores": other, "attempts": att}
    return out


def cpu_baseline(budget_s: float) -> dict | None:
    """The CPU baseline of the JSON line, measured by cpu_baseline_run in a child
    process (OpenMP reads its binding from the environment at start-up)."""
    env = dict(os.environ, OMP_PROC_BIND="close", OMP_PLACES="cores")
    r = subprocess.run([sys.executable, str(Path(__file__).resolve()), "--cpu-baseline-only",
                        "--cpu-seconds", str(budget_s), "--cpu-host", json.dumps(host_cpu())],
                       capture_output=True, text=True, env=env, timeout=600)
    if r.returncode != 0:
        log(f"cpu baseline child failed (rc {r.returncode}): {r.stderr[-2000:]}")
        return None
    res = json.loads(r.stdout.strip().splitlines()[-1])
    if res is None:
        return None
    nt = res["threads"]
    head = res["legs"][f"w4a8_{nt}t"]
    one = res["legs"]["w4a8_1t"]
    h = res["host"]
    return {
        "value": head["weight_gbps"],
        "unit": "weight GB/s",
        "cores": nt,
        "kind": "reference",
        "sample": (f"reference C lb_gemm_w4a8 (oracle/_ref, {head['isa']} path), M=1 N=11008 K=4096 int4 g128 "
                   f"asym, {head['pool_copies']} rotating weight copies (> 2x the {res['llc_bytes'] >> 20} MiB "
                   f"LLC), median of {head['reps']} calls: {head['us']:.0f} us at {nt} threads "
                   f"(OMP_PROC_BIND=close), {one['us']:.0f} us at 1 thread ({one['weight_gbps']:.2f} GB/s); host "
                   f"{h['model']}, {h['sockets']} socket(s) x {h['cores_per_socket']} cores, nproc "
                   f"{h['nproc']}, {h['affinity']} CPUs usable, threads capped at one socket and the job's "
                   f"{CPU_SHARE}-CPU share; other tenants used {head.get('other_tenant_cores')} cores during "
                   f"the timed calls (attempt {head.get('attempts')} of at most 3)"),
        "other_tenant_cores": head.get("other_tenant_cores"),
        "legs": res["legs"],
        "host": h,
    }


# Qwen2.5-0.5B-shaped decoder, 64-token random prompt, 128 greedy
# decode steps (src/lowbit/e2e.py:119-122,194: tok/s = decode forwards / decode time).
# The reference's published decode tok/s on its Xeon (README.md:199-200, real weights,
# 1 / 4 threads).
DECODER_REF_TOKS = {"w4a8": (25.87, 63.80), "mxfp4": (19.74, 50.13)}


def measure_decoder(backends, n_decode: int = 128, prompt_len: int = 64, reps: int = 3, graph: bool = True) -> dict:
    """Greedy decode of the config-5 decoder with random weights (the shapes of
    Qwen2.5-0.5B), device-resident, each decode step one replayed HIP graph
    (graph=False: the same kernels launched one by one)."""
    from lowbit_amd import model as DM
    cfg = DM.qwen2_config()
    t0 = time.perf_counter()
    W = DM.random_weights(cfg, seed=0, float32_draws=True)
    log(f"decoder: random weights in {time.perf_counter() - t0:.1f} s")
    prompt = np.random.default_rng(0).integers(0, cfg.vocab_size, prompt_len).tolist()
    out = {}
    for be in backends:
        m = DM.Model(cfg, W, be, max_tokens=prompt_len)
        m.generate(prompt[:8], 4, graph=graph)  # warm-up: kernels loaded, t16 copies built
        best = None
        for _ in range(reps):
            tim = {}
            toks = m.generate(prompt, n_decode + 1, timings=tim, graph=graph)
            dec = tim["decode_s"] / tim["decode_forwards"]
            if best is None or dec < best[0]:
                best = (dec, tim["prefill_s"], toks)
        dec, pre, toks = best
        wb = m.linear_weight_bytes
        ref1, ref4 = DECODER_REF_TOKS[be]
        out[be] = {
            "decode_tok_s": round(1.0 / dec, 1), "ms_per_token": round(dec * 1e3, 4),
            "prefill_tok_s": round(prompt_len / pre, 1), "prompt": prompt_len, "decode_steps": n_decode,
            "fused_decode": m.fused, "graph": graph, "linear_weight_bytes": wb,
            # weight stream per token against HBM: the bound is wb / 8 TB/s
            "weight_gbps": round(wb / dec / 1e9, 1), "hbm_frac": round(wb / dec / 1e9 / HBM_PEAK_GBS, 4),
            "hbm_bound_tok_s": round(HBM_PEAK_GBS * 1e9 / wb, 1),
            "reference_cpu_tok_s": {"1_thread": ref1, "4_threads": ref4},
            "first_tokens": toks[:4],
        }
        log(f"decoder {be}: decode {1.0 / dec:8.1f} tok/s ({dec * 1e3:.3f} ms/token, "
            f"{wb / dec / 1e9:.0f} GB/s of weights), prefill {prompt_len / pre:8.1f} tok/s")
        del m
    return out


def traffic_bytes() -> int | None:
    """HBM bytes per launch of the headline kernel, from the committed counter summary."""
    if not TRAFFIC_FILE.exists():
        return None
    for ln in TRAFFIC_FILE.read_text().splitlines():
        if ln.startswith("traffic_bytes_per_launch:"):
            return int(float(ln.split(":", 1)[1]))
    return None


def traced_kernel_us() -> float | None:
    """Mean kernel-trace duration of the headline kernel's timed dispatches, from the
    committed trace summary (a traced run launches every kernel on its own)."""
    if not TRACE_FILE.exists():
        return None
    for ln in TRACE_FILE.read_text().splitlines():
        if ln.startswith("traced_kernel_mean_us:"):
            return float(ln.split(":", 1)[1])
    return None


# ------------------------------------------------------------------ main

def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--cpu-seconds", type=float, default=6.0, help="CPU baseline time budget")
    ap.add_argument("--no-graph", action="store_true", help="time plain launches instead of a graph replay")
    ap.add_argument("--only-headline", action="store_true", help="measure only the headline W4A8 decode")
    ap.add_argument("--no-decoder", action="store_true", help="skip the config-5 decoder (tokens/s)")
    ap.add_argument("--only-decoder", action="store_true",
                    help="measure only the config-5 decoder and print its JSON (for kernel traces)")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run the plain 16-byte copy kernel 5 times over MIB MiB (the reference "
                         "point that scales the FETCH_SIZE / WRITE_SIZE counters), then exit")
    ap.add_argument("--read-floor", action="store_true",
                    help="only sweep the plain streaming read of the headline weight bytes (cold and hot) "
                         "and print its JSON")
    ap.add_argument("--no-floor", action="store_true", help="skip the plain-read floor sweep")
    ap.add_argument("--no-call-time", action="store_true",
                    help="skip the synchronous Python call timings (kernel traces of the timed launches only)")
    ap.add_argument("--batch-m", type=int, default=BATCH[0], metavar="M",
                    help="rows of the hot batch GEMMs (default 64, the BASELINE shape)")
    ap.add_argument("--shape", default=None, metavar="N,K",
                    help="only time the three formats' decode (M = 1, cold) and batch (--batch-m rows, hot) "
                         "GEMMs at N x K and print their JSON (profiles of the other benchmark shapes, e.g. "
                         "4096,11008); no headline line")
    ap.add_argument("--machine-facts", action="store_true",
                    help="only measure the device facts the kernels are designed around (VALU issue cost per "
                         "instruction form, launch cost, the plain-read floor) and print their JSON")
    ap.add_argument("--cpu-baseline-only", action="store_true", help=argparse.SUPPRESS)
    ap.add_argument("--cpu-host", default=None, help=argparse.SUPPRESS)
    args = ap.parse_args()
    if args.cpu_baseline_only:
        print(json.dumps(cpu_baseline_run(args.cpu_seconds, json.loads(args.cpu_host) if args.cpu_host
                                          else host_cpu())), flush=True)
        return 0
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}): the hot path has no "
              "multi-GPU part in this build; run with --gpus 1.", file=sys.stderr)
        return 2
    if int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py is single-process, single-GPU", file=sys.stderr)
        return 2

    import lowbit_amd as lb

    dev = Dev()
    if args.copy_calibration:
        nbytes = args.copy_calibration << 20
        src, dst = dev.K.DeviceBuffer(nbytes), dev.K.DeviceBuffer(nbytes)
        for _ in range(5):
            dev.check(dev.L.lbd_copy_kernel(dst.ptr, src.ptr, nbytes, dev.stream), "copy kernel")
        dev.check(dev.L.lb_stream_synchronize(dev.stream), "sync")
        print(json.dumps({"copy_calibration_bytes": nbytes, "launches": 5}), flush=True)
        return 0
    info = dev.K.cpu_info()
    log(f"device {info.get('arch')} with {info.get('compute_units')} CUs")
    graph = not args.no_graph
    headline_bytes = 11008 * (4096 // 2 + (4096 // 128) * 5)  # int4 g128 asym weights of the headline
    if args.read_floor:
        print(json.dumps({"read_floor": read_floor(dev, headline_bytes, args.steps, args.warmup, graph),
                          "read_floor_sizes": read_floor_sizes(dev, headline_bytes, args.steps, args.warmup,
                                                               graph)}), flush=True)
        return 0
    if args.machine_facts:
        facts = machine_facts(dev, args.warmup)
        facts["read_floor"] = read_floor(dev, headline_bytes, args.steps, args.warmup, graph)
        print(json.dumps({"machine_facts": facts}), flush=True)
        return 0
    if args.only_decoder:
        print(json.dumps({"decoder": measure_decoder(["w4a8", "mxfp4"], graph=graph)}), flush=True)
        return 0
    if args.shape:
        n_s, k_s = (int(v) for v in args.shape.split(","))
        rng = np.random.default_rng(0)
        w = rng.standard_normal((n_s, k_s)).astype(np.float32)
        packed = {"int4": lb.quantize_int4(w, asym=True), "mxfp4": lb.quantize_mxfp4(w)}
        runs = {}
        for mm, cold in ((1, True), (args.batch_m, False)):
            xs = rng.standard_normal((mm, k_s)).astype(np.float32)
            for fmt in ["w4a8", "w4a16", "mxfp4"]:
                W = packed["mxfp4" if fmt == "mxfp4" else "int4"]
                r = measure(dev, fmt, (mm, n_s, k_s), W, xs, cold=cold, steps=args.steps,
                            warmup=args.warmup, graph=graph, call=False)
                r["max_rel_err"] = float(f"{rel_err(fmt, W, xs, r.pop('y')):.3g}")
                runs[f"{fmt}_m{mm}"] = r
                log(f"{fmt:6s} {mm}x{n_s}x{k_s} {'cold' if cold else 'hot'}: {r['us_per_call']:8.2f} us  "
                    f"path {r['path']}  rel err {r['max_rel_err']}")
        print(json.dumps({"shape_runs": runs}), flush=True)
        return 0
    rng = np.random.default_rng(0)
    results = {}

    # decode: all three formats at 1 x 11008 x 4096, cold
    m, n, k = DECODE
    w = rng.standard_normal((n, k)).astype(np.float32)
    x = rng.standard_normal((m, k)).astype(np.float32)
    w4 = lb.quantize_int4(w, asym=True)
    mx = lb.quantize_mxfp4(w)
    order = ["w4a8"] if args.only_headline else ["w4a8", "w4a16", "mxfp4"]
    for fmt in order:
        W = mx if fmt == "mxfp4" else w4
        r = measure(dev, fmt, DECODE, W, x, cold=True, steps=args.steps, warmup=args.warmup, graph=graph,
                    eager_too=(fmt == "w4a8"), call=not args.no_call_time)
        r["max_rel_err"] = float(f"{rel_err(fmt, W, x, r.pop('y')):.3g}")
        r["hbm_frac"] = round(r["weight_gbps"] / HBM_PEAK_GBS, 4)
        # the same call on the host container: implicit residency, and the pointer ABI
        if not args.no_call_time:
            r["call_us_host_container"] = call_time_host(dev, fmt, W, x, 200, implicit=True)
            r["call_us_pointer_abi"] = call_time_host(dev, fmt, W, x, 20, implicit=False)
        results[f"{fmt}_decode"] = r
        calls = ("" if args.no_call_time else
                 f"call through ctypes {r['call_us']:.1f} us (host container {r['call_us_host_container']:.1f}, "
                 f"pointer ABI {r['call_us_pointer_abi']:.0f})  ")
        eager = "" if r["us_per_call_eager"] is None else f"(plain launches {r['us_per_call_eager']:.2f} us)  "
        log(f"{fmt:6s} M=1 cold: {r['us_per_call']:8.2f} us  {eager}{r['weight_gbps']:7.1f} GB/s "
            f"({100 * r['hbm_frac']:.1f}% HBM)  path {r['path']}  rel err {r['max_rel_err']}  "
            f"{calls}({r['timed_launches']} launches, {r['bytes_rotated'] >> 20} MiB rotated)")

    # batch: M=64, hot (the reference measures batch shapes hot, src/lowbit/bench.py:167);
    # --batch-m selects another M (the counter profiles of the M = 16 kernels)
    if not args.only_headline:
        mb, nb, kb = args.batch_m, BATCH[1], BATCH[2]
        xb = rng.standard_normal((mb, kb)).astype(np.float32)
        for fmt in ["w4a8", "w4a16", "mxfp4"]:
            W = mx if fmt == "mxfp4" else w4
            r = measure(dev, fmt, (mb, nb, kb), W, xb, cold=False, steps=args.steps,
                        warmup=max(2, args.warmup // 4), graph=graph, call=not args.no_call_time)
            r["max_rel_err"] = float(f"{rel_err(fmt, W, xb, r.pop('y')):.3g}")
            if fmt == "w4a8":
                r["mfma"] = "int8"
                r["mfma_frac"] = round(r["gflops"] / 1e3 / INT8_PEAK_TOPS, 4)
            elif r["weight_layout"] in ("t16", "t16f8"):
                # MXFP4: three bf16 products per fp32 product; W4A16: two float16
                # products per product (the same dense peak for both types)
                terms = F16X2_TERMS if fmt == "w4a16" else BF16X3_TERMS
                r["mfma"] = "f16x2" if fmt == "w4a16" else "bf16x3"
                r["mfma_frac"] = round(terms * r["gflops"] / 1e3 / BF16_PEAK_TFLOPS, 4)
                r["fp32_equiv_frac"] = round(r["gflops"] / 1e3 / FP32_PEAK_TFLOPS, 4)
            else:
                r["mfma"] = "fp32"
                r["mfma_frac"] = round(r["gflops"] / 1e3 / FP32_PEAK_TFLOPS, 4)
            results[f"{fmt}_m{mb}"] = r
            log(f"{fmt:6s} M={mb} hot: {r['us_per_call']:8.2f} us  {r['gflops']:9.1f} GFLOP/s "
                f"({100 * r['mfma_frac']:.1f}% of {r['mfma']} MFMA peak)  path {r['path']}" +
                ("" if r["call_us"] is None else f"  call through ctypes {r['call_us']:.1f} us"))

    floor = sizes = None
    if not args.no_floor:
        floor = read_floor(dev, headline_bytes, args.steps, args.warmup, graph)
        for kk, r in results.items():
            if r["M"] == 1:
                r["frac_of_read_floor"] = round(floor["cold"]["us"] / r["us_per_call"], 4)
        sizes = read_floor_sizes(dev, headline_bytes, args.steps, args.warmup, graph)

    decoder = None
    if not (args.only_headline or args.no_decoder):
        decoder = measure_decoder(["w4a8", "mxfp4"], graph=graph)

    head = results["w4a8_decode"]
    t_launch_s = head["us_per_call"] * 1e-6
    # algorithmic bytes of one launch: packed weights + fp32 X + fp32 Y
    algo_bytes = head["weight_bytes"] + 4 * k * m + 4 * n * m
    achieved = algo_bytes / t_launch_s / 1e9
    eager = None
    if head["us_per_call_eager"]:
        a_e = algo_bytes / (head["us_per_call_eager"] * 1e-6) / 1e9
        # plain launches, the way a kernel trace sees them (durations comparable method for method)
        eager = {"us_per_launch": head["us_per_call_eager"], "achieved": round(a_e, 1),
                 "frac": round(a_e / HBM_PEAK_GBS, 4)}
    cpu = None
    if not args.no_cpu:
        try:
            cpu = cpu_baseline(args.cpu_seconds)
        except Exception as e:  # the baseline is reported, never required
            log(f"cpu baseline failed: {e}")
    line = {
        "metric": "weight GB/s (%HBM peak) at 1x11008x4096; GFLOP/s at M=64, per format",
        "value": head["weight_gbps"],
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(head["us_per_call"] * 1e-3, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic",
        "config": {"workload": "W4A8 decode GEMV, M=1 N=11008 K=4096, int4 g128 asym weights, int8 "
                               "per-token activations quantized in-call, cold (weights rotated over "
                               f"{head['pool_copies']} HBM copies), HIP-graph replay",
                   "M": m, "N": n, "K": k, "format": "w4a8", "cache": "cold", "parallelism": "single GPU",
                   "timing": "graph" if graph else "launch"},
        "hbm_frac": head["hbm_frac"],
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic_bytes(),
                     "algorithmic_bytes": int(algo_bytes),
                     # the fastest plain read of the same weight bytes, timed the same way
                     "read_floor": None if floor is None else {
                         "cold_us": floor["cold"]["us"], "cold_gbps": floor["cold"]["gbps"],
                         "hot_us": floor["hot"]["us"], "hot_gbps": floor["hot"]["gbps"],
                         "config": floor["cold"]["config"],
                         "frac_of_floor": round(floor["cold"]["us"] / head["us_per_call"], 4),
                         "size_sweep": sizes,
                         "frac_of_asymptotic": None if sizes is None else round(
                             achieved / sizes["fit"]["asymptotic_gbps"], 4),
                         # the launch's bytes over its time past the fitted fixed cost t0
                         "streaming_frac_of_peak": None if sizes is None else round(
                             algo_bytes / ((head["us_per_call"] - sizes["fit"]["t0_us"]) * 1e-6) / 1e9
                             / HBM_PEAK_GBS, 4)},
                     "eager": eager,
                     "traced": None if traced_kernel_us() is None else {
                         "kernel_us": traced_kernel_us(),
                         "frac": round(algo_bytes / (traced_kernel_us() * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                         "source": TRACE_FILE.name}},
        "timed_launches": head["timed_launches"],
        "bytes_rotated": head["bytes_rotated"],
        "call_us": head["call_us"],
        "call_us_host_container": head.get("call_us_host_container"),
        "call_us_pointer_abi": head.get("call_us_pointer_abi"),
        "cpu_baseline": cpu,
        "per_format": {kk: {f: v for f, v in vv.items() if f not in ("N", "K")} for kk, vv in results.items()},
        "decoder": decoder,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
