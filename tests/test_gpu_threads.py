"""Concurrent calls from several host threads (GPU).

include/lowbit_hip.h promises that the lb_* entry points may be called from several
threads at once: each thread has its own stream and staging memory. The reference's
ctypes binding releases the GIL around every call (src/lowbit/kernels.py:46-74), so
Python callers do run them concurrently. Here eight threads call the host-pointer
ABI (lb_gemm_*), the resident-weight path (gemm_* on to_device handles) and host
containers made resident on first use (one device copy shared by every thread) on
different shapes and formats, interleaved; every result must equal, bit for bit,
the same call made alone beforehand (the kernels are deterministic).
"""
import threading
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest

import lowbit_amd as lb
from lowbit_amd import kernels as K

pytestmark = pytest.mark.gpu

# (format, M, N, K): both regimes, odd shapes, the headline shape
CASES = [("w4a8", 1, 11008, 4096), ("w4a16", 1, 4096, 4096), ("mxfp4", 1, 3000, 1000),
         ("w4a8", 64, 4096, 4096), ("w4a16", 17, 700, 1152), ("mxfp4", 40, 2048, 4096),
         ("w4a8", 3, 5000, 640), ("w4a16", 1, 151936, 128)]


def _operands(rng, fmt, m, n, k):
    x = rng.standard_normal((m, k)).astype(np.float32)
    w = rng.standard_normal((n, k)).astype(np.float32)
    W = lb.quantize_mxfp4(w) if fmt == "mxfp4" else lb.quantize_int4(w, asym=(fmt == "w4a8"))
    return x, W, lb.to_device(W)


def _pointer(fn):
    """fn through the host-pointer ABI (lb_gemm_*) on the calling thread."""
    def call(x, w):
        with K.implicit_residency(False):
            return fn(x, w)
    return call


def test_concurrent_calls_match_serial(rng):
    ops = [_operands(rng, *c) for c in CASES]
    calls = []
    for (fmt, m, n, k), (x, W, D) in zip(CASES, ops):
        fn = K.GEMMS[fmt]
        calls.append((f"{fmt} {m}x{n}x{k} host", _pointer(fn), x, W))
        calls.append((f"{fmt} {m}x{n}x{k} implicit", fn, x, W))
        calls.append((f"{fmt} {m}x{n}x{k} resident", fn, x, D))
    serial = {name: fn(x, w).copy() for name, fn, x, w in calls}
    paths = {}
    errors = []
    lock = threading.Lock()

    def worker(tid):
        # each thread walks the calls in its own order, several times
        order = np.random.default_rng(tid).permutation(len(calls))
        for rep in range(3):
            for i in order:
                name, fn, x, w = calls[i]
                y = fn(x, w)
                with lock:
                    paths.setdefault(name, set()).add(K.last_path())
                if not np.array_equal(y, serial[name]):
                    errors.append(f"thread {tid} rep {rep}: {name} differs from the serial result")

    with ThreadPoolExecutor(max_workers=8) as ex:
        list(ex.map(worker, range(8)))
    assert not errors, errors[:5]
    # last_path() is per thread: every thread saw one path per call
    assert all(len(p) == 1 for p in paths.values()), paths


def test_threads_share_one_resident_matrix(rng):
    """Threads that share a resident handle whose matrix-core tiles are not built yet:
    the t16 repack runs once and every thread's result equals the serial one."""
    x = rng.standard_normal((32, 4096)).astype(np.float32)
    W = lb.quantize_int4(rng.standard_normal((2048, 4096)).astype(np.float32), asym=True)
    want = K.gemm_w4a8(x, W)
    D = lb.to_device(W)
    assert D.t16 is None
    with ThreadPoolExecutor(max_workers=6) as ex:
        outs = list(ex.map(lambda _: K.gemm_w4a8(x, D), range(12)))
    for y in outs:
        np.testing.assert_array_equal(y, want)
