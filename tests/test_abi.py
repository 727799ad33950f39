"""The C-ABI library and its host logic (CPU; no kernel is launched).

The library must load, export every function include/lowbit_hip.h declares,
and reject bad shapes and tiles with the reference's return codes before it
touches a device.
"""
import ctypes as C
import re
import subprocess
from pathlib import Path

import numpy as np
import pytest

import lowbit_amd as lb
from lowbit_amd import _build
from lowbit_amd import kernels as K

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "lowbit_hip.h"


def header_functions() -> set[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return set(re.findall(r"\b(lbd?_[a-z0-9_]+)\s*\(", text))


def test_header_declares_reference_abi():
    names = header_functions()
    # the reference's exported API (src/lowbit/csrc/lowbit.h:95-123)
    ref = {"lb_version", "lb_cpu_isa", "lb_active_isa", "lb_has_vnni", "lb_has_openmp",
           "lb_max_threads", "lb_effective_isa", "lb_gemm_w4a16", "lb_gemm_mxfp4", "lb_gemm_w4a8",
           "lb_gemm_w4a8_q", "lb_quant_act_int8", "lb_w4a8_group_acc"}
    assert ref <= names


def test_library_exports_every_declared_symbol():
    so = _build.lib_path()
    out = subprocess.run(["nm", "-D", "--defined-only", str(so)], capture_output=True, text=True,
                         check=True).stdout
    exported = {ln.split()[-1] for ln in out.splitlines() if " T " in ln}
    missing = header_functions() - exported
    assert not missing, f"declared but not exported: {sorted(missing)}"
    # and the ctypes layer binds exactly the declared set
    assert set(K.SIGNATURES) == header_functions()


def test_library_loads_and_binds():
    L = K.lib()
    for name in K.SIGNATURES:
        assert hasattr(L, name)
    assert L.lb_version() == 1
    assert L.lb_has_vnni() == 0 and L.lb_max_threads() == 1


def test_public_surface_matches_reference():
    # src/lowbit/__init__.py:2-11
    ref = {"GROUP", "MXBLOCK", "Int4Weights", "Int8Acts", "MXFP4Weights", "Params", "cpu_info",
           "gemm_mxfp4", "gemm_w4a8", "gemm_w4a16", "quantize_act_int8", "quantize_int4",
           "quantize_mxfp4"}
    assert ref <= set(lb.__all__)
    for name in ref:
        assert hasattr(lb, name)
    assert lb.GROUP == 128 and lb.MXBLOCK == 32


def test_shape_errors_before_device(rng):
    # rc -1 on M, N, Kp <= 0 or Kp % block (src/lowbit/csrc/dispatch.c:205-208): checked on the host
    L = K.lib()
    x = np.zeros((1, 128), np.float32)
    qw = np.zeros((1, 64), np.uint8)
    s = np.ones((1, 1), np.float32)
    y = np.zeros((1, 1), np.float32)
    assert L.lb_gemm_w4a16(x, 0, 128, qw, s, None, 1, y, None) == -1
    assert L.lb_gemm_w4a16(x, 1, 100, qw, s, None, 1, y, None) == -1
    assert L.lb_gemm_w4a8(x, 1, 128, qw, s, None, 0, y, None) == -1
    assert L.lb_gemm_mxfp4(x, 1, 48, qw, np.zeros((1, 2), np.uint8), 1, y, None) == -1
    assert "shape" in L.lb_last_error().decode()


def test_bad_tile_rejected_like_reference(rng):
    # Params(mr=3, nr=3) names no compiled micro-tile: ValueError (tests/test_kernels.py:176-181)
    W = lb.quantize_int4(rng.standard_normal((8, 128)).astype(np.float32))
    with pytest.raises(ValueError):
        K.gemm_w4a16(np.ones((1, 128), np.float32), W, K.Params(mr=3, nr=3))
    with pytest.raises(ValueError):
        K.gemm_w4a8(np.ones((1, 128), np.float32), W, K.Params(mr=8, nr=4))
    with pytest.raises(ValueError):
        K.gemm_mxfp4(np.ones((1, 128), np.float32), lb.quantize_mxfp4(np.ones((2, 128), np.float32)),
                     K.Params(mr=5))


def test_params_and_isa_host_logic():
    with pytest.raises(ValueError):
        K._params("fastest", None, None, "w4a16", (1, 1, 1))
    p = K._params("auto", "gfx950-mfma", 4, "w4a16", (1, 1, 1))
    assert p.isa == K.ISA_GFX950_MFMA and p.nthreads == 4
    assert K._isa_id("avx512") == -1 and K._isa_id(None) == -1 and K._isa_id("gfx950") == 16
    with pytest.raises(ValueError):
        K._isa_id("sse2")
    assert K.Params(mr=4, nr=2).as_dict()["mr"] == 4
    assert K.amx_available() is False


def test_prepared_pads_and_reshapes():
    pr = K._Prepared(np.arange(5, dtype=np.float64), 128, 3)
    assert pr.x.shape == (1, 128) and pr.x.dtype == np.float32
    assert pr.x[0, 4] == 4 and pr.x[0, 5:].sum() == 0
    assert pr.y.shape == (1, 3)


def test_no_device_reports_unavailable():
    if Path("/dev/kfd").exists():
        pytest.skip("a GPU is present")
    L = K.lib()
    assert L.lb_cpu_isa() == -4
    assert K.cpu_info()["cpu_isa"] == "none"


def test_t16_sizes_and_argument_checks():
    """t16 array sizes (S = ceil(N/16) subtiles, groups padded to a multiple of 4) and
    the shape / argument errors of the repack and GEMM entry points, before any
    device work."""
    L = K.lib()
    bq, bs, bz = C.c_size_t(0), C.c_size_t(0), C.c_size_t(0)
    assert L.lbd_int4_t16_bytes(17, 256, C.byref(bq), C.byref(bs), C.byref(bz)) == 0
    assert (bq.value, bs.value, bz.value) == (2 * 4 * 1024, 2 * 16 * 4 * 4, 2 * 16 * 4)
    assert L.lbd_int4_t16_bytes(11008, 4096, C.byref(bq), C.byref(bs), C.byref(bz)) == 0
    assert bq.value == 11008 * 2048 and bs.value == 11008 * 32 * 4 and bz.value == 11008 * 32
    assert L.lbd_int4_t16_bytes(17, 200, C.byref(bq), None, None) == -1   # Kp % 128
    assert L.lbd_int4_t16_bytes(0, 256, None, None, None) == -1
    assert L.lbd_repack_int4_t16(None, None, None, 16, 256, None, None, None, None) == -6
    prm = K._Params(-1, 0, 0, 0, 0, 0, 0)
    assert L.lbd_gemm_w4a8_t16(None, 1, 256, None, None, None, 16, None, C.byref(prm), None, 0, None) == -6
    assert L.lbd_gemm_w4a8_t16(None, 0, 256, None, None, None, 16, None, C.byref(prm), None, 0, None) == -1
    # t16f8: one byte per code, so twice the t16 tile bytes; the same scale array
    assert L.lbd_int4_t16f8_bytes(17, 256, C.byref(bq), C.byref(bs)) == 0
    assert (bq.value, bs.value) == (2 * 2 * 4 * 1024, 2 * 16 * 4 * 4)
    assert L.lbd_int4_t16f8_bytes(11008, 4096, C.byref(bq), None) == 0 and bq.value == 11008 * 4096
    assert L.lbd_int4_t16f8_bytes(17, 200, C.byref(bq), None) == -1
    assert L.lbd_repack_int4_t16f8(None, None, None, 16, 256, None, None, None) == -6
    assert L.lbd_repack_int4_t16f8(None, None, None, 16, 200, None, None, None) == -1
    assert L.lbd_gemm_w4a16_t16f8(None, 1, 256, None, None, 16, None, C.byref(prm), None, 0, None) == -6
    assert L.lbd_gemm_w4a16_t16f8(None, 1, 0, None, None, 16, None, C.byref(prm), None, 0, None) == -1
    # without a device the rule assumes 256 compute units
    assert L.lbd_w4a16_prefers_t16f8(64, 11008, 4096) == 1 and L.lbd_w4a16_prefers_t16f8(16, 11008, 4096) == 0
    # at K = 11008 the split launch counts: 64 rows split in two give 4 subtiles per workgroup
    assert L.lbd_w4a16_prefers_t16f8(64, 4096, 11008) == 1 and L.lbd_w4a16_prefers_t16f8(0, 16, 128) == -1
    assert L.lbd_w4a16_prefers_t16f8(16, 4096, 11008) == 0 and L.lbd_w4a16_prefers_t16f8(32, 4096, 11008) == 0
    assert L.lbd_gemm_path(2, 1, 4096, C.byref(prm)) == K.ISA_GFX950
    assert L.lbd_gemm_path(2, 64, 4096, C.byref(prm)) == K.ISA_GFX950_MFMA
    assert L.lbd_gemm_path(7, 1, 4096, C.byref(prm)) == -6


def test_bf16x3_split_workspace_sizes():
    """The split workspace adds the slices' partial outputs only where K is split."""
    L = K.lib()
    base = L.lbd_bf16x3_workspace_bytes(16, 11008)
    align = (base + 255) // 256 * 256
    assert L.lbd_bf16x3_workspace_bytes_split(0, 16, 4096, 11008) == align  # W4A16, one row block: no split
    assert L.lbd_bf16x3_workspace_bytes_split(1, 16, 4096, 11008) == align + 4 * 16 * 4096 * 4
    a32 = (L.lbd_bf16x3_workspace_bytes(32, 11008) + 255) // 256 * 256
    assert L.lbd_bf16x3_workspace_bytes_split(0, 32, 4096, 11008) == a32 + 2 * 32 * 4096 * 4
    b64 = L.lbd_bf16x3_workspace_bytes(64, 11008)
    assert L.lbd_bf16x3_workspace_bytes_split(1, 64, 4096, 11008) == (b64 + 255) // 256 * 256  # MXFP4, 64 rows: no split
    b4 = L.lbd_bf16x3_workspace_bytes(16, 4096)
    assert L.lbd_bf16x3_workspace_bytes_split(0, 16, 4096, 4096) == (b4 + 255) // 256 * 256
    for args in ((2, 16, 64, 4096), (-1, 16, 64, 4096), (0, 0, 64, 4096), (0, 16, 0, 4096), (1, 16, 64, 0)):
        assert L.lbd_bf16x3_workspace_bytes_split(*args) == 0


def test_probe_argument_checks():
    """The measurement probes (lbd_probe_valu, lbd_empty_kernel, lbd_read_kernel,
    lbd_probe_grid_barrier) reject
    bad arguments before any device work, and the probe count matches the instruction
    forms bench.py names."""
    import bench
    L = K.lib()
    assert L.lbd_probe_forms() == len(bench.PROBE_FORMS) == 18
    assert L.lbd_probe_valu(0, 16, 1, None, None) == -6            # no output buffer
    out = C.c_void_p(16)                                            # never dereferenced
    assert L.lbd_probe_valu(18, 16, 1, out, None) == -6             # past the last form
    assert L.lbd_probe_valu(-1, 16, 1, out, None) == -6
    assert L.lbd_probe_valu(0, 0, 1, out, None) == -6               # no iterations
    assert L.lbd_probe_valu(0, 16, 0, out, None) == -6              # no workgroups
    assert L.lbd_empty_kernel(0, None) == -6
    assert L.lbd_probe_mfma_valu(0, 16, 1, 256, None, None) == -6      # no output buffer
    assert L.lbd_probe_mfma_valu(4, 16, 1, 256, out, None) == -6       # past the last variant
    assert L.lbd_probe_mfma_valu(0, 16, 1, 128, out, None) == -6       # 128 threads
    assert L.lbd_probe_mfma_valu(0, 0, 1, 512, out, None) == -6        # no iterations
    assert L.lbd_empty_kernel(70000, None) == -6
    assert L.lbd_read_kernel(None, 1024, 1, 256, 1, None, None) == -6
    assert L.lbd_read_kernel(out, 1000, 1, 256, 1, out, None) == -6   # not a multiple of 16
    assert L.lbd_read_kernel(out, 1024, 1, 128, 1, out, None) == -6   # 128 threads
    assert L.lbd_read_kernel(out, 1024, 1, 256, 3, out, None) == -6   # 3 loads
    sync = (64 + 256) * 4
    assert L.lbd_probe_grid_barrier(256, 10, 0, None, sync, out, None) == -6    # no sync buffer
    assert L.lbd_probe_grid_barrier(256, 10, 0, out, sync, None, None) == -6    # no status word
    assert L.lbd_probe_grid_barrier(0, 10, 0, out, sync, out, None) == -6       # no workgroups
    assert L.lbd_probe_grid_barrier(1025, 10, 0, out, 8192, out, None) == -6    # past 1024 workgroups
    assert L.lbd_probe_grid_barrier(256, -1, 0, out, sync, out, None) == -6     # negative rounds
    assert L.lbd_probe_grid_barrier(256, 100001, 0, out, sync, out, None) == -6
    assert L.lbd_probe_grid_barrier(256, 10, 3, out, sync, out, None) == -6     # no mode 3
    assert L.lbd_probe_grid_barrier(256, 10, 0, out, sync - 4, out, None) == -6  # sync too small


def test_argmax_slot_count_matches_header():
    import re

    from lowbit_amd import model as DM
    m = re.search(r"#define LBD_ARGMAX_SLOTS (\d+)", HEADER.read_text())
    assert m and int(m.group(1)) == DM.ARGMAX_SLOTS


_CAP_PROBE = """
import ctypes as C, json
from lowbit_amd import kernels as K
L = K.lib()
def path(isa, m):
    return L.lbd_gemm_path(2, m, 4096, C.byref(K._Params(isa, 0, 0, 0, 0, 0, 0)))
print(json.dumps({"mfma_m1": path(K.ISA_GFX950_MFMA, 1), "auto_m1": path(-1, 1),
                  "valu_m1": path(K.ISA_GFX950, 1), "mfma_m64": path(K.ISA_GFX950_MFMA, 64),
                  "valu_m64": path(K.ISA_GFX950, 64)}))
"""


@pytest.mark.parametrize("cap,mfma_m1", [(None, K.ISA_GFX950_MFMA), ("gfx950", K.ISA_GFX950)])
def test_isa_cap_clamps_requests(cap, mfma_m1):
    """LOWBIT_ISA=gfx950 clamps a matrix-core request to the VALU kernels where the
    shape allows, as the reference clamps requests to its cap
    (src/lowbit/csrc/dispatch.c:77-80,151); shapes the VALU kernels cannot run stay
    on the matrix cores. Run in a fresh process: the cap is read once."""
    import json
    import os
    import sys
    env = {k: v for k, v in os.environ.items() if k != "LOWBIT_ISA"}
    if cap:
        env["LOWBIT_ISA"] = cap
    out = subprocess.run([sys.executable, "-c", _CAP_PROBE], capture_output=True, text=True, check=True,
                         cwd=ROOT, env=env).stdout
    got = json.loads(out.strip().splitlines()[-1])
    assert got["mfma_m1"] == mfma_m1
    assert got["auto_m1"] == got["valu_m1"] == K.ISA_GFX950
    assert got["mfma_m64"] == got["valu_m64"] == K.ISA_GFX950_MFMA
