"""Exhaustive check of the one-row W4A8 quantizer's division by 127 (CPU only).

The paced one-row W4A8 GEMV computes its token scale amax / 127 as lbk::div127
(lowbit_amd/csrc/lb_device.h): one multiply and two fused multiply-adds. The
reference divides in IEEE float32 (src/lowbit/csrc/dispatch.c:231-257), so the two
must agree on every input the kernel can see: every non-negative finite float32
and +inf. tests/csrc/div127_exhaustive.hip runs the same header function on the
host over all 2^31 - 2^23 + 1 of them. Its "plain" mode checks the uncorrected
product instead and must report mismatches, which shows the check can fail.
The GPU twin of this check (lbd_probe_div127, the device build of the same
function) is in tests/test_gpu_w4a8_quant_exact.py.
"""
import re
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
SRC = ROOT / "tests" / "csrc" / "div127_exhaustive.hip"


def _hipcc():
    p = Path("/opt/rocm/bin/hipcc")
    return str(p) if p.exists() else shutil.which("hipcc")


@pytest.fixture(scope="module")
def checker(tmp_path_factory):
    cc = _hipcc()
    if cc is None:
        pytest.skip("hipcc not available")
    exe = tmp_path_factory.mktemp("div127") / "div127_exhaustive"
    cmd = [cc, "--offload-host-only", "-x", "hip", "-O2", "-ffp-contract=off", "-std=c++17",
           f"-I{ROOT / 'lowbit_amd' / 'csrc'}", f"-I{ROOT / 'include'}", str(SRC), "-o", str(exe), "-pthread"]
    subprocess.run(cmd, check=True, capture_output=True, text=True)
    return exe


def _run(exe, *args):
    r = subprocess.run([str(exe), *args], capture_output=True, text=True, timeout=600)
    m = re.search(r"checked (\d+) mismatches (\d+)", r.stdout)
    assert m, r.stdout + r.stderr
    return r.returncode, int(m.group(1)), int(m.group(2))


def test_div127_equals_ieee_division_for_every_input(checker):
    rc, checked, bad = _run(checker)
    assert checked == 0x7F800001  # +0 through +inf
    assert bad == 0 and rc == 0


def test_checker_catches_the_uncorrected_product(checker):
    rc, checked, bad = _run(checker, "plain")
    assert checked == 1 << 23 and bad > 0 and rc == 1
