"""The measurement kernels behind bench.py --machine-facts and the read floor, run on
the GPU through the C ABI: each completes and leaves its outputs as documented.
They measure; nothing here checks a time."""
import ctypes as C

import numpy as np
import pytest

from lowbit_amd import kernels as K

pytestmark = pytest.mark.gpu


def _sync():
    assert K.lib().lb_dev_synchronize() == 0


def test_read_kernel_leaves_the_sink():
    """The plain read XORs what it reads and writes the sink only when the XOR hits a
    fixed value; a zero buffer never does, whatever the grid."""
    L = K.lib()
    src = K.DeviceBuffer.from_array(np.zeros(1 << 16, np.uint32))
    sink = K.DeviceBuffer.from_array(np.array([0xDEADBEEF], np.uint32))
    for wgs, threads, loads in ((1, 256, 1), (7, 512, 8), (256, 256, 4)):
        assert L.lbd_read_kernel(src.ptr, src.nbytes, wgs, threads, loads, sink.ptr, None) == 0
    _sync()
    assert sink.to_array((1,), np.uint32)[0] == 0xDEADBEEF


def test_empty_and_valu_probes_run():
    L = K.lib()
    out = K.DeviceBuffer(2 * 512 * 4)
    assert L.lbd_empty_kernel(2, None) == 0
    for op in range(L.lbd_probe_forms()):
        assert L.lbd_probe_valu(op, 4, 2, out.ptr, None) == 0
    _sync()
    assert np.isfinite(out.to_array((2 * 512,), np.float32)).all()


@pytest.mark.parametrize("mode", [0, 1, 2])
@pytest.mark.parametrize("workgroups,rounds", [(1, 5), (64, 50), (64, 0)])
def test_grid_barrier_completes(mode, workgroups, rounds):
    """Every round's barrier completes (no bounded wait times out) with a resident
    grid, and the counter / flags end where the rounds leave them."""
    L = K.lib()
    sync = K.DeviceBuffer((64 + 1024) * 4)
    status = K.DeviceBuffer(4)
    s = C.c_void_p()
    assert L.lb_stream_create(C.byref(s)) == 0
    assert L.lbd_probe_grid_barrier(workgroups, rounds, mode, sync.ptr, sync.nbytes, status.ptr, s.value) == 0
    assert L.lb_stream_synchronize(s.value) == 0
    assert status.to_array((1,), np.uint32)[0] == 0
    words = sync.to_array((64 + workgroups,), np.uint32)
    if mode == 0:
        assert words[0] == rounds * workgroups
    else:
        assert (words[64:] == rounds).all()
    L.lb_stream_destroy(s.value)
