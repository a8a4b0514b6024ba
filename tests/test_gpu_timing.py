"""The measurement hook tq4_time_next_launch: the next launch stamps the caller's events
with its own start and end, inside the interval of events recorded around it; the hook
then clears itself."""
import ctypes

import pytest
import torch

from conftest import to_dev
from tq4_decode import _lib, ops, workloads

pytestmark = pytest.mark.gpu


def test_next_launch_stamps_kernel_interval(dev):
    hip = ctypes.CDLL("libamdhip64.so.7")
    w = workloads.small(201, 4, [3000, 2048, 17, 4096], 8)
    t = lambda a: to_dev(a, dev)  # noqa: E731
    args = (t(w.q_rot), t(w.kv_cache), t(w.block_table), t(w.seq_lens), t(w.pair_lut))
    mid = torch.empty(4, 32, 8, 129, device=dev)
    ev = []
    for _ in range(6):
        e = ctypes.c_void_p()
        assert hip.hipEventCreate(ctypes.byref(e)) == 0
        ev.append(e)
    a, b, ka, kb, ka2, kb2 = ev
    stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    ops.stage1(*args, mid)
    torch.cuda.synchronize()
    assert hip.hipEventRecord(a, stream) == 0
    assert _lib.load().tq4_time_next_launch(ka, kb) == 0
    ops.stage1(*args, mid)
    assert hip.hipEventRecord(b, stream) == 0
    ops.stage1(*args, mid)  # the hook is cleared: ka2 / kb2 are never recorded
    torch.cuda.synchronize()
    ms = ctypes.c_float()
    assert hip.hipEventElapsedTime(ctypes.byref(ms), ka, kb) == 0
    kernel = ms.value
    assert hip.hipEventElapsedTime(ctypes.byref(ms), a, b) == 0
    around = ms.value
    print(f"kernel {kernel * 1e3:.2f} us, around {around * 1e3:.2f} us")
    assert 0 < kernel <= around
    # never-recorded events: hipEventElapsedTime reports an error, which stays the thread's
    # last HIP error until read: read it here, or the next torch call reports it
    assert hip.hipEventElapsedTime(ctypes.byref(ms), ka2, kb2) != 0
    assert hip.hipGetLastError() != 0
    assert hip.hipGetLastError() == 0
    for e in ev:
        hip.hipEventDestroy(e)
