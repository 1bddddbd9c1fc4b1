"""ops_wait and ops_copy_rows (include/osmos/gpu/ops.h) on the MI355X: the lane's hand-off of rows a host job computes
(reference src/run/hip_lane.c:218-219, include/osmos/gpu/ops.h:340-347). The stream is held while the host's flag
holds anything but the value; released by the value with its top bit set (a failed job's mark); the rows the host
wrote before the flag are what ops_copy_rows reads after it. The host always posts the value in the end (a timer, and
a finally), so the wait ends in every outcome."""
import threading
import time

import numpy as np
import pytest

from libosmos_amd import capi

pytestmark = pytest.mark.gpu


def test_wait_then_copy_rows():
    import torch
    L = capi.lib()
    flag = torch.zeros(1, dtype=torch.int32, pin_memory=True)  # (host memory the GPU maps)
    rows, n = 64, 256
    src = torch.zeros(rows, n, pin_memory=True)
    dst = torch.full((rows, n), -1.0, device="cuda")
    pick = [3, 7, 8, 63]
    idx = torch.tensor(pick, dtype=torch.int32, device="cuda")
    s = torch.cuda.Stream()
    release = threading.Timer(20.0, lambda: flag.fill_(7))
    release.start()
    print("ops_wait hand-off", flush=True)
    try:
        assert L.ops_wait(capi.addr(flag), 7, s.cuda_stream)
        assert L.ops_copy_rows(capi.addr(dst), capi.addr(src), capi.addr(idx), len(pick), n, s.cuda_stream)
        done = torch.cuda.Event()
        done.record(s)
        time.sleep(0.2)
        assert not done.query(), "the stream ran past an unposted flag"
        rng = np.random.default_rng(3)
        want = rng.normal(0, 1, (rows, n)).astype(np.float32)
        src.copy_(torch.from_numpy(want))  # the host job's rows, written before the flag
        flag.fill_(5)  # another value: still held
        time.sleep(0.1)
        assert not done.query(), "the stream ran on a value that is not the one awaited"
        flag.fill_(7 - (1 << 31))  # 7 with the top bit set: released
        done.synchronize()
    finally:
        flag.fill_(7)
        release.cancel()
    torch.cuda.synchronize()
    out = dst.cpu().numpy()
    for r in range(rows):
        if r in pick:
            assert (out[r].view(np.int32) == want[r].view(np.int32)).all(), r
        else:
            assert (out[r] == -1.0).all(), r


def test_refusals():
    L = capi.lib()
    assert not L.ops_wait(None, 1, None)
    p = capi.ctypes.c_void_p(8)
    assert not L.ops_copy_rows(None, p, p, 1, 1, None)
    assert not L.ops_copy_rows(p, p, p, 0, 1, None) and not L.ops_copy_rows(p, p, p, 1, 0, None)


def test_wait_bound_then_nan_rows():
    """a flag the host never posts: with the bound set to 2 ms the wait ends by itself and the copy after it writes NaN
    rows (not the host's unwritten ones); the next wait that sees its value makes copies copy again"""
    import torch
    L = capi.lib()
    flag = torch.zeros(1, dtype=torch.int32, pin_memory=True)
    rows, n = 8, 64
    src = torch.full((rows, n), 3.0, pin_memory=True)
    dst = torch.zeros(rows, n, device="cuda")
    idx = torch.tensor([1, 5], dtype=torch.int32, device="cuda")
    print("ops_wait bound", flush=True)
    L.osmos_wait_limit(2000)
    try:
        assert L.ops_wait(capi.addr(flag), 9, None)
        assert L.ops_copy_rows(capi.addr(dst), capi.addr(src), capi.addr(idx), 2, n, None)
        torch.cuda.synchronize()
    finally:
        L.osmos_wait_limit(0)
    out = dst.cpu().numpy()
    assert np.isnan(out[[1, 5]]).all() and (out[[0, 2, 3, 4, 6, 7]] == 0).all()
    flag.fill_(9 - (1 << 31))  # 9 with the top bit set (a failed job), as a signed int32: still the post
    assert L.ops_wait(capi.addr(flag), 9, None)
    assert L.ops_copy_rows(capi.addr(dst), capi.addr(src), capi.addr(idx), 2, n, None)
    torch.cuda.synchronize()
    assert (dst.cpu().numpy()[[1, 5]] == 3.0).all()
    assert not L.ops_wait(capi.addr(flag), 9 | (1 << 31), None)  # a value with the mark's bit: refused


def test_expiry_is_per_stream():
    """two flags on two streams: the wait on stream A expires (A's copies write NaN) while the wait on stream B sees its
    value (B's copies copy), and a third stream that never waited copies; then B expires and A's next wait succeeds,
    each stream's copies following its own wait only"""
    import torch
    L = capi.lib()
    fa = torch.zeros(1, dtype=torch.int32, pin_memory=True)
    fb = torch.full((1,), 4, dtype=torch.int32, pin_memory=True)
    n = 64
    src = torch.full((4, n), 2.0, pin_memory=True)
    idx = torch.tensor([0, 1, 2, 3], dtype=torch.int32, device="cuda")
    sa, sb, sc = torch.cuda.Stream(), torch.cuda.Stream(), torch.cuda.Stream()
    print("ops_wait per stream", flush=True)

    def step(wa, wb):
        da, db, dc = (torch.zeros(4, n, device="cuda") for _ in range(3))
        torch.cuda.synchronize()
        assert L.ops_wait(capi.addr(fa), wa, sa.cuda_stream)
        sa.synchronize()
        assert L.ops_wait(capi.addr(fb), wb, sb.cuda_stream)
        sb.synchronize()
        for d, s in ((da, sa), (db, sb), (dc, sc)):
            assert L.ops_copy_rows(capi.addr(d), capi.addr(src), capi.addr(idx), 4, n, s.cuda_stream)
        torch.cuda.synchronize()
        return da.cpu().numpy(), db.cpu().numpy(), dc.cpu().numpy()

    L.osmos_wait_limit(2000)
    try:
        a, b, c = step(9, 4)  # A's flag never posts 9: expires; B's holds 4
        assert np.isnan(a).all() and (b == 2.0).all() and (c == 2.0).all()
        fa.fill_(9)
        a, b, c = step(9, 5)  # now A sees its value, B expires
        assert (a == 2.0).all() and np.isnan(b).all() and (c == 2.0).all()
    finally:
        L.osmos_wait_limit(0)
