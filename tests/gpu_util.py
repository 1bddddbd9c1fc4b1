"""GPU-test plumbing: device buffers from numpy (torch is the allocator here, nothing more), pointer tables, and calls
through the C ABI (libosmos_amd.capi) that must be queued (return true)."""
import numpy as np
import torch

from libosmos_amd import capi


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def table(tensors):
    """a device-readable table of device pointers"""
    return torch.tensor([t.data_ptr() for t in tensors], dtype=torch.int64, device="cuda")


def a(t):
    return capi.addr(t)


def call(name, *args):
    ok = getattr(capi.lib(), name)(*args)
    assert ok, "%s refused" % name
    return ok


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def bits(x):
    return np.ascontiguousarray(x, np.float32).view(np.uint32)
