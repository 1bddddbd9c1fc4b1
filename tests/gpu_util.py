"""GPU-test plumbing: device buffers from numpy (torch is the allocator here, nothing more), pointer tables, and calls
through the C ABI (libosmos_amd.capi) that must be queued (return true)."""
import numpy as np
import torch

from libosmos_amd import capi


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


# every buffer whose address was handed to a call stays referenced until that call's work has finished: a tensor freed
# while its address is in flight goes back to torch's caching allocator, and the next argument's buffer can be given
# the same address (two arguments aliasing one buffer)
_alive = []


def table(tensors):
    """a device-readable table of device pointers; the tensors live as long as the table does"""
    t = torch.tensor([x.data_ptr() for x in tensors], dtype=torch.int64, device="cuda")
    t._keep = list(tensors)
    return t


def a(t):
    if t is not None:
        _alive.append(t)
    return capi.addr(t)


def call(name, *args):
    ok = getattr(capi.lib(), name)(*args)
    assert ok, "%s refused" % name
    torch.cuda.synchronize()
    _alive.clear()
    return ok


def host(t):
    torch.cuda.synchronize()
    _alive.clear()
    return t.cpu().numpy()


def bits(x):
    return np.ascontiguousarray(x, np.float32).view(np.uint32)
