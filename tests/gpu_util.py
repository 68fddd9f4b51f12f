"""Device-memory plumbing for the GPU tests (torch tensors as buffers only).

Tensors made here stay referenced until the end of the test (see the autouse
fixture in conftest.py), so a pointer passed inline to an asynchronous HIP
call can never be freed and reused by the caching allocator before the
kernel has run."""
import numpy as np
import torch

import tbn_hip

_KEEP = []


def to_dev(a):
    t = torch.from_numpy(np.ascontiguousarray(a)).to("cuda:0")
    _KEEP.append(t)
    return t


def empty(shape, dtype):
    t = torch.empty(shape, dtype=dtype, device="cuda:0")
    _KEEP.append(t)
    return t


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def P(t):
    return tbn_hip.ptr(t)


def release():
    if _KEEP:
        torch.cuda.synchronize()
        _KEEP.clear()
