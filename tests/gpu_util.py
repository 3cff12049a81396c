"""Helpers for GPU tests: numpy <-> device tensors (u64 travels as int64 bits)."""
import sys

import numpy as np
import torch


def dev(a):
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint64:
        a = a.view(np.int64)
    return torch.from_numpy(a.copy()).to("cuda")


def host(t, dtype=None):
    a = t.detach().cpu().numpy()
    if dtype is not None:
        a = a.view(dtype)
    return a


def u64(t):
    return host(t).view(np.uint64)


def say(msg):
    """Names the case before a GPU step (so a fault report identifies it)."""
    sys.stdout.write("[gpu-case] %s\n" % msg)
    sys.stdout.flush()


class Pins:
    """Keeps device tensors alive for the duration of a test step:
    p(arr) uploads arr and returns its device address."""

    def __init__(self):
        self.held = []

    def __call__(self, a):
        if a is None:
            return None
        t = a if isinstance(a, torch.Tensor) else dev(a)
        self.held.append(t)
        return t.data_ptr()
