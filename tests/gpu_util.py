"""Helpers for the GPU parity tests (host <-> device plumbing via torch)."""
import sys

import numpy as np


def say(*a):
    """Name the case before each GPU step (flushed, so a failing run still shows it)."""
    print("[gpu-case]", *a, flush=True)
    sys.stdout.flush()


def to_dev(a: np.ndarray, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def to_host(t) -> np.ndarray:
    import torch
    torch.cuda.synchronize()
    return t.detach().cpu().numpy()


def act_host(m27q, act):
    codes, d, s = act.parts()
    return to_host(codes), to_host(d), to_host(s).view(np.uint32)


def int_dot_tol(norm):
    """fp32 reassociation bound for the int8-activation products (rows of <= 68 blocks)."""
    return 1e-5 * norm + 1e-30
