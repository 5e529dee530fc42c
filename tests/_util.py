"""Shared helpers for the tests."""
import numpy as np


def to_dev(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def to_np(t):
    return t.detach().cpu().numpy()


def gemm_tol(k, a, b):
    """fp32 GEMM bound: max|err| <= 1e-4 * sqrt(K) * max|a| * max|b|."""
    return 1e-4 * np.sqrt(max(k, 1)) * float(np.abs(a).max(initial=0)) * float(np.abs(b).max(initial=0))
