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


def assert_rel(got, ref, tol=1e-4):
    """Attention bar: max|err| / max|ref| <= tol and, per element,
    |err| <= tol * (|ref| + mean|ref|)."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    assert got.shape == ref.shape
    err = np.abs(got - ref)
    scale = np.abs(ref).max()
    assert err.max() <= tol * scale + 1e-30, (err.max(), scale)
    bound = tol * (np.abs(ref) + np.abs(ref).mean())
    bad = err > bound
    assert not bad.any(), (int(bad.sum()), float(err[bad].max()))


def rows_parallel(fn, a_rows, *args, workers=None, chunk=32):
    """fn(a_rows[i:j], *args) over row chunks on a few threads, stacked.

    For oracle functions whose output rows depend only on the same input rows
    (matmul_blocked, Linear::forward, the INT8 linear): each chunk gives the
    same bits as one call on all rows.  ctypes releases the GIL during the C
    call, so the chunks run in parallel."""
    import os
    from concurrent.futures import ThreadPoolExecutor
    a_rows = np.ascontiguousarray(a_rows)
    n = a_rows.shape[0]
    if n == 0:
        return fn(a_rows, *args)
    workers = workers or min(16, os.cpu_count() or 1)
    parts = [a_rows[i:i + chunk] for i in range(0, n, chunk)]
    with ThreadPoolExecutor(workers) as pool:
        outs = list(pool.map(lambda p: fn(p, *args), parts))
    return np.concatenate(outs, axis=0)
