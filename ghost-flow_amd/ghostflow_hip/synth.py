"""Seeded, counter-based synthetic inputs.

The reference draws test tensors from an unseeded thread_rng
(ghostflow-core/src/tensor.rs:91-110), so "seed 0" has no reference meaning;
this generator defines one.  Element i of tensor `tensor_id` under `seed` is
a pure function of (seed, tensor_id, i):

    c      = i + tensor_id * 2^40 + seed * 2^52          (mod 2^64)
    h_j    = splitmix64_output((2c + j + 1) * 0x9E3779B97F4A7C15), j = 0, 1
    U(a,b) = a + (b - a) * (h_0 >> 40) * 2^-24                (fp64 -> f32)
    N(m,s) = m + s * sqrt(-2 ln u1) * cos(2 pi u2)            (fp64 -> f32)
             u1 = ((h_0 >> 11) + 1) * 2^-53,  u2 = (h_1 >> 11) * 2^-53

so any sub-block of a large tensor can be regenerated on its own (the tests
use that to check sampled rows of full-size outputs).
"""
from __future__ import annotations

import os
from concurrent.futures import ThreadPoolExecutor

import numpy as np

_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)
_CHUNK = 1 << 22


def _mix64(z):
    z = (z ^ (z >> np.uint64(30))) * _M1
    z = (z ^ (z >> np.uint64(27))) * _M2
    return z ^ (z >> np.uint64(31))


def _hashes(seed, tensor_id, start, count, j):
    c = np.arange(start, start + count, dtype=np.uint64)
    c += np.uint64((int(tensor_id) << 40) + (int(seed) << 52) & 0xFFFFFFFFFFFFFFFF)
    with np.errstate(over="ignore"):
        return _mix64((c * np.uint64(2) + np.uint64(j + 1)) * _GOLDEN)


def _fill(n, chunk_fn):
    """Fills a float32 vector of n elements chunk by chunk; chunks are
    independent (counter-based), so large tensors are filled by a few
    threads (numpy releases the GIL in these element-wise passes) with the
    same values as a sequential fill."""
    out = np.empty(n, np.float32)
    starts = range(0, n, _CHUNK)

    def one(s):
        cnt = min(_CHUNK, n - s)
        out[s:s + cnt] = chunk_fn(s, cnt)

    workers = min(8, os.cpu_count() or 1, len(starts))
    if workers <= 1:
        for s in starts:
            one(s)
    else:
        with ThreadPoolExecutor(workers) as pool:
            list(pool.map(one, starts))
    return out


def uniform(shape, low, high, *, seed=0, tensor_id=0, start=0):
    """U(low, high) as float32, element i drawn from counter start + i."""
    n = int(np.prod(shape)) if len(shape) else 1

    def chunk(s, cnt):
        h0 = _hashes(seed, tensor_id, start + s, cnt, 0)
        u = (h0 >> np.uint64(40)).astype(np.float64) * (2.0 ** -24)
        return (low + (high - low) * u).astype(np.float32)

    return _fill(n, chunk).reshape(shape)


def normal(shape, mean=0.0, std=1.0, *, seed=0, tensor_id=0, start=0):
    """N(mean, std) as float32 via fp64 Box-Muller, element i from counter start + i."""
    n = int(np.prod(shape)) if len(shape) else 1

    def chunk(s, cnt):
        h0 = _hashes(seed, tensor_id, start + s, cnt, 0)
        h1 = _hashes(seed, tensor_id, start + s, cnt, 1)
        u1 = ((h0 >> np.uint64(11)).astype(np.float64) + 1.0) * (2.0 ** -53)
        u2 = (h1 >> np.uint64(11)).astype(np.float64) * (2.0 ** -53)
        z = np.sqrt(-2.0 * np.log(u1)) * np.cos(2.0 * np.pi * u2)
        return (mean + std * z).astype(np.float32)

    return _fill(n, chunk).reshape(shape)


def rows(shape, r0, r1, dist, *, seed=0, tensor_id=0, **kw):
    """Rows [r0, r1) of a 2-D tensor of `shape` drawn with `dist` (normal/uniform)."""
    cols = shape[1]
    return dist((r1 - r0, cols), seed=seed, tensor_id=tensor_id, start=r0 * cols, **kw)
