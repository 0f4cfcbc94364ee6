"""Batch sums of the oracle over a thread pool -- test infrastructure.

Weight and bias gradients are sums over the images (rows) of a batch.  At the
BASELINE configurations' full batch the single-threaded oracle needs minutes
per layer, so these helpers run an oracle function on chunks of the leading
axis in a thread pool (the oracle's ctypes calls release the GIL) and add the
chunk results in float64.  Every chunk result is the oracle's own f32
evaluation; adding the chunks in float64 only changes the order of the outer
sum, which the parity gate's accumulation allowance (8 K u S) covers.

The scale S of the gate is the same sum with every array argument replaced by
its absolute value (the functions are bilinear)."""
from __future__ import annotations

import os
from concurrent.futures import ThreadPoolExecutor

import numpy as np

# The GPU box gives one GPU's job 16 host cores.
WORKERS = max(1, min(16, os.cpu_count() or 1))


def batch_sum(fn, batched, rest=(), kw=None, pick=None):
    """(ref, scale): sum over chunks [i, j) of the leading axis of
    fn(*[b[i:j] for b in batched], *rest, **kw), and the same with every array
    argument by absolute value; both float64.  pick(result) selects one output
    of a function that returns several."""
    kw = kw or {}
    n = batched[0].shape[0]
    assert all(b.shape[0] == n for b in batched)
    step = max(1, -(-n // (2 * WORKERS)))
    bounds = [(i, min(n, i + step)) for i in range(0, n, step)]

    def one(ij, absval):
        i, j = ij
        args = [np.abs(b[i:j]) if absval else b[i:j] for b in batched]
        args += [np.abs(r) if (absval and isinstance(r, np.ndarray)) else r for r in rest]
        out = fn(*args, **kw)
        return np.asarray(out if pick is None else pick(out), np.float64)

    with ThreadPoolExecutor(WORKERS) as ex:
        refs = list(ex.map(lambda ij: one(ij, False), bounds))
        scs = list(ex.map(lambda ij: one(ij, True), bounds))
    return sum(refs[1:], refs[0].copy()), sum(scs[1:], scs[0].copy())
