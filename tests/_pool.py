"""The oracle's systolic reducer spread over host cores, for parity checks at the benchmark shapes.

Every output of Y = A^T B is an independent chain, so the oracle runs on tiles of Y (a slice of A's columns
against a slice of B's) in a forked process pool and the tiles are put back together.  The workers run numpy
only (never the GPU); the operands reach them through the fork (copy on write), and only the tiles' results
travel back.  Tiles of about 16K outputs keep each numpy step in cache.  The pool holds at most 16 processes
(a GPU box's CPU share), fewer where this process may use fewer CPUs.
"""
import multiprocessing as mp
import os

import numpy as np

from oracle import numerics as nx
from oracle import systolic as osys

_JOB = None
TILE = 1 << 14


def cores():
    return max(1, min(16, len(os.sched_getaffinity(0))))


def _tile(rc):
    pa, xa, pb, xb, arith, schedule, size, bs, tm, tn = _JOB
    r, c = rc
    return osys.systolic(pa[:, r:r + tm], xa[:, r:r + tm], pb[:, c:c + tn], xb[:, c:c + tn], arith, schedule, size,
                         bs)


def systolic(pa, xa, pb, xb, arith=None, schedule=None, size=16, block_size=32):
    """oracle.systolic.systolic(pa, xa, pb, xb, arith, schedule, size, block_size), tiles in parallel.
    arith defaults to MXGEMMINI(), schedule to HW_FINAL."""
    global _JOB
    arith = arith or nx.MXGEMMINI()
    schedule = schedule or osys.HW_FINAL
    M, N = pa.shape[1], pb.shape[1]
    tn = max(1, min(N, TILE // max(M, 1)))
    tm = max(1, min(M, TILE // tn))
    _JOB = tuple(np.ascontiguousarray(t, np.float32) for t in (pa, xa, pb, xb)) + (arith, schedule, size,
                                                                                     block_size, tm, tn)
    try:
        tiles = [(r, c) for r in range(0, M, tm) for c in range(0, N, tn)]
        n = min(cores(), len(tiles))
        if n <= 1:
            parts = [_tile(t) for t in tiles]
        else:
            with mp.get_context("fork").Pool(n) as pool:
                parts = pool.map(_tile, tiles, chunksize=1)
    finally:
        _JOB = None
    Y = np.zeros((M, N), np.float32)
    for (r, c), y in zip(tiles, parts):
        Y[r:r + y.shape[0], c:c + y.shape[1]] = y
    return Y


def reducer(arith=None, schedule=None):
    """A numpy reduce callable (P_A, X_A, P_B, X_B) -> Y for oracle.attend.Side, parallel over tiles."""
    return lambda pa, xa, pb, xb: systolic(pa, xa, pb, xb, arith, schedule)
