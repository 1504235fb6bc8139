"""Oracle systolic reducer (the PE column) and fp64_accum.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

`systolic` follows mxq/matmul/_systolic.py:23-62 step for step: per block of K its scale map, per reduction
of `size` a fresh sum, one product per k and one lane accumulate in schedule[k % size]'s format, then the
rescaled sum added into C.  Vectorised over the M x N outputs, like the reference's eager path.

Pins: oracle/brute.py's exact-rational scalar model of the same datapath (tiny M, N, K); invariants
(columns independent, an all-zero K block leaves C unchanged); fixtures the reference wrote for the
composed MXGEMMINI / MXQUANT end to end (tests/golden/).
"""
import math

import numpy as np

from . import block as ob
from . import numerics as nx

F32, F64 = np.float32, np.float64
HW_FINAL = [(4, 4)] * 8 + [(4, 5)] * 2 + [(4, 6)] * 5 + [(8, 7)]


def scale_map(X_A, X_B, g):
    """mxq/matmul/_common.py:32-34."""
    with np.errstate(all="ignore"):
        return (X_A[g][:, None] * X_B[g][None, :]).astype(F32)


def systolic(P_A, X_A, P_B, X_B, arith, schedule, size=16, block_size=32):
    """mxq/matmul/_systolic.py:23-62."""
    P_A, X_A, P_B, X_B = (np.asarray(t, dtype=F32) for t in (P_A, X_A, P_B, X_B))
    K, M = P_A.shape
    N = P_B.shape[1]
    assert len(schedule) == size and block_size % size == 0
    assert X_A.shape == (math.ceil(K / block_size), M) and X_B.shape == (math.ceil(K / block_size), N)
    C = np.zeros((M, N), dtype=F32)
    for g in range(0, K, block_size):
        g_end = min(g + block_size, K)
        scales = scale_map(X_A, X_B, g // block_size)
        for k_base in range(g, g_end, size):
            k_end = min(k_base + size, g_end)
            S = np.zeros((M, N), dtype=F32)
            for k in range(k_base, k_end):
                p = arith.product(P_A[k][:, None], P_B[k][None, :])
                e, m = schedule[k % size]
                S = arith.acc_add(S, p, e, m)
            with np.errstate(all="ignore"):
                tile = (S * scales).astype(F32)
            C = arith.tile_add(C, tile)
    return C.astype(F32)


def fp64_accum(P_A, X_A, P_B, X_B, block_size=32):
    """mxq/_fp64_accum.py:24-29."""
    A = ob.dequantize(np.asarray(P_A, F32), np.asarray(X_A, F32), 0, block_size).astype(F64)
    B = ob.dequantize(np.asarray(P_B, F32), np.asarray(X_B, F32), 0, block_size).astype(F64)
    return (A.T @ B).astype(F32)
