"""mxq.matmul -- the array dataflow: Y = A^T B from codes and scales, in the order the hardware sums them.

    Y = systolic(P_A, X_A, P_B, X_B, arith, schedule, size=16)      the PE column (MX-Gemmini, MXQuant)

A: K x M, B: K x N, X: one row of scales per 32-block of K, Y: M x N, all float32.  The Arithmetic (MXGEMMINI
or MXQUANT) is how each step rounds; the schedule is one float(e, m) per PE lane.  For the same codes with no
rounding inside the multiply, see mxq.fp64_accum.
"""
from ._arithmetic import Arithmetic, MXQUANT, MXGEMMINI, compiled
from ._systolic import systolic
from ..schedule import HW_FINAL

__all__ = ["Arithmetic", "MXQUANT", "MXGEMMINI", "compiled", "systolic", "HW_FINAL"]
