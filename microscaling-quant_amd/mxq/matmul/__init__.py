"""mxq.matmul -- the array dataflows: Y = A^T B from codes and scales, in the order the hardware sums them.

    Y = systolic(P_A, X_A, P_B, X_B, arith, schedule, size=16)        the PE column (MX-Gemmini, MXQuant)
    Y = anchor_tree(P_A, X_A, P_B, X_B, arith, schedule=None, size=16, *, width, bits, drop, headroom, emin)
                                                                      MxGen's anchor tree: one anchor, integer adds
    Y = adder_tree(P_A, X_A, P_B, X_B, arith, schedule, size=16)      an adder tree, one float(e, m) per level

All three take the same operands, Arithmetic, size and block_size and return the same M x N float32, so a
Scheme swaps one for another in `reduce=`.  A schedule entry is a lane (systolic, size entries), a tree's
output format (anchor_tree, size / width entries) or a tree level (adder_tree, log2 size entries).

A: K x M, B: K x N, X: one row of scales per 32-block of K, Y: M x N, all float32.  The Arithmetic (MXGEMMINI
or MXQUANT) is how each step rounds.  For the same codes with no rounding inside the multiply, see
mxq.fp64_accum.
"""
from ._arithmetic import Arithmetic, MXQUANT, MXGEMMINI, compiled
from ._systolic import systolic
from ._anchor import anchor_tree
from ._adder import adder_tree
from ..schedule import HW_FINAL

__all__ = ["Arithmetic", "MXQUANT", "MXGEMMINI", "compiled", "systolic", "anchor_tree", "adder_tree", "HW_FINAL"]
