"""fp64_accum (mxq/_fp64_accum.py:1-29): the same codes and scales a reducer takes, with no rounding inside the
multiply -- the measuring stick that separates the operand format's error from the array's rounding error.

    Y = fp64_accum(P_A, X_A, P_B, X_B)     A^T B in float64 from the dequantized operands, float32 out

On the GPU: the dequantize kernel, then a float64 GEMM (hipBLAS).  The float64 sums run in a different order
from a CPU BLAS, so an output may differ from the reference's by one float32 ulp where the float64 sum lies
within a few float64 ulps of a float32 rounding boundary (stated tolerance: |diff| <= 1 float32 ulp).
"""
import torch

from .block import BLOCK, dequantize

__all__ = ["fp64_accum"]


def fp64_accum(P_A: torch.Tensor, X_A: torch.Tensor, P_B: torch.Tensor, X_B: torch.Tensor,
               block_size: int = BLOCK) -> torch.Tensor:
    """Y = A^T B in float64, float32 out; A is K x M, B is K x N."""
    A = dequantize(P_A, X_A, axis=0, block_size=block_size).to(torch.float64)
    B = dequantize(P_B, X_B, axis=0, block_size=block_size).to(torch.float64)
    return (A.t() @ B).to(torch.float32)
