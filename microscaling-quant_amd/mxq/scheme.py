"""mxq.scheme -- one explicit chain for one matmul (mxq/scheme.py:1-68).

    Scheme(name, a, b, reduce, rows=1, block_size=32)
        a(V) -> (P, X)    operand A (K x M, blocks along K) to codes and scales
        b(V) -> (P, X)    operand B (K x N)
        reduce(P_A, X_A, P_B, X_B) -> Y    a dataflow with its Arithmetic and schedule bound
        rows              columns of A that `a` must see in one call (a LUT operand shares a table over 2^G)
        block_size        the block length along K that a and b use
    Scheme.matmul(A, B) = reduce(*a(A), *b(B)), Y = A^T B
"""
import math
from dataclasses import dataclass
from typing import Callable, Tuple

import torch

from .block import BLOCK

__all__ = ["Scheme"]

Tensor = torch.Tensor
Quantizer = Callable[[Tensor], Tuple[Tensor, Tensor]]
Reducer = Callable[[Tensor, Tensor, Tensor, Tensor], Tensor]


@dataclass(frozen=True)
class Scheme:
    name: str
    a: Quantizer
    b: Quantizer
    reduce: Reducer
    rows: int = 1
    block_size: int = BLOCK

    def __post_init__(self):
        for field in ("rows", "block_size"):
            v = getattr(self, field)
            if not isinstance(v, int) or isinstance(v, bool) or v < 1:
                raise ValueError(f"Scheme: {field} {v!r} must be a positive integer")

    def check_scales(self, X: Tensor, K: int, operand: str) -> None:
        """X must hold one row of scales per block_size of K."""
        need = math.ceil(K / self.block_size)
        if X.shape[0] != need:
            raise ValueError(f"Scheme {self.name!r}: {operand} has {X.shape[0]} scale rows for K = {K}, "
                             f"block_size {self.block_size} needs {need}; "
                             "the Scheme's block_size and its quantizer's disagree")

    def matmul(self, A: Tensor, B: Tensor) -> Tensor:
        """Y = A^T B for A: K x M and B: K x N."""
        P_A, X_A = self.a(A)
        P_B, X_B = self.b(B)
        self.check_scales(X_A, A.shape[0], "a")
        self.check_scales(X_B, B.shape[0], "b")
        return self.reduce(P_A, X_A, P_B, X_B)
