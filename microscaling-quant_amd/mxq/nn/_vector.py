"""Precision of the vector steps around the matmuls (mxq/nn/_vector.py:1-89).

A setting names, per op, how its steps round:
    None     the op as transformers writes it (float32 inside)
    "bf16"   the same steps in the same order, each result rounded to bfloat16 nearest-even at once

    softmax   in mxq.nn.attend      scores*scale and +mask (rounded by attend), then row max subtracted, exp,
                                    row sum, divide (the max itself is exact)
    rmsnorm   *RMSNorm forwards     square, mean, + eps, rsqrt, times rsqrt, times weight

Each step is one float32 torch op on bf16-valued inputs rounded once to bf16; for + - * / that equals a
correctly rounded bf16 operation (float32 carries more than 2*8+2 significant bits), exp and rsqrt are the
float32 library functions rounded once, and the long sums add in float32 and round once.

EXACT, the Scheme an attention module gets when softmax is set and no core rule chose it, computes Q K^T and
P V with no quantization: float32 operands, float64 sums, float32 result (mxq.fp64_accum).
"""
from functools import partial
from typing import Callable, Dict, Optional

import torch

from .. import rounding
from .._fp64_accum import fp64_accum
from ..block import mxgemmini
from ..scheme import Scheme

__all__ = ["OPS", "PRECISIONS", "EXACT", "resolve", "rounder", "softmax", "rmsnorm"]

#: ops a setting can name
OPS = ("softmax", "rmsnorm")

#: the precisions an op can have
PRECISIONS = (None, "bf16")

EXACT = Scheme("exact", a=partial(mxgemmini.quantize, fmt="FP32", axis=0),
               b=partial(mxgemmini.quantize, fmt="FP32", axis=0), reduce=fp64_accum)


def _valid(precision) -> bool:
    return precision is None or (isinstance(precision, str) and precision in PRECISIONS)


def resolve(vector) -> Dict[str, Optional[str]]:
    """None, "bf16" (every op) or {op: precision} (a missing op is None) -> {op: precision} over OPS."""
    if vector is None or isinstance(vector, str):
        table = dict.fromkeys(OPS, vector)
    elif isinstance(vector, dict):
        table = vector
    else:
        table = None
    if table is None or not set(table) <= set(OPS) or not all(_valid(p) for p in table.values()):
        raise ValueError(f"vector must be None, 'bf16' or {{op: None or 'bf16'}} with op in {OPS}, got {vector!r}")
    return {op: table.get(op) for op in OPS}


def _keep(x: torch.Tensor) -> torch.Tensor:
    return x


def _to_bf16(x: torch.Tensor) -> torch.Tensor:
    return rounding.bf16(x).to(x.dtype)


def rounder(precision: Optional[str]) -> Callable[[torch.Tensor], torch.Tensor]:
    """The rounding applied after each step (the tensor keeps its dtype)."""
    if not _valid(precision):
        raise ValueError(f"precision must be one of {PRECISIONS}, got {precision!r}")
    return _keep if precision is None else _to_bf16


def softmax(S: torch.Tensor, precision: Optional[str]) -> torch.Tensor:
    """Softmax over the last dim of scaled, masked scores: torch.softmax, or its four steps each rounded."""
    if precision is None:
        return torch.softmax(S, dim=-1)
    rnd = rounder(precision)
    shifted = rnd(S - S.amax(dim=-1, keepdim=True))
    num = rnd(torch.exp(shifted))
    return rnd(num / rnd(num.sum(dim=-1, keepdim=True)))


def rmsnorm(x: torch.Tensor, weight: torch.Tensor, eps: float, precision: Optional[str]) -> torch.Tensor:
    """transformers' LlamaRMSNorm forward (float32 inside, weight times the result cast back to x's dtype),
    its steps rounded by `precision`.  With None it is that forward op for op."""
    rnd = rounder(precision)
    h = x.to(torch.float32)
    mean_sq = rnd(rnd(h.pow(2)).mean(-1, keepdim=True))
    inv = rnd(torch.rsqrt(rnd(mean_sq + eps)))
    return rnd(weight * rnd(h * inv).to(x.dtype))
