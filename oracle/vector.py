"""Oracle vector steps with vector="bf16": softmax and RMSNorm with every step rounded to bfloat16.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

`softmax_bf16` follows mxq/nn/_vector.py:70-77 and `rmsnorm` mxq/nn/_vector.py:80-89: the same float32 steps in
the same order, each rounded to bf16 (nearest even) by numerics.bf16.  The three steps that are library
reductions or library functions in the reference -- exp, the row sum of the softmax and RMSNorm's mean of
squares, and rsqrt -- are taken as callables, as oracle/attend.py takes the softmax: the torch calls of the
device under test.  Their own bits are torch's; everything around them is pinned here.

Pins: the reference's outputs (tests/golden/vector.npz, written with torch's CPU exp, sum, mean and rsqrt),
reproduced bit for bit with those same CPU calls (tests/test_oracle_golden.py).
"""
import numpy as np

from . import numerics as nx

F32 = np.float32


def _identity(x):
    return x


def rounder(precision):
    """mxq/nn/_vector.py:61-67: None keeps the value, "bf16" rounds it to bf16 (nearest even), float32 kept."""
    return _identity if precision is None else (lambda x: nx.bf16(np.asarray(x, F32)))


def softmax_bf16(S, exp, rowsum):
    """mxq/nn/_vector.py:70-77 with precision "bf16": S - rowmax, exp, row sum, divide, each rounded.
    exp(x) and rowsum(x) (the sum over the last axis, kept as a column) are float32 callables."""
    r = rounder("bf16")
    S = np.asarray(S, F32)
    with np.errstate(all="ignore"):
        e = r(exp(r(S - S.max(axis=-1, keepdims=True))))
        return r((e / r(rowsum(e))).astype(F32))


def rmsnorm(x, weight, eps, precision, mean, rsqrt, x_bf16, w_bf16):
    """mxq/nn/_vector.py:80-89: h = float32(x); v = r(r(h^2).mean); h = r(h * r(rsqrt(r(v + eps)))); then
    r(weight * h cast to x's dtype), computed in the promoted dtype of weight and x (bf16 when both are bf16).
    x, weight: float32 arrays holding the values; x_bf16 / w_bf16: whether each is a bfloat16 tensor.
    mean(x) (over the last axis, kept as a column) and rsqrt(x) are float32 callables."""
    r = rounder(precision)
    h = np.asarray(x, F32)
    with np.errstate(all="ignore"):
        v = r(mean(r((h * h).astype(F32))))
        inv = r(rsqrt(r((v + F32(eps)).astype(F32))))
        h = r((h * inv).astype(F32))
        hx = nx.bf16(h) if x_bf16 else h                              # h.to(x.dtype)
        y = (np.asarray(weight, F32) * hx).astype(F32)                # exact for two bf16 factors
        if x_bf16 and w_bf16:
            y = nx.bf16(y)                                            # a bf16 result: rounded once
        return r(y)
