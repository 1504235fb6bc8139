"""MXLinear: an nn.Linear whose product runs through a Scheme, for inference (mxq/nn/_linear.py:1-80).

    y = MXLinear(linear, scheme)(x)      x: (..., in) -> (..., out), in x's dtype

Per call the tokens are flattened to an M x in float32 matrix; the Scheme computes Y = A^T B with A = x^T
(in x M, quantized by scheme.a) and B = W^T (in x out, quantized once by scheme.b and kept); the bias is added
in float32 and Y is cast to x's dtype.  This is MXQuant's MXLinearSim.forward.

Token rows may be computed in several calls: row m of Y depends on token m alone (scales run along `in` for
each token, and every product and rounding is per output), except that a LUT activation shares one table
among `scheme.rows` consecutive tokens, so a call always starts at a multiple of scheme.rows.  The result is
the same however the rows are cut.  On a GPU a larger call keeps more of the chip busy, so rows are cut only
to bound the size of one call's output.

`weight` and `bias` stay the wrapped layer's own Parameters (state_dict, .to() and tied weights behave as
before); the codes are non-persistent buffers, rebuilt by refresh().
"""
from typing import Optional

import torch
from torch import nn

from ..scheme import Scheme

__all__ = ["MXLinear"]

#: output elements (token rows x out) per reducer call when `chunk` is None: 1 GiB of float32
ELEMENTS_PER_CALL = 1 << 28


class MXLinear(nn.Module):
    """chunk: token rows per reducer call, a positive multiple of scheme.rows (None: ELEMENTS_PER_CALL decides).
    cache_weights: keep the weight codes (False: quantize the weight on every call)."""

    def __init__(self, linear: nn.Linear, scheme: Scheme, chunk: Optional[int] = None, cache_weights: bool = True):
        super().__init__()
        if chunk is not None:
            if chunk < 1:
                raise ValueError(f"chunk must be >= 1, got {chunk}")
            if chunk % scheme.rows:
                raise ValueError(f"chunk {chunk} must be a multiple of scheme {scheme.name!r} rows = {scheme.rows}")
        self.in_features = linear.in_features
        self.out_features = linear.out_features
        self.weight, self.bias = linear.weight, linear.bias
        self.scheme, self.chunk, self.cache_weights = scheme, chunk, cache_weights
        self.register_buffer("P_W", None, persistent=False)
        self.register_buffer("X_W", None, persistent=False)
        if cache_weights:
            self.refresh()

    @torch.no_grad()
    def refresh(self) -> None:
        """Quantize the current weight again into the cached codes and scales."""
        self.P_W, self.X_W = self._weight_codes()

    def _weight_codes(self):
        W_T = self.weight.detach().to(torch.float32).t().contiguous()              # in x out
        return self.scheme.b(W_T)

    def _rows_per_call(self, M: int) -> int:
        if self.chunk is not None:
            return self.chunk
        r = self.scheme.rows
        return max(r, ELEMENTS_PER_CALL // max(self.out_features, 1) // r * r)

    @torch.no_grad()
    def forward(self, x: torch.Tensor) -> torch.Tensor:
        lead = x.shape[:-1]
        tokens = x.reshape(-1, self.in_features).to(torch.float32)                 # M x in
        P_W, X_W = (self.P_W, self.X_W) if self.cache_weights else self._weight_codes()
        step = self._rows_per_call(tokens.shape[0])
        pieces = []
        for first in range(0, tokens.shape[0], step):
            A = tokens[first:first + step].t().contiguous()                         # in x m
            pieces.append(self.scheme.reduce(*self.scheme.a(A), P_W, X_W))         # m x out
        if not pieces:                                                              # no tokens
            pieces.append(self.scheme.reduce(*self.scheme.a(tokens.t().contiguous()), P_W, X_W))
        Y = pieces[0] if len(pieces) == 1 else torch.cat(pieces)
        if self.bias is not None:
            Y = Y + self.bias.to(torch.float32)
        return Y.to(x.dtype).reshape(*lead, self.out_features)

    def extra_repr(self) -> str:
        return f"in_features={self.in_features}, out_features={self.out_features}, scheme={self.scheme.name!r}"
