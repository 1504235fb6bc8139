"""mxq.block.mxquant -- MXQuant's block quantization (mxq/block/mxquant.py:1-37): the codes of every MXQuant
linear-layer simulation.

    P, X = quantize(V, "MXFP8_E4M3", axis=0)        V_hat = dequantize(P, X, axis=0)

= scale_factor.mxquant (X = 2^floor(log2 amax), block max in [1, 2), floor 1e-38) then float_em on the qtorch
grid, ties away from zero; one fused kernel.  FP32 is the pass-through.
"""
from typing import Tuple, Union

import torch

from .. import _lib
from ..element_quant.formats import Format, get
from ..scale_factor import MXQUANT_FLOOR, f32_scalar
from . import _driver

__all__ = ["quantize", "dequantize"]


@_lib.memo_spec
def spec(f: Format) -> _lib.BlockSpec:
    return _lib.BlockSpec(scale_rule=_lib.SCALE_MXQUANT, scale_floor=f32_scalar(MXQUANT_FLOOR),
                          elem=_lib.ELEM_QTORCH, e=f.e, m=f.m, rounding=_lib.MODE_CODE["ties_away"])


def quantize(V: torch.Tensor, fmt: Union[str, Format], axis: int = 0,
             block_size: int = _driver.BLOCK) -> Tuple[torch.Tensor, torch.Tensor]:
    """MXQuant-simulation block quantize V along `axis`: (P codes, X power-of-two scales), float32."""
    f = get(fmt)
    return _driver.quantize_fused(V, axis, block_size, _lib.BlockSpec() if f is None else spec(f))


def dequantize(P: torch.Tensor, X: torch.Tensor, axis: int = 0, block_size: int = _driver.BLOCK) -> torch.Tensor:
    """V_hat = P * expand(X): each scale repeated block_size times along `axis`, cut to P's length."""
    return _driver.dequantize(P, X, axis, block_size)
