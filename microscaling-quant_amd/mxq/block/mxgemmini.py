"""mxq.block.mxgemmini -- MX-Gemmini's operand codes (mxq/block/mxgemmini.py:1-64).

    P, X = quantize(V, "MXFP8_E4M3", axis=0)        V_hat = dequantize(P, X, axis=0)

= scale_factor.mxquant (block max in [1, 2), no emax offset) then float_em on the OCP element grid (true
subnormals, saturate at max_norm); one fused kernel.  Knobs:
    rounding_mode   "ties_away" (default; the frozen RTL capture) or "rne" (the RTL since), or "truncate"
    scale_floor     scale_factor.MXQUANT_FLOOR (default) or HARDWARE_FLOOR = 2^-23
    via=(e, m)      round on the ieee float(e, m) grid first, same rounding (fmt="MXFP4", rounding_mode="rne",
                    via=(3, 1) is the fp4 requantizer's bf16 -> E3M1 -> E2M1)
"""
from typing import Optional, Tuple, Union

import torch

from .. import _lib
from ..element_quant import float_em
from ..element_quant.formats import Format, get
from ..scale_factor import MXQUANT_FLOOR, f32_scalar
from . import _driver

__all__ = ["quantize", "dequantize"]


@_lib.memo_spec
def spec(f: Format, rounding_mode: str, scale_floor: float, via: Optional[Tuple[int, int]]) -> _lib.BlockSpec:
    """The fused kernel's spec, after the reference's own checks (made when its element step runs)."""
    if via is not None:
        float_em.check(via[0], via[1], rounding_mode, "ieee")
    float_em.check(f.e, f.m, rounding_mode, "ocp")
    ve, vm = (0, 0) if via is None else (int(via[0]), int(via[1]))
    return _lib.BlockSpec(scale_rule=_lib.SCALE_MXQUANT, scale_floor=f32_scalar(scale_floor), elem=_lib.ELEM_OCP,
                          e=f.e, m=f.m, rounding=_lib.MODE_CODE[rounding_mode], max_norm=f.max_norm,
                          via_e=ve, via_m=vm)


def quantize(V: torch.Tensor, fmt: Union[str, Format], axis: int = 0, block_size: int = _driver.BLOCK,
             rounding_mode: str = "ties_away", scale_floor: float = MXQUANT_FLOOR,
             via: Optional[Tuple[int, int]] = None) -> Tuple[torch.Tensor, torch.Tensor]:
    """MX-Gemmini block quantize V along `axis`: (P codes, X power-of-two scales), float32."""
    f = get(fmt)
    if f is None:
        return _driver.quantize_fused(V, axis, block_size, _lib.BlockSpec())
    _driver._axis(V, axis)                      # IndexError before the element step's ValueErrors, as compose
    return _driver.quantize_fused(V, axis, block_size, spec(f, rounding_mode, scale_floor, via))


def dequantize(P: torch.Tensor, X: torch.Tensor, axis: int = 0, block_size: int = _driver.BLOCK) -> torch.Tensor:
    """V_hat = P * expand(X): each scale repeated block_size times along `axis`, cut to P's length."""
    return _driver.dequantize(P, X, axis, block_size)
