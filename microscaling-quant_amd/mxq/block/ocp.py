"""mxq.block.ocp -- OCP Microscaling v1.0 block quantization (mxq/block/ocp.py:1-54), codes and scales.

    P, X = quantize(V, "MXFP8_E4M3", axis=0)        V_hat = dequantize(P, X, axis=0)

= scale_factor.ocp (shared exponent floor(log2 amax) - emax, E8M0) then microxcaling's element step
(saturate, subnormals kept); one fused kernel.  P * expand(X) equals microxcaling's _quantize_mx.
`rounding_mode`: "even" (RNE), "nearest" (ties away), "floor", "dither" (uniforms drawn as the reference draws
them: for no_clip one per block maximum first, then one per element of the blocked, zero-padded tensor, on V's
device).  `placement` picks step 1:
    top         the spec: block max in the format's top binade, clipped to max_norm when it rounds above
    below_top   one binade down: never clips, the top binade unused
    no_clip     top, except the blocks that would clip go one binade down
"""
from typing import Tuple, Union

import torch

from .. import _lib
from ..element_quant.formats import Format, get
from ..element_quant.microsoft import check_mode
from ..scale_factor import _check_bits
from . import _driver

__all__ = ["quantize", "dequantize", "PLACEMENTS"]

PLACEMENTS = ("top", "below_top", "no_clip")


@_lib.memo_spec
def spec(f: Format, rounding_mode: str, scale_bits: int, placement: str) -> _lib.BlockSpec:
    _check_bits(scale_bits)
    check_mode(rounding_mode)
    rule = _lib.SCALE_OCP_NO_CLIP if placement == "no_clip" else _lib.SCALE_OCP
    emax = f.emax - 1 if placement == "below_top" else f.emax
    return _lib.BlockSpec(scale_rule=rule, scale_emax=emax, scale_bits=int(scale_bits), elem=_lib.ELEM_MICROSOFT,
                          e=f.e, m=f.ms_bits, rounding=_lib.MS_MODE_CODE[rounding_mode], max_norm=f.max_norm)


def quantize(V: torch.Tensor, fmt: Union[str, Format], axis: int = 0, block_size: int = _driver.BLOCK,
             rounding_mode: str = "even", scale_bits: int = 8,
             placement: str = "top") -> Tuple[torch.Tensor, torch.Tensor]:
    """OCP block quantize V along `axis`: (P codes, X power-of-two scales), float32."""
    f = get(fmt)
    if placement not in PLACEMENTS:
        raise ValueError(f"placement must be one of {PLACEMENTS}, got {placement!r}")
    if f is None:
        return _driver.quantize_fused(V, axis, block_size, _lib.BlockSpec())
    _driver._axis(V, axis)
    sp = spec(f, rounding_mode, scale_bits, placement)
    if rounding_mode == "dither":
        return _driver.quantize_dither(V, axis, block_size, sp)
    return _driver.quantize_fused(V, axis, block_size, sp)


def dequantize(P: torch.Tensor, X: torch.Tensor, axis: int = 0, block_size: int = _driver.BLOCK) -> torch.Tensor:
    """V_hat = P * expand(X): each scale repeated block_size times along `axis`, cut to P's length."""
    return _driver.dequantize(P, X, axis, block_size)
