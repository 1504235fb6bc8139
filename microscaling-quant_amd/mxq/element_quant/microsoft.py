"""The OCP reference's element step: microxcaling's `_quantize_elemwise` with `_quantize_mx`'s flags (saturate
out-of-range normals to max_norm, keep subnormals), mxq/element_quant/microsoft.py:18-23, on the GPU.

`rounding_mode` uses microxcaling's names: "nearest" (ties away), "even" (RNE) or "floor".  The float32
operation sequence is the reference's: private exponent floor(log2(|A|)) clipped at the format's min, scale
up, round the mantissa, scale back, clamp.  FP32 (pass-through) has no element format and is rejected.
Input is float32 (the block quantizers' only use); other dtypes are refused rather than silently recomputed
at a different precision.
"""
from typing import Union

import torch

from .. import _lib
from .formats import Format, get

__all__ = ["quantize"]

ROUNDINGS = ("nearest", "even", "floor")


def check_mode(rounding_mode: str) -> None:
    """microxcaling raises a plain Exception for a rounding method it does not know (elemwise.py:53-54)."""
    if rounding_mode == "dither":
        raise NotImplementedError("mxq.element_quant.microsoft: 'dither' draws random numbers; no bit-exact "
                                  "implementation exists, use 'even', 'nearest' or 'floor'")
    if rounding_mode not in ROUNDINGS:
        raise Exception("Unrecognized round method %s" % (rounding_mode))


def elementwise(z: torch.Tensor, f: Format, rounding_mode: str, saturate_normals: bool = True) -> torch.Tensor:
    check_mode(rounding_mode)
    if z.dtype != torch.float32:
        raise TypeError(f"mxq.element_quant.microsoft: float32 input required, got {z.dtype}")
    dev, zd = _lib.ew_prepare(z, torch.float32)
    out = torch.empty_like(zd)
    with torch.cuda.device(dev):
        _lib.run("mxq_microsoft", _lib.ptr(zd), _lib.ptr(out), out.numel(), f.e, f.ms_bits, f.max_norm,
                 _lib.MS_MODE_CODE[rounding_mode], int(saturate_normals), _lib.stream(dev))
    return _lib.back(out, z)


def quantize(z: torch.Tensor, fmt: Union[str, Format], rounding_mode: str = "even") -> torch.Tensor:
    f = get(fmt)
    if f is None:
        raise ValueError(f"{fmt!r} is pass-through (no element format); nothing to quantize")
    return elementwise(z, f, rounding_mode, True)
