"""The OCP reference's element step: microxcaling's `_quantize_elemwise` with `_quantize_mx`'s flags (saturate
out-of-range normals to max_norm, keep subnormals), mxq/element_quant/microsoft.py:18-23, on the GPU.

`rounding_mode` uses microxcaling's names: "nearest" (ties away), "even" (RNE), "floor", or "dither"
(floor(|A| + u) with u from torch.rand_like of the tensor rounded, drawn here as the reference draws it: on the
input's device, from torch's default generator for that device).  The float32
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

ROUNDINGS = ("nearest", "even", "floor", "dither")


def check_mode(rounding_mode: str) -> None:
    """microxcaling raises a plain Exception for a rounding method it does not know (elemwise.py:53-54)."""
    if rounding_mode not in ROUNDINGS:
        raise Exception("Unrecognized round method %s" % (rounding_mode))


def draws(like: torch.Tensor, numel: int) -> torch.Tensor:
    """`numel` uniforms in [0, 1) as torch.rand_like of a float32 tensor of that many elements on `like`'s device
    draws them (mxq/microxcaling/elemwise.py:42), flat."""
    return torch.rand(numel, dtype=torch.float32, device=like.device)


def elementwise(z: torch.Tensor, f: Format, rounding_mode: str, saturate_normals: bool = True) -> torch.Tensor:
    check_mode(rounding_mode)
    if z.dtype != torch.float32:
        raise TypeError(f"mxq.element_quant.microsoft: float32 input required, got {z.dtype}")
    u = draws(z, z.numel()) if rounding_mode == "dither" else None
    dev, zd = _lib.ew_prepare(z, torch.float32)
    out = torch.empty_like(zd)
    with _lib.on(dev):
        if u is None:
            _lib.run("mxq_microsoft", _lib.ptr(zd), _lib.ptr(out), out.numel(), f.e, f.ms_bits, f.max_norm,
                     _lib.MS_MODE_CODE[rounding_mode], int(saturate_normals), _lib.stream(dev))
        else:
            ud = _lib.to_device(u, dev)
            _lib.run("mxq_microsoft_dither", _lib.ptr(zd), _lib.ptr(ud), _lib.ptr(out), out.numel(), f.e, f.ms_bits,
                     f.max_norm, int(saturate_normals), _lib.stream(dev))
    return _lib.back(out, z)


def quantize(z: torch.Tensor, fmt: Union[str, Format], rounding_mode: str = "even") -> torch.Tensor:
    f = get(fmt)
    if f is None:
        raise ValueError(f"{fmt!r} is pass-through (no element format); nothing to quantize")
    return elementwise(z, f, rounding_mode, True)
