"""mxq.scale_factor -- step 1 of block quantization: the per-block scale X = f(amax) (mxq/scale_factor.py:1-81).

    mxquant(amax, floor)         X = 2^floor(log2 max(amax, floor)), floored at `floor`; block max in [1, 2)
    ocp(amax, emax)              X = 2^(floor(log2 amax) - emax), E8M0 range: NaN above, clamp below
    ocp_below_top(amax, emax)    ocp with emax - 1: the block max one binade below the top, never clipped
    ocp_no_clip(amax, fmt)       ocp's X, doubled for the blocks whose max would clip

floor(log2 amax) is the reference's floor of a correctly rounded float32 log2: just below a power of two it
rounds up, so the block max can land at 1 - 2^-24 rather than in [1, 2).  The kernels reproduce that with an
exact per-binade threshold table.

    MXQUANT_FLOOR   1e-38   MXQuant's simulation (a float32 subnormal; the resulting X is not a power of two)
    HARDWARE_FLOOR  2^-23   MXQuant's end_to_end_linear quantizer and the MX-Gemmini requantizer (FLT_EPSILON)

Each call is one elementwise kernel (mxq_scale_factor); inside block quantization the same device code runs
fused in the quantize kernel.
"""
import numpy as np
import torch

from . import _lib

__all__ = ["mxquant", "ocp", "ocp_below_top", "ocp_no_clip", "MXQUANT_FLOOR", "HARDWARE_FLOOR"]

MXQUANT_FLOOR = 1e-38
HARDWARE_FLOOR = 2.0 ** -23
FP32_MIN_NORMAL = 2.0 ** -126


def f32_scalar(x: float) -> float:
    """The float32 value torch gives a Python float scalar meeting a float32 tensor."""
    return float(np.float32(x))


def mxquant_spec(floor: float) -> _lib.BlockSpec:
    return _lib.BlockSpec(scale_rule=_lib.SCALE_MXQUANT, scale_floor=f32_scalar(floor))


def _check_bits(scale_bits: int) -> None:
    if not isinstance(scale_bits, int) or not 1 <= scale_bits <= 30:
        raise ValueError(f"mxq.scale_factor: scale_bits {scale_bits!r} must be an integer in [1, 30]")


def ocp_spec(emax: int, scale_bits: int) -> _lib.BlockSpec:
    _check_bits(scale_bits)
    return _lib.BlockSpec(scale_rule=_lib.SCALE_OCP, scale_emax=int(emax), scale_bits=int(scale_bits))


def ocp_no_clip_spec(f, rounding_mode: str, scale_bits: int) -> _lib.BlockSpec:
    _check_bits(scale_bits)
    return _lib.BlockSpec(scale_rule=_lib.SCALE_OCP_NO_CLIP, scale_emax=f.emax, scale_bits=int(scale_bits),
                          elem=_lib.ELEM_MICROSOFT, e=f.e, m=f.ms_bits, rounding=_lib.MS_MODE_CODE[rounding_mode],
                          max_norm=f.max_norm)


def _apply(amax: torch.Tensor, spec: _lib.BlockSpec) -> torch.Tensor:
    if amax.dtype != torch.float32:
        raise TypeError(f"mxq.scale_factor: float32 block maxima required, got {amax.dtype}")
    dev, a = _lib.ew_prepare(amax, torch.float32)
    out = torch.empty_like(a)
    with _lib.on(dev):
        _lib.run("mxq_scale_factor", _lib.ptr(a), _lib.ptr(out), out.numel(), spec, _lib.stream(dev))
    return _lib.back(out, amax)


def mxquant(amax: torch.Tensor, floor: float = MXQUANT_FLOOR) -> torch.Tensor:
    """MXQuant's scale: 2^floor(log2 max(amax, floor)), floored at `floor`."""
    return _apply(amax, mxquant_spec(floor))


def ocp(amax: torch.Tensor, emax: int, scale_bits: int = 8) -> torch.Tensor:
    """OCP's scale 2^(floor(log2 amax) - emax) with microxcaling's E8M0 range handling: a zero block uses
    2^-126 for the log; a shared exponent above 2^(scale_bits-1)-1 is NaN, below its negative is clamped."""
    return _apply(amax, ocp_spec(emax, scale_bits))


def ocp_below_top(amax: torch.Tensor, emax: int, scale_bits: int = 8) -> torch.Tensor:
    """OCP's scale times two: the block max lands one binade below the format's top and is never clipped."""
    return ocp(amax, emax - 1, scale_bits)


def ocp_no_clip(amax: torch.Tensor, fmt, rounding_mode: str = "even", scale_bits: int = 8) -> torch.Tensor:
    """OCP's scale, doubled for exactly the blocks whose max, rounded to the format the way the elements are
    (microxcaling, `rounding_mode`, no saturation), exceeds max_norm."""
    from .element_quant.formats import get
    from .element_quant.microsoft import check_mode
    f = get(fmt)
    if f is None:
        raise ValueError(f"{fmt!r} is pass-through (no element format); it has no scale")
    check_mode(rounding_mode)
    spec = ocp_no_clip_spec(f, rounding_mode, scale_bits)
    if rounding_mode != "dither":
        return _apply(amax, spec)
    # dither rounds amax / X with one draw per maximum, as rand_like(amax / X) (mxq/scale_factor.py:78-80)
    from .element_quant.microsoft import draws
    if amax.dtype != torch.float32:
        raise TypeError(f"mxq.scale_factor: float32 block maxima required, got {amax.dtype}")
    u = draws(amax, amax.numel())
    dev, a = _lib.ew_prepare(amax, torch.float32)
    out = torch.empty_like(a)
    with _lib.on(dev):
        _lib.run("mxq_scale_factor_dither", _lib.ptr(a), _lib.ptr(_lib.to_device(u, dev)), _lib.ptr(out),
                 out.numel(), spec, _lib.stream(dev))
    return _lib.back(out, amax)
