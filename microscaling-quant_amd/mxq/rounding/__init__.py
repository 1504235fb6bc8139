"""mxq.rounding -- the three rounding rules of the MX datapath (mxq/rounding/__init__.py:1-85), on the GPU.

    mode        a tie goes                  used by
    ties_away   away from zero              qtorch's float_quantize (MXQuant)
    rne         to even                     lane accumulators, bf16, operand codes
    truncate    (no tie: drop the bits)     the PE product stage

    round_bits(bits, keep, mode)   int64 tensor of float32 bit patterns, rounded to keep `keep` fraction bits
                                   (keep an int or a tensor in [0, 22]); the carry runs into the exponent
    round_int(k, mode)             float32 / float64 tensor of integer-valued quantities rounded to integers
    bf16(x)                        float32 rounded to the bf16 grid nearest-even on its bit pattern; NaN passes

Each call is one elementwise kernel of libmxq_hip.so (round_bits, round_int, bf16 entry points).
"""
from typing import Union

import torch

from .. import _lib

MODES = ("ties_away", "rne", "truncate")

__all__ = ["MODES", "round_bits", "round_int", "bf16", "ties_away", "rne", "truncate"]


def _check_mode(mode: str) -> None:
    if mode not in MODES:
        raise ValueError(f"mode must be one of {MODES}, got {mode!r}")


def _keep_error():
    return ValueError("keep must be in [0, 22] (23 = identity is not a rounding)")


def round_bits(bits: torch.Tensor, keep: Union[int, torch.Tensor], mode: str) -> torch.Tensor:
    _check_mode(mode)
    if isinstance(keep, int):
        if not 0 <= keep <= 22:
            raise _keep_error()
        keep_t = None
    else:
        keep_t = torch.as_tensor(keep, dtype=torch.int64, device=bits.device)
        if bool((keep_t < 0).any()) or bool((keep_t > 22).any()):
            raise _keep_error()
    shape = bits.shape if keep_t is None else torch.broadcast_shapes(bits.shape, keep_t.shape)
    dev, b = _lib.ew_prepare(bits.expand(shape), torch.int64)
    out = torch.empty(shape, dtype=torch.int64, device=dev)
    kd = None
    if keep_t is not None:
        kd = _lib.to_device(keep_t, dev).expand(shape).contiguous()
    with _lib.on(dev):
        _lib.run("mxq_round_bits", _lib.ptr(b), _lib.ptr(kd), int(keep) if keep_t is None else 0, _lib.ptr(out),
                 out.numel(), _lib.MODE_CODE[mode], _lib.stream(dev))
    return _lib.back(out, bits)


def round_int(k: torch.Tensor, mode: str) -> torch.Tensor:
    _check_mode(mode)
    if k.dtype not in (torch.float32, torch.float64):
        raise TypeError(f"mxq.rounding.round_int: float32 or float64 input required, got {k.dtype}")
    dev, kd = _lib.ew_prepare(k, k.dtype)
    out = torch.empty_like(kd)
    with _lib.on(dev):
        _lib.run("mxq_round_int", _lib.ptr(kd), 0 if k.dtype == torch.float32 else 3, _lib.ptr(out), out.numel(),
                 _lib.MODE_CODE[mode], _lib.stream(dev))
    return _lib.back(out, k)


def _integer(k: torch.Tensor, mode: str) -> torch.Tensor:
    return round_int(k, mode)


def bf16(x: torch.Tensor) -> torch.Tensor:
    """Round to the bf16 grid, nearest-even, on the float32 bit pattern; float32 out, NaN unchanged.
    (Not a cast pair: the bit form is exact on subnormals, rounds the largest finite values to Inf as IEEE
    does, keeps the sign of +-0 and passes NaN through.)"""
    dev, xd = _lib.ew_prepare(x, torch.float32)
    out = torch.empty_like(xd)
    with _lib.on(dev):
        _lib.run("mxq_bf16", _lib.ptr(xd), _lib.ptr(out), out.numel(), _lib.stream(dev))
    return _lib.back(out, x)


from . import rne, ties_away, truncate  # noqa: E402  (they call back into round_int)
