"""What a PE does between quantizations (mxq/arith.py:1-137), as elementwise GPU kernels.

    exact_add(a, b, e, m)         a + b exactly, then one rounding to float(e, m); a zero addend returns the other
    truncate_significand(x, m)    keep m fraction bits of |x|'s significand (subnormals normalised), toward zero
    flush_product(x, floor_exp)   |x| < 2^floor_exp becomes +0
    saturate(x, limit, value)     |x| > limit becomes sign(x) * value (-0 -> +0, NaN stays)

exact_add keeps the reference's three evaluation paths, chosen on (e, m, rounding_mode, grid) alone: a float32
sum when two grid values always add exactly in float32 (2^e - 1 + m <= 24), Knuth's TwoSum pair for the other
lanes with e <= 7, and a float64 sum otherwise.  For grid inputs all three are the correctly rounded exact sum;
for arbitrary float32 inputs each path gives what the reference's gives.
"""
import torch

from . import _lib
from .element_quant import float_em
from .scale_factor import f32_scalar

__all__ = ["exact_add", "truncate_significand", "flush_product", "saturate"]


def _unary(name: str, x: torch.Tensor, *args) -> torch.Tensor:
    dev, xd = _lib.ew_prepare(x, torch.float32)
    out = torch.empty_like(xd)
    with _lib.on(dev):
        _lib.run(name, _lib.ptr(xd), _lib.ptr(out), out.numel(), *args, _lib.stream(dev))
    return _lib.back(out, x)


def exact_add(a: torch.Tensor, b: torch.Tensor, e: int, m: int, rounding_mode: str = "rne",
              grid: str = "ieee") -> torch.Tensor:
    """a + b computed exactly, then quantized once to float(e, m) (reference model fp_add_exact / bf16_accum_add).
    float32 operands (others are cast to float32 first)."""
    max_norm = float_em.check(e, m, rounding_mode, grid)
    dev = _lib.compute_device(a, b)
    shape = torch.broadcast_shapes(a.shape, b.shape)
    ad = _lib.to_device(a.detach(), dev).to(torch.float32).expand(shape).contiguous()
    bd = _lib.to_device(b.detach(), dev).to(torch.float32).expand(shape).contiguous()
    out = torch.empty(shape, dtype=torch.float32, device=dev)
    with _lib.on(dev):
        _lib.run("mxq_exact_add", _lib.ptr(ad), _lib.ptr(bd), _lib.ptr(out), out.numel(), e, m,
                 _lib.MODE_CODE[rounding_mode], _lib.GRID_CODE[grid], max_norm, _lib.stream(dev))
    return _lib.back(out, a)


def truncate_significand(x: torch.Tensor, m: int) -> torch.Tensor:
    """|x| = s * 2^E, s in [1, 2): keep m fraction bits of s, toward zero; zeros, Inf and NaN pass."""
    return _unary("mxq_truncate_significand", x, int(m))


def flush_product(x: torch.Tensor, floor_exp: int) -> torch.Tensor:
    """Zero (as +0) a value whose magnitude is below 2^floor_exp; everything else passes unchanged."""
    return _unary("mxq_flush_product", x, f32_scalar(2.0 ** floor_exp))


def saturate(x: torch.Tensor, limit: float, value: float) -> torch.Tensor:
    """sign(x) * value where |x| > limit, x elsewhere (+-Inf counts as above any finite limit)."""
    return _unary("mxq_saturate", x, f32_scalar(limit), f32_scalar(value))
