"""Truncate toward zero (mxq/rounding/truncate.py): drop the low bits; the PE product stage."""
import torch

from . import _integer


def bits(bits: torch.Tensor, drop, mask, half) -> torch.Tensor:
    """One step of round_bits on int64 patterns: bits & ~mask."""
    return bits & ~mask


def integer(k: torch.Tensor) -> torch.Tensor:
    """trunc(k)."""
    return _integer(k, "truncate")
