"""Round to nearest, ties to even (mxq/rounding/rne.py): IEEE 754's default, hardfloat's round_near_even.
Bit form: add (half - 1 + lsb) and drop the low bits, so an exact tie rounds up only when the kept LSB is 1."""
import torch

from . import _integer


def bits(bits: torch.Tensor, drop, mask, half) -> torch.Tensor:
    """One step of round_bits on int64 patterns: (bits + half - 1 + lsb) & ~mask (no 32-bit wrap)."""
    lsb = (bits >> drop) & 1
    return (bits + half - 1 + lsb) & ~mask


def integer(k: torch.Tensor) -> torch.Tensor:
    """Integer-valued k rounded half to even (torch.round)."""
    return _integer(k, "rne")
