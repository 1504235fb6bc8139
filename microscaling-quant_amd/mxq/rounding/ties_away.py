"""Round to nearest, ties away from zero (mxq/rounding/ties_away.py): qtorch's "nearest"."""
import torch

from . import _integer


def bits(bits: torch.Tensor, drop, mask, half) -> torch.Tensor:
    """One step of round_bits on int64 patterns: (bits + half) & ~mask (no 32-bit wrap)."""
    return (bits + half) & ~mask


def integer(k: torch.Tensor) -> torch.Tensor:
    """sign(k) * floor(|k| + 0.5), evaluated in k's dtype."""
    return _integer(k, "ties_away")
