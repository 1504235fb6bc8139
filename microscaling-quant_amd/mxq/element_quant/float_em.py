"""Element quantization to float(e, m) on one of three grids (mxq/element_quant/float_em.py:1-123), on the GPU.

    grid="qtorch"   qtorch 0.2.0 float_quantize: round the float32 bits at m, clip the biased exponent to
                    [127-L, 127+L] (L = 2^(e-1)-1): top exponent reserved, one binade of fake subnormals at
                    2^-L, flush below 2^(-L-1), saturate on overflow (NaN/Inf too)
    grid="ieee"     IEEE-like float(e, m): normals in [1-bias, bias], true subnormals, overflow -> Inf,
                    NaN/Inf/+-0 pass, underflow -> +0 (e < 8; e = 8 keeps the sign)
    grid="ocp"      the OCP MX element formats only: ieee's subnormals, the top exponent holds normals, values
                    beyond max_norm saturate; an exact +-0 becomes +0, a negative value rounding to zero -0

`rounding_mode` is one of mxq.rounding.MODES.  A float64 input is rounded from float64 (ieee, ocp) or first
cast to float32 (qtorch); any other input is cast to float32.  Output is float32.  (8, 23) is float32 itself.
One elementwise kernel per call (the mxq_float_em entry point).
"""
import torch

from .. import _lib
from ..rounding import MODES
from .formats import FORMATS

__all__ = ["quantize", "bias", "GRIDS"]

GRIDS = ("qtorch", "ieee", "ocp")


def bias(e: int) -> int:
    """Exponent bias of a float with e exponent bits: 2^(e-1) - 1."""
    return (1 << (e - 1)) - 1


def check(e: int, m: int, rounding_mode: str, grid: str) -> float:
    """The reference's argument checks, in its order; returns the ocp grid's max_norm (0 otherwise)."""
    if rounding_mode not in MODES:
        raise ValueError(f"rounding_mode must be one of {MODES}, got {rounding_mode!r}")
    if grid not in GRIDS:
        raise ValueError(f"grid must be one of {GRIDS}, got {grid!r}")
    if (e, m) == (8, 23):
        return 0.0
    if not (1 <= e <= 8 and 1 <= m <= 22):
        raise ValueError(f"unsupported widths e={e}, m={m}")
    if grid == "ocp":
        f = next((f for f in FORMATS.values() if (f.e, f.m) == (e, m)), None)
        if f is None:
            raise ValueError(f"grid='ocp' is defined only for the OCP element formats, not (e={e}, m={m})")
        return f.max_norm
    return 0.0


def quantize(z: torch.Tensor, e: int, m: int, rounding_mode: str = "ties_away", grid: str = "qtorch") -> torch.Tensor:
    max_norm = check(e, m, rounding_mode, grid)
    f64 = z.dtype == torch.float64
    dev, zd = _lib.ew_prepare(z, torch.float64 if f64 else torch.float32)
    out = torch.empty(zd.shape, dtype=torch.float32, device=dev)
    with _lib.on(dev):
        _lib.run("mxq_float_em", _lib.ptr(zd), 3 if f64 else 0, _lib.ptr(out), out.numel(), e, m,
                 _lib.MODE_CODE[rounding_mode], _lib.GRID_CODE[grid], max_norm, _lib.stream(dev))
    return _lib.back(out, z)
