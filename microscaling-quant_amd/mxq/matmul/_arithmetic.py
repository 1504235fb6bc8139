"""The three rounding points of a reducer as one object (mxq/matmul/_arithmetic.py:1-211).

    product(a, b)          multiply two codes, round to the product format
    acc_add(S, p, e, m)    add product p into the running sum S of an accumulator lane of format float(e, m)
    tile_add(C, tile)      add a finished, rescaled block sum into the output C

    stage        MXQUANT(prod_e, prod_m)                       MXGEMMINI(prod_e=4, prod_m=3, prod_floor=-16)
    product      fp32 a*b, then float_em ties_away on the      truncate_significand to prod_m fraction bits,
                 qtorch grid to float(prod_e, prod_m)          flush_product below 2^prod_floor, saturate with
                                                               spike's (limit, value) (e4m3: above 448 -> 448)
    acc_add      fp32 S+p, then float_em ties_away, qtorch     S and p each rounded rne on the ieee grid to the
                 grid, to float(e, m)                          lane (bf16 by bits for (8, 7)), +0 for zeros;
                                                               exact_add: exact sum, one rne rounding
    tile_add     fp32 C+tile                                   C and tile rounded rne to bf16, +0; exact_add to bf16

An Arithmetic built here also carries `kernel`: the description the systolic HIP kernel executes, so
matmul.systolic runs the whole K loop on the GPU.  The three callables remain, as GPU elementwise kernels,
for direct use and for reducers other than systolic.  An Arithmetic made by hand from arbitrary callables
(kernel None) still works with systolic, which then runs the reference's loop with those callables.

`compiled(arith)` returns the same Arithmetic under the name "compiled(...)": the HIP path is already one
fused kernel per call, so there is nothing left for torch.compile to fuse (and no Triton is used).
"""
from dataclasses import dataclass
from typing import Callable, Hashable, Optional, Sequence, Tuple

import torch

from .. import _lib, arith, rounding
from ..element_quant import float_em
from ..scale_factor import f32_scalar

__all__ = ["Arithmetic", "MXQUANT", "MXGEMMINI", "compiled", "KernelArith", "PROD_FLOOR"]

Tensor = torch.Tensor

#: products below 2^PROD_FLOOR flush to +0 (spike's mx_fp_math.h:63, the reference's recipe value)
PROD_FLOOR = -16


@dataclass(frozen=True)
class KernelArith:
    """What the systolic kernel needs to know about an Arithmetic (mxq_arith_spec)."""
    kind: int
    prod_e: int
    prod_m: int
    prod_floor: Optional[int] = None
    sat_limit: float = 0.0
    sat_value: float = 0.0

    def ctype(self) -> "_lib.ArithSpec":
        return _lib.ArithSpec(kind=self.kind, prod_e=self.prod_e, prod_m=self.prod_m,
                              has_floor=0 if self.prod_floor is None else 1,
                              flush_thr=0.0 if self.prod_floor is None else f32_scalar(2.0 ** self.prod_floor),
                              sat_limit=f32_scalar(self.sat_limit), sat_value=f32_scalar(self.sat_value))


@dataclass(frozen=True)
class Arithmetic:
    name: str
    product: Callable[[Tensor, Tensor], Tensor]
    acc_add: Callable[[Tensor, Tensor, int, int], Tensor]
    tile_add: Callable[[Tensor, Tensor], Tensor]
    fused_reduction: Optional[Callable[[Sequence[Tuple[int, int]], int], Callable]] = None
    fused_block: Optional[Callable[[Sequence[Tuple[int, int]], int, int], Callable]] = None
    fuse: Optional[Callable[[Hashable, Callable], Callable]] = None
    kernel: Optional[KernelArith] = None


def _canon(x: Tensor) -> Tensor:
    """A NaN made by arithmetic enters a qtorch rounding as the canonical quiet NaN (the kernels do the same)."""
    return torch.where(torch.isnan(x), torch.full_like(x, float("nan")), x)


def MXQUANT(prod_e: int, prod_m: int) -> Arithmetic:
    """MXQuant's `_simulate_atw` datapath: qtorch "nearest" on the fp32 product, on the fp32 lane sum; fp32 block add."""
    q = lambda x, e, m: float_em.quantize(_canon(x), e, m, rounding_mode="ties_away", grid="qtorch")  # noqa: E731
    float_em.check(prod_e, prod_m, "ties_away", "qtorch")
    return Arithmetic(
        name=f"mxquant(prod=e{prod_e}m{prod_m})",
        product=lambda a, b: q(a * b, prod_e, prod_m),
        acc_add=lambda S, p, e, m: q(S + p, e, m),
        tile_add=lambda C, tile: C + tile,
        kernel=KernelArith(_lib.ARITH_MXQUANT, prod_e, prod_m),
    )


def _saturation(prod_e: int, prod_m: int) -> Tuple[float, float]:
    """(limit, value) of spike's product saturation (mx_fp_math.h:42-56): above max_normal -> sign * sat_val.
    max_normal: e4m3 448 (mantissa 2^m - 2 at exponent b + 1), else 2^b * (2 - 2^-m);
    sat_val: 2^(b + 1) * (1 + (2^m - 2) / 2^m); Inf when beyond float32."""
    b = float_em.bias(prod_e)
    fp8 = (prod_e, prod_m) == (4, 3)
    limit = 2.0 ** (b + 1 if fp8 else b) * (1 + ((2 ** prod_m - 2) if fp8 else (2 ** prod_m - 1)) / 2 ** prod_m)
    value = 2.0 ** (b + 1) * (1 + (2 ** prod_m - 2) / 2 ** prod_m)
    if value > torch.finfo(torch.float32).max:
        value = float("inf")
    return limit, value


def _unsigned_zero(x: Tensor) -> Tensor:
    """-0 becomes +0: spike's lane and bf16 roundings never return a negative zero."""
    return torch.where(x == 0, torch.zeros_like(x), x)


def MXGEMMINI(prod_e: int = 4, prod_m: int = 3, prod_floor: Optional[int] = PROD_FLOOR) -> Arithmetic:
    """MX-Gemmini's PE column as spike computes it: product significand truncated to prod_m bits, flushed below
    2^prod_floor (None: no flush), saturated; both addends rounded rne to the lane, added exactly, rounded once;
    across blocks the same in bf16.  Every lane and bf16 rounding returns +0 for a zero."""
    limit, value = _saturation(prod_e, prod_m)
    rne = lambda x, e, m: (rounding.bf16(x) if (e, m) == (8, 7)                            # noqa: E731
                           else float_em.quantize(x, e, m, rounding_mode="rne", grid="ieee"))
    lane = lambda x, e, m: _unsigned_zero(rne(x, e, m))                                     # noqa: E731
    flush = (lambda x: x) if prod_floor is None else (lambda x: arith.flush_product(x, prod_floor))
    return Arithmetic(
        name=f"mxgemmini(prod=e{prod_e}m{prod_m})",
        product=lambda a, b: arith.saturate(flush(arith.truncate_significand(a * b, prod_m)), limit, value),
        acc_add=lambda S, p, e, m: arith.exact_add(lane(S, e, m), lane(p, e, m), e, m),
        tile_add=lambda C, tile: arith.exact_add(lane(C, 8, 7), lane(tile, 8, 7), 8, 7),
        kernel=KernelArith(_lib.ARITH_MXGEMMINI, prod_e, prod_m, prod_floor, limit, value),
    )


def compiled(arith_: Arithmetic) -> Arithmetic:
    """The same Arithmetic under the name "compiled(...)".  The systolic kernel already runs a whole call as one
    fused GPU kernel, bit-identical to the step-by-step rule, so no torch.compile graph is built."""
    return Arithmetic(name=f"compiled({arith_.name})", product=arith_.product, acc_add=arith_.acc_add,
                      tile_add=arith_.tile_add, fused_reduction=arith_.fused_reduction,
                      fused_block=arith_.fused_block, fuse=arith_.fuse, kernel=arith_.kernel)
