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
import math
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


class _QtorchStages:
    """MXQuant's rounding points: qtorch nearest (ties away) on the float32 product and on the float32 lane sum,
    plain float32 block adds."""

    def __init__(self, prod_e: int, prod_m: int):
        float_em.check(prod_e, prod_m, "ties_away", "qtorch")
        self.prod = (prod_e, prod_m)

    @staticmethod
    def _q(x: Tensor, e: int, m: int) -> Tensor:
        return float_em.quantize(_canon(x), e, m, rounding_mode="ties_away", grid="qtorch")

    def product(self, a: Tensor, b: Tensor) -> Tensor:
        return self._q(a * b, *self.prod)

    def acc_add(self, S: Tensor, p: Tensor, e: int, m: int) -> Tensor:
        return self._q(S + p, e, m)

    @staticmethod
    def tile_add(C: Tensor, tile: Tensor) -> Tensor:
        return C + tile


def MXQUANT(prod_e: int, prod_m: int) -> Arithmetic:
    """MXQuant's `_simulate_atw` datapath (mxq/matmul/_arithmetic.py:64-73)."""
    st = _QtorchStages(prod_e, prod_m)
    return Arithmetic(name=f"mxquant(prod=e{prod_e}m{prod_m})", product=st.product, acc_add=st.acc_add,
                      tile_add=st.tile_add, kernel=KernelArith(_lib.ARITH_MXQUANT, prod_e, prod_m))


def _saturation(prod_e: int, prod_m: int) -> Tuple[float, float]:
    """(limit, value) of the chip model's product saturation (mxq/matmul/_arithmetic.py:88-102): a product above
    `limit` becomes sign * `value`.  value = 2^(b+1) (2 - 2^(1-m)) (E4M3's 448), limit = value for E4M3 and the
    IEEE largest normal 2^b (2 - 2^-m) otherwise; a value beyond float32 is Inf."""
    b = float_em.bias(prod_e)
    value = math.ldexp(2.0 - math.ldexp(1.0, 1 - prod_m), b + 1)
    limit = value if (prod_e, prod_m) == (4, 3) else math.ldexp(2.0 - math.ldexp(1.0, -prod_m), b)
    return limit, (value if value <= torch.finfo(torch.float32).max else math.inf)


def _unsigned_zero(x: Tensor) -> Tensor:
    """-0 becomes +0: the chip model's lane and bf16 roundings never return a negative zero."""
    return torch.where(x == 0, torch.zeros_like(x), x)


class _GemminiStages:
    """MX-Gemmini's PE column: the product's significand truncated to prod_m bits, flushed below 2^prod_floor
    (None: no flush), saturated; a lane add rounds both addends to the lane's float(e, m) (bf16 on the bit
    pattern), adds exactly and rounds once; the block add is the same in bf16.  Zeros come out as +0."""

    def __init__(self, prod_e: int, prod_m: int, prod_floor: Optional[int]):
        self.prod_m, self.prod_floor = prod_m, prod_floor
        self.limit, self.value = _saturation(prod_e, prod_m)

    @staticmethod
    def lane(x: Tensor, e: int, m: int) -> Tensor:
        r = rounding.bf16(x) if (e, m) == (8, 7) else float_em.quantize(x, e, m, rounding_mode="rne", grid="ieee")
        return _unsigned_zero(r)

    def product(self, a: Tensor, b: Tensor) -> Tensor:
        t = arith.truncate_significand(a * b, self.prod_m)
        if self.prod_floor is not None:
            t = arith.flush_product(t, self.prod_floor)
        return arith.saturate(t, self.limit, self.value)

    def acc_add(self, S: Tensor, p: Tensor, e: int, m: int) -> Tensor:
        return arith.exact_add(self.lane(S, e, m), self.lane(p, e, m), e, m)

    def tile_add(self, C: Tensor, tile: Tensor) -> Tensor:
        return self.acc_add(C, tile, 8, 7)


def MXGEMMINI(prod_e: int = 4, prod_m: int = 3, prod_floor: Optional[int] = PROD_FLOOR) -> Arithmetic:
    """MX-Gemmini's PE column as the chip's reference model computes it (mxq/matmul/_arithmetic.py:111-134)."""
    st = _GemminiStages(prod_e, prod_m, prod_floor)
    return Arithmetic(name=f"mxgemmini(prod=e{prod_e}m{prod_m})", product=st.product, acc_add=st.acc_add,
                      tile_add=st.tile_add,
                      kernel=KernelArith(_lib.ARITH_MXGEMMINI, prod_e, prod_m, prod_floor, st.limit, st.value))


def compiled(arith: Arithmetic) -> Arithmetic:
    """The same Arithmetic under the name "compiled(...)" (mxq/matmul/_arithmetic.py:154-211).  The systolic kernel
    already runs a whole call as one fused GPU kernel, bit-identical to the step-by-step rule, so no torch.compile
    graph is built."""
    return Arithmetic(name=f"compiled({arith.name})", product=arith.product, acc_add=arith.acc_add,
                      tile_add=arith.tile_add, fused_reduction=arith.fused_reduction,
                      fused_block=arith.fused_block, fuse=arith.fuse, kernel=arith.kernel)
