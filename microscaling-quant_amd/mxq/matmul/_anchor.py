"""The anchor tree (mxq/matmul/_anchor.py:1-138), MxGen's MxAnchorAccTree as a reducer with systolic's call.

A reduction of `size` products is size / width trees chained through a running sum c.  One tree:

    S1  anchor: the largest label among its nonzero products and c, plus headroom.  A product's label is
        e(a) + e(b), e(x) = floor(log2|x|) of the code (frexp's; at least `emin` when given); c's label is
        floor(log2|c|) - 1
    S2  every term (the width products, then c) cut to an integer on the grid 2^(anchor + 2 - bits[0]):
        toward zero ("truncate") or to nearest even ("rne")
    S3  adjacent pairs added level by level, an odd last term passed up; where the next level is narrower,
        every term is cut again onto its grid
    S4  the root, one rounding to float32, then the Arithmetic's lane rounding to schedule[t]

Defaults: headroom max(4, ceil(log2(width + 1)) + 1); every level (m + 1) + headroom + ceil(log2(width + 1)) + 1
bits; drop "truncate".  K tail: missing products are zeros.

With MXGEMMINI or MXQUANT (or compiled(...) of them), size dividing 32 and integer widths, the whole call is one
HIP launch (include/mxq_hip.h mxq_anchor_tree): one thread per output, each tree's terms held in registers as
exact integers.  For MXGEMMINI without emin, bf16 trees and equal level widths (the defaults) a fast kernel runs
first and the general one computes only the tiles whose codes it could not take.  Otherwise the reference's loop runs with the Arithmetic's callables on the operands'
device.
"""
import math
from typing import Optional, Sequence, Tuple

import torch

from .. import _lib
from ..block import BLOCK
from ._arithmetic import Arithmetic
from ._common import check_operands, check_schedule, scale_map
from ._systolic import _lanes_check, workspace_elements

__all__ = ["anchor_tree", "DROPS"]

DROPS = ("truncate", "rne")


def _levels_for(width: int) -> int:
    """Addition levels for width + 1 terms."""
    return math.ceil(math.log2(width + 1))


def anchor_tree(P_A: torch.Tensor, X_A: torch.Tensor, P_B: torch.Tensor, X_B: torch.Tensor,
                arith: Arithmetic, schedule: Optional[Sequence[Tuple[int, int]]] = None, size: int = 16,
                block_size: int = BLOCK, *, width: Optional[int] = None, bits: Optional[Sequence[int]] = None,
                drop: str = "truncate", headroom: Optional[int] = None, emin: Optional[int] = None,
                force_general: bool = False) -> torch.Tensor:
    """Y = A^T B, each reduction of `size` products summed by chained anchor trees of `width` products.
    `schedule`: one (e, m) per tree (default bf16).  `force_general` (not in the reference) runs the general
    kernel even where the fast one applies; the two are bit-identical."""
    K, M, N = check_operands(P_A, X_A, P_B, X_B, block_size)
    width = size if width is None else width
    if width < 1 or size % width or block_size % size:
        raise ValueError(f"width {width} must divide size {size}, and size must divide block size {block_size}")
    trees = size // width
    schedule = [(8, 7)] * trees if schedule is None else list(schedule)
    check_schedule(schedule, trees)
    if drop not in DROPS:
        raise ValueError(f"drop must be one of {DROPS}, got {drop!r}")
    lg = _levels_for(width)
    head = max(4, lg + 1) if headroom is None else headroom
    if head < lg + 1:
        raise ValueError(f"headroom {head} < {lg + 1}: the sum of {width + 1} terms could overflow")

    def level_widths(m):
        widths = [(m + 1) + head + lg + 1] * (lg + 1) if bits is None else list(bits)
        if len(widths) != lg + 1 or max(widths) > 24 or any(a < b for a, b in zip(widths, widths[1:])):
            raise ValueError(f"bits needs {lg + 1} non-increasing entries, each <= 24; got {widths}")
        return widths

    per_tree = [(e, m, level_widths(m)) for e, m in schedule]
    kernel = getattr(arith, "kernel", None)
    integral = all(isinstance(v, int) for v in (head, emin if emin is not None else 0)) and \
        all(isinstance(b, int) and b >= 1 for _, _, ws in per_tree for b in ws)
    if kernel is None or 32 % size or not integral or not (lg + 1 <= head <= 64) or \
            (emin is not None and abs(emin) > 1000):
        return _stage_loop(P_A, X_A, P_B, X_B, arith, per_tree, size, block_size, width, drop, head, emin, K, M, N)
    if K > 0:
        _lanes_check(kernel, schedule, trees)
    dev = _lib.compute_device(P_A)
    ops = [_lib.to_device(t.detach(), dev).contiguous() for t in (P_A, X_A, P_B, X_B)]
    C = torch.empty((M, N), dtype=torch.float32, device=dev)
    if M == 0 or N == 0:
        return _lib.back(C, P_A)
    import ctypes
    te = (ctypes.c_int32 * trees)(*[int(e) for e, _, _ in per_tree])
    tm = (ctypes.c_int32 * trees)(*[int(m) for _, m, _ in per_tree])
    tb = (ctypes.c_int32 * (trees * (lg + 1)))(*[int(b) for _, _, ws in per_tree for b in ws])
    spec = _lib.AnchorSpec(width=width, drop=DROPS.index(drop), headroom=head, has_emin=int(emin is not None),
                           emin=0 if emin is None else emin, nbits=lg + 1)
    work = torch.empty(workspace_elements(K, M, N, 1), dtype=torch.int32, device=dev)
    with _lib.on(dev):
        _lib.run("mxq_anchor_tree", *(_lib.ptr(t) for t in ops), _lib.ptr(C), K, M, N, te, tm, tb, size, block_size,
                 ctypes.byref(spec), kernel.ctype(), _lib.ptr(work), int(force_general), _lib.stream(dev))
    return _lib.back(C, P_A)


# ---------------------------------------------------------------- the reference's loop, Arithmetic callables
def _label(x: torch.Tensor) -> torch.Tensor:
    """floor(log2|x|) by frexp, float64; non-finite values count as 0.5 (label -1); zeros' labels are unused."""
    x = torch.where(torch.isfinite(x), x, torch.full_like(x, 0.5))
    return (torch.frexp(x.abs())[1] - 1).to(torch.float64)


def _cut(x: torch.Tensor, drop: str) -> torch.Tensor:
    return torch.trunc(x) if drop == "truncate" else torch.round(x)


def _one_tree(prods, labels, c, e, m, widths, drop, head, arith):
    none = torch.full(c.shape, -math.inf, dtype=torch.float64, device=c.device)
    top = torch.where(c != 0, _label(c) - 1, none)
    for p, lab in zip(prods, labels):
        top = torch.maximum(top, torch.where(p != 0, lab, none))
    anchor = torch.where(torch.isfinite(top), top, torch.zeros_like(top)) + head
    step = torch.exp2(anchor + 2 - widths[0])
    terms = [_cut(v.to(torch.float64) / step, drop) for v in prods + [c]]
    for lvl in range(1, len(widths)):
        nxt = [terms[2 * i] + terms[2 * i + 1] for i in range(len(terms) // 2)]
        if len(terms) % 2:
            nxt.append(terms[-1])
        if widths[lvl] != widths[lvl - 1]:
            nxt = [_cut(v / 2.0 ** (widths[lvl - 1] - widths[lvl]), drop) for v in nxt]
        terms = nxt
    root = (terms[0] * torch.exp2(anchor + 2 - widths[-1])).to(torch.float32)
    return arith.acc_add(torch.zeros_like(c), root, e, m)


def _stage_loop(P_A, X_A, P_B, X_B, arith, per_tree, size, block_size, width, drop, head, emin, K, M, N):
    la, lb = _label(P_A), _label(P_B)
    if emin is not None:
        la, lb = la.clamp(min=emin), lb.clamp(min=emin)
    C = torch.zeros((M, N), dtype=torch.float32, device=P_A.device)
    zero = torch.zeros((M, N), dtype=torch.float32, device=P_A.device)
    for g in range(0, K, block_size):
        g_end = min(g + block_size, K)
        scales = scale_map(X_A, X_B, g // block_size)
        for k0 in range(g, g_end, size):
            k1 = min(k0 + size, g_end)
            c = zero
            for t, (e, m, widths) in enumerate(per_tree):
                ks = range(k0 + t * width, min(k0 + (t + 1) * width, k1))
                prods = [arith.product(P_A[k].unsqueeze(1), P_B[k].unsqueeze(0)) for k in ks]
                labels = [la[k].unsqueeze(1) + lb[k].unsqueeze(0) for k in ks]
                prods += [zero] * (width - len(prods))
                labels += [zero.to(torch.float64)] * (width - len(labels))
                c = _one_tree(prods, labels, c, e, m, widths, drop, head, arith)
            C = arith.tile_add(C, c * scales)
    return C.to(torch.float32)
