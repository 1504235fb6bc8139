"""The systolic PE column (mxq/matmul/_systolic.py:1-62): Y = A^T B in the hardware's summation order.

For each block of K its scale map; for each reduction of `size` k inside it a fresh sum, one product per k
rounded by the Arithmetic's product, accumulated in lane k % size's format from `schedule`; the finished sum
is multiplied by the scale map and added into the output by tile_add.  `size` must divide `block_size`.
K tail: the last reduction leaves the column after its last real product, as MXQuant's `_simulate_atw`.

With MXGEMMINI or MXQUANT (or compiled(...) of them) the whole call is one HIP launch sequence on the GPU
(include/mxq_hip.h mxq_systolic): every output element's chain is computed in order by one thread, the K
loop staged through LDS.  A hand-made Arithmetic, or a size the kernel does not take (it needs size | 32),
runs the reference's loop with the Arithmetic's own callables.
"""
from typing import Optional, Sequence, Tuple

import torch

from .. import _lib
from ..block import BLOCK
from ..element_quant import float_em
from ._arithmetic import Arithmetic, KernelArith
from ._common import check_operands, check_schedule, scale_map

__all__ = ["systolic"]


def _lanes_check(kernel: KernelArith, schedule, used: int) -> None:
    """The checks the reference's lane roundings make the first time each lane runs."""
    for e, m in list(schedule)[:used]:
        if kernel.kind == _lib.ARITH_MXGEMMINI:
            if (e, m) == (8, 7):
                continue
            float_em.check(e, m, "rne", "ieee")
        else:
            float_em.check(e, m, "ties_away", "qtorch")


def systolic(P_A: torch.Tensor, X_A: torch.Tensor, P_B: torch.Tensor, X_B: torch.Tensor,
             arith: Arithmetic, schedule: Sequence[Tuple[int, int]], size: int = 16,
             block_size: int = BLOCK, *, force_general: bool = False) -> torch.Tensor:
    """Y = A^T B.  A: K x M codes, X_A: ceil(K/block_size) x M scales; B: K x N, X_B: ceil(K/block_size) x N.
    Y: M x N float32 on the operands' device.  `force_general` (not in the reference) runs the general kernel
    even where the fast one applies; the two are bit-identical."""
    K, M, N = check_operands(P_A, X_A, P_B, X_B, block_size)
    check_schedule(schedule, size)
    if block_size % size != 0:
        raise ValueError(f"size {size} must divide block size {block_size}")
    kernel = getattr(arith, "kernel", None)
    if kernel is None or size > 64 or 32 % size != 0:
        return _reference_loop(P_A, X_A, P_B, X_B, arith, schedule, size, block_size, K, M, N)
    if K > 0:
        _lanes_check(kernel, schedule, min(size, K))
    dev = _lib.compute_device(P_A)
    ops = [_lib.to_device(t.detach(), dev).contiguous() for t in (P_A, X_A, P_B, X_B)]
    if K == 0 or M == 0 or N == 0:
        return _lib.back(torch.zeros((M, N), dtype=torch.float32, device=dev), P_A)
    C = torch.empty((M, N), dtype=torch.float32, device=dev)          # every element is written
    import ctypes
    le = (ctypes.c_int32 * size)(*[int(e) for e, _ in schedule])
    lm = (ctypes.c_int32 * size)(*[int(m) for _, m in schedule])
    work = torch.empty(workspace_elements(K, M, N, 1), dtype=torch.int32, device=dev)
    with _lib.on(dev):
        _lib.run("mxq_systolic", *(_lib.ptr(t) for t in ops), _lib.ptr(C), K, M, N, le, lm, size, block_size,
                 kernel.ctype(), _lib.ptr(work), int(force_general), _lib.stream(dev))
    return _lib.back(C, P_A)


def workspace_elements(K: int, M: int, N: int, count: int) -> int:
    """int32 elements of device workspace a systolic launch of `count` problems (K x M codes A, K x N codes B)
    needs."""
    return int(_lib.load().mxq_systolic_workspace(K, M, N, count))


def systolic_batched(ops, layout: "_lib.SystolicLayout", count: int, K: int, M: int, N: int, C: torch.Tensor,
                     arith: Arithmetic, schedule: Sequence[Tuple[int, int]], size: int = 16,
                     block_size: int = BLOCK, *, skip: Optional[torch.Tensor] = None,
                     k_end: Optional[torch.Tensor] = None, a_live: Optional[torch.Tensor] = None,
                     c_end: Optional[torch.Tensor] = None,
                     epilogue: Optional["_lib.SystolicEpilogue"] = None) -> None:
    """`count` problems of one shape in one launch, written into C (mxq_systolic_batched).  ops: the four
    device tensors the layout's strides address (codes A, scales X_A, codes B, scales X_B), float32 on C's
    device.  Each problem's result equals systolic() on that problem alone.  The Arithmetic must carry a
    kernel description (MXGEMMINI, MXQUANT, compiled).
    Hints (include/mxq_hip.h mxq_systolic_hints): `skip`, uint8 count x ceil(M/32) x ceil(N/32), nonzero where
    the caller does not need C's 32 x 32 group (such tiles come back +0); `k_end`, int32 count x ceil(M/64), a
    bound on the rows of A holding nonzero codes in each 64-column group (checked: a wrong one costs time);
    `a_live`, with k_end, uint8 count x ceil(K/32) x ceil(M/32), the caller's answer to that check for A (nonzero
    unless the 32 x 32 piece of A is +-0 with finite scales; trusted, so it must be exact); `c_end`, with skip,
    int32 count x ceil(M/64): skipped tiles whose columns start at or past it are not stored at all.
    `epilogue` (mxq_systolic_epilogue): R(R(C * scale) + mask value) applied to every output as it is stored."""
    import ctypes
    kernel = getattr(arith, "kernel", None)
    if kernel is None or size > 64 or 32 % size != 0 or block_size % size != 0:
        raise ValueError("systolic_batched needs a kernel Arithmetic and size dividing 32 and block_size")
    check_schedule(schedule, size)
    if count == 0 or M == 0 or N == 0:
        return
    if K > 0:
        _lanes_check(kernel, schedule, min(size, K))
    dev = C.device
    if any(t.device != dev or t.dtype != torch.float32 for t in ops) or C.dtype != torch.float32:
        raise ValueError("codes, scales and C must be float32 on one device")
    le = (ctypes.c_int32 * size)(*[int(e) for e, _ in schedule])
    lm = (ctypes.c_int32 * size)(*[int(m) for _, m in schedule])
    for t, dt, shape in ((skip, torch.uint8, (count, -(-M // 32), -(-N // 32))),
                         (k_end, torch.int32, (count, -(-M // 64))),
                         (a_live, torch.uint8, (count, -(-K // 32), -(-M // 32))),
                         (c_end, torch.int32, (count, -(-M // 64)))):
        if t is not None and (t.dtype != dt or tuple(t.shape) != shape or t.device != dev or not t.is_contiguous()):
            raise ValueError(f"systolic_batched: a hint must be a contiguous {dt} tensor of shape {shape} on {dev}")
    hints = _lib.SystolicHints(skip=_lib.ptr(skip), k_end=_lib.ptr(k_end), a_live=_lib.ptr(a_live),
                               c_end=_lib.ptr(c_end))
    work = torch.empty(workspace_elements(K, M, N, count), dtype=torch.int32, device=dev)
    with _lib.on(dev):
        _lib.run("mxq_systolic_batched", *(_lib.ptr(t) for t in ops), _lib.ptr(C), ctypes.byref(layout), count,
                 K, M, N, le, lm, size, block_size, kernel.ctype(), ctypes.byref(hints),
                 None if epilogue is None else ctypes.byref(epilogue), _lib.ptr(work), 0, _lib.stream(dev))


def fast_lanes(arith: Arithmetic, schedule: Sequence[Tuple[int, int]], size: int = 16) -> bool:
    """Whether the library runs its fast kernel for this Arithmetic and lane schedule (mxq_systolic_fast_lanes):
    then a launch under k_end never reads rows of A past it that its check passes."""
    import ctypes
    kernel = getattr(arith, "kernel", None)
    if kernel is None or len(schedule) != size:
        return False
    le = (ctypes.c_int32 * size)(*[int(e) for e, _ in schedule])
    lm = (ctypes.c_int32 * size)(*[int(m) for _, m in schedule])
    return bool(_lib.load().mxq_systolic_fast_lanes(le, lm, size, kernel.ctype()))


def _reference_loop(P_A, X_A, P_B, X_B, arith, schedule, size, block_size, K, M, N):
    """The reference's reducer loop with the Arithmetic's callables (their fused forms when offered)."""
    C = torch.zeros((M, N), dtype=torch.float32, device=P_A.device)
    whole = arith.fused_block(schedule, size, block_size) if getattr(arith, "fused_block", None) else None
    body = arith.fused_reduction(schedule, size) if getattr(arith, "fused_reduction", None) else None
    for g in range(0, K, block_size):
        g_end = min(g + block_size, K)
        scales = scale_map(X_A, X_B, g // block_size)
        if whole is not None and g_end - g == block_size:
            C = whole(P_A[g:g_end], P_B[g:g_end], scales, C)
            continue
        for k_base in range(g, g_end, size):
            k_end = min(k_base + size, g_end)
            if body is not None and k_end - k_base == size:
                S = body(P_A[k_base:k_end], P_B[k_base:k_end])
            else:
                S = torch.zeros((M, N), dtype=torch.float32, device=P_A.device)
                for k in range(k_base, k_end):
                    p = arith.product(P_A[k].unsqueeze(1), P_B[k].unsqueeze(0))
                    e, m = schedule[k % size]
                    S = arith.acc_add(S, p, e, m)
            C = arith.tile_add(C, S * scales)
    return C.to(torch.float32)
