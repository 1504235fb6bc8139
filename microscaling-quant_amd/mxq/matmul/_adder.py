"""The adder tree (mxq/matmul/_adder.py:1-71): systolic's call, with each reduction of `size` products formed
at once (zeros past a K tail) and folded by log2(size) levels of adjacent-pair adds, level l rounding to
schedule[l] with the Arithmetic's acc_add; the root is rescaled by the block's scale map and tile-added into
the output.  The pairing is fixed, (0, 1), (2, 3), ..., since a floating-point tree's result depends on it.

With MXGEMMINI or MXQUANT (or compiled(...) of them) and size <= 32 the whole call is one HIP launch
(include/mxq_hip.h mxq_adder_tree): every output's reductions run in one thread, products entering a
binary-counter stack of one pending sum per level.  For MXGEMMINI with e4 levels of non-decreasing m followed by
bf16 levels (the README's [(4, 4), (4, 5), (4, 6), (8, 7)], or all bf16) a fast kernel runs first and the general
one computes only the tiles whose codes it could not take.  A hand-made Arithmetic, or a larger size, runs the
reference's loop with the Arithmetic's own callables on the operands' device.
"""
from typing import Sequence, Tuple

import torch

from .. import _lib
from ..block import BLOCK
from ._arithmetic import Arithmetic
from ._common import check_operands, check_schedule, scale_map
from ._systolic import _lanes_check, workspace_elements

__all__ = ["adder_tree"]


def adder_tree(P_A: torch.Tensor, X_A: torch.Tensor, P_B: torch.Tensor, X_B: torch.Tensor,
               arith: Arithmetic, schedule: Sequence[Tuple[int, int]], size: int = 16,
               block_size: int = BLOCK, *, force_general: bool = False) -> torch.Tensor:
    """Y = A^T B.  A: K x M codes, X_A: ceil(K/block_size) x M scales; B: K x N, X_B: ceil(K/block_size) x N.
    One schedule entry per tree level, level 1 first; `size` a power of two dividing `block_size`.
    `force_general` (not in the reference) runs the general kernel even where the fast one applies; the two are
    bit-identical."""
    K, M, N = check_operands(P_A, X_A, P_B, X_B, block_size)
    levels = size.bit_length() - 1
    if size < 2 or (1 << levels) != size:
        raise ValueError(f"size {size} must be a power of two >= 2")
    if block_size % size != 0:
        raise ValueError(f"size {size} must divide block size {block_size}")
    check_schedule(schedule, levels)
    kernel = getattr(arith, "kernel", None)
    if kernel is None or size > 32:
        return _stage_loop(P_A, X_A, P_B, X_B, arith, schedule, size, block_size, K, M, N)
    if K > 0:
        _lanes_check(kernel, schedule, levels)
    dev = _lib.compute_device(P_A)
    ops = [_lib.to_device(t.detach(), dev).contiguous() for t in (P_A, X_A, P_B, X_B)]
    C = torch.empty((M, N), dtype=torch.float32, device=dev)
    if M == 0 or N == 0:
        return _lib.back(C, P_A)
    import ctypes
    le = (ctypes.c_int32 * levels)(*[int(e) for e, _ in schedule])
    lm = (ctypes.c_int32 * levels)(*[int(m) for _, m in schedule])
    work = torch.empty(workspace_elements(K, M, N, 1), dtype=torch.int32, device=dev)
    with _lib.on(dev):
        _lib.run("mxq_adder_tree", *(_lib.ptr(t) for t in ops), _lib.ptr(C), K, M, N, le, lm, size, block_size,
                 kernel.ctype(), _lib.ptr(work), int(force_general), _lib.stream(dev))
    return _lib.back(C, P_A)


def _stage_loop(P_A, X_A, P_B, X_B, arith, schedule, size, block_size, K, M, N):
    """The reference's adder-tree loop with the Arithmetic's callables."""
    C = torch.zeros((M, N), dtype=torch.float32, device=P_A.device)
    zero = torch.zeros((M, N), dtype=torch.float32, device=P_A.device)
    for g in range(0, K, block_size):
        g_end = min(g + block_size, K)
        scales = scale_map(X_A, X_B, g // block_size)
        for k0 in range(g, g_end, size):
            k1 = min(k0 + size, g_end)
            level = [arith.product(P_A[k].unsqueeze(1), P_B[k].unsqueeze(0)) for k in range(k0, k1)]
            level += [zero] * (size - len(level))
            for e, m in schedule:
                level = [arith.acc_add(level[2 * i], level[2 * i + 1], e, m) for i in range(len(level) // 2)]
            C = arith.tile_add(C, level[0] * scales)
    return C.to(torch.float32)
