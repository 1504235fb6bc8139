"""Attention whose two matmuls run through Schemes (mxq/nn/_attention.py:1-167).

    out = attend(q, k, v, mask, scale, qk, pv, chunk=None, vector=None)
          q: B x H x Tq x D, k and v: B x Hkv x Tk x D (H a multiple of Hkv), out: B x Tq x H x D

The work is cut into calls.  For each batch row b and KV head h, K^T (D x Tk, blocks along D) is quantized by
qk.b and V (Tk x D, blocks along the keys) by pv.b, once.  The queries are taken `step` at a time; inside a
chunk the H/Hkv query heads that share h go into one call as n*m head-major columns, as far as a multiple of
the schemes' rows reaches, and the rest of the chunk goes head by head.  Each call:

    A = qk.a(Q^T)                    Q^T: D x n*m
    S = fl(reduce(A, K^T) * scale)   n*m x Tk, then fl(S + mask) when there is a mask   (each rounded by `vector`)
    P = softmax(S)                   torch.softmax on the device, or its rounded steps
    O = pv.reduce(pv.a(P^T), V)      contraction over the keys

Columns are grouped exactly so because a LUT activation shares tables among `rows` adjacent columns.

Masked keys.  A key whose mask value absorbs every score the call can produce (fl(mask + s) == mask for all
|s| <= bound, where bound = SLACK * |scale| * sum over d of max|Q_d| * max|K_d| over the dequantized codes, in
float64, tested in float32 on both sides of each mask value) has score fl(mask), so only the keys between the
first and last key some query of the call still sees, widened to pv.block_size boundaries, are multiplied.
P V then runs over the same key blocks, provided P is exactly zero on every key outside them; otherwise over
all keys.  Outside keys contribute whole all-zero blocks, which add nothing to any reducer's tile sum.
"""
import ctypes
from dataclasses import dataclass
from functools import partial
from typing import Iterator, Optional, Tuple

import numpy as np
import torch

from ..scheme import Scheme
from ._vector import rounder, softmax

__all__ = ["attend", "register", "NAME"]

#: the transformers attention-implementation name patch() installs
NAME = "mxq"

#: score entries (n*m x Tk float32) per call when no chunk is given
ELEMENTS_PER_STEP = 1 << 26

#: factor by which a reducer's rounded score may exceed the exact sum of the magnitudes of its products:
#: (1 + 2^-(m+1)) per rounding over at most 32 lane roundings and 256 block adds stays under it
SLACK = 2.0 ** 16


@dataclass(frozen=True)
class _Dims:
    B: int
    H: int
    Hkv: int
    Tq: int
    Tk: int
    D: int

    @property
    def group(self) -> int:
        return self.H // self.Hkv


def _dims(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> _Dims:
    B, H, Tq, D = q.shape
    Hkv, Tk = k.shape[1], k.shape[2]
    if H % Hkv or v.shape[1] != Hkv or v.shape[2] != Tk:
        raise ValueError(f"attend: q has {H} heads, k {tuple(k.shape)}, v {tuple(v.shape)}")
    return _Dims(B, H, Hkv, Tq, Tk, D)


def _calls(heads: range, Tq: int, step: int, rows: int) -> Iterator[Tuple[range, int, int]]:
    """(query heads, first query, end query) of each call for one KV head, in order."""
    for start in range(0, Tq, step):
        end = min(start + step, Tq)
        joint = end - (end - start) % rows
        if joint > start:
            yield heads, start, joint
        if joint < end:
            for hq in heads:
                yield range(hq, hq + 1), joint, end


def _code_amax(codes: torch.Tensor, scales: torch.Tensor, block_size: int) -> torch.Tensor:
    """max over columns of |code| * its block scale, per contraction row (float32 products): K float64."""
    per_row = scales.repeat_interleave(block_size, dim=0)[:codes.shape[0]]
    return (codes.abs() * per_row).amax(dim=1).to(torch.float64)


def _live_span(mask_rows: torch.Tensor, bound: float, block: int) -> Tuple[int, int]:
    """[lo, hi) of the keys whose mask value does not absorb `bound` for some query row, widened to whole
    blocks of `block` keys; the first block when every key is absorbed."""
    Tk = mask_rows.shape[1]
    absorbed = ((mask_rows + bound) == mask_rows) & ((mask_rows - bound) == mask_rows)
    live = (~absorbed.all(dim=0)).nonzero()
    if not live.numel():
        return 0, min(Tk, block)
    first, last = int(live[0]), int(live[-1])
    return first - first % block, min(Tk, -(-(last + 1) // block) * block)


def _bias(mask: Optional[torch.Tensor], dims: _Dims) -> Optional[torch.Tensor]:
    """The mask as Bm x Tq x Tk float32: mask[:, 0, :, :Tk], its query and key dimensions broadcast where they
    are 1 (batch row b reads mask row b, or row 0 when Bm == 1).  Extents that cannot serve B x 1 x Tq x Tk are
    refused here, before a kernel reads Tk values from each mask row."""
    if mask is None:
        return None
    if mask.dim() != 4:
        raise ValueError(f"attend: mask must be B x 1 x Tq x Tk, got {tuple(mask.shape)}")
    bias = mask[:, 0, :, :dims.Tk].to(torch.float32)
    Bm, Tq_m, Tk_m = bias.shape
    if (Bm != 1 and Bm < dims.B) or Tq_m not in (1, dims.Tq) or Tk_m not in (1, dims.Tk):
        raise ValueError(f"attend: mask {tuple(mask.shape)} does not broadcast to "
                         f"{dims.B} x 1 x {dims.Tq} x {dims.Tk}")
    return bias.expand(Bm, dims.Tq, dims.Tk)


@torch.no_grad()
def attend(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, mask: Optional[torch.Tensor], scale: float,
           qk: Scheme, pv: Scheme, chunk: Optional[int] = None, vector: Optional[str] = None) -> torch.Tensor:
    """S = Q K^T through `qk`, O = P V through `pv`; scale, additive mask and softmax in float32, or each step
    rounded to bf16 with vector="bf16".  mask: None or additive, broadcastable to B x 1 x Tq x Tk (HF eager).
    chunk: queries per step, a positive multiple of max(qk.rows, pv.rows); None: the most that keep
    n*chunk*Tk under ELEMENTS_PER_STEP."""
    dims = _dims(q, k, v)
    rows = max(qk.rows, pv.rows)
    if chunk is not None and (chunk < 1 or chunk % rows):
        raise ValueError(f"attend: chunk {chunk} must be a positive multiple of the schemes' rows = {rows}")
    step = chunk or max(rows, ELEMENTS_PER_STEP // (dims.group * dims.Tk) // rows * rows)
    rnd = rounder(vector)
    out = q.new_empty(dims.B, dims.Tq, dims.H, dims.D)
    bias = _bias(mask, dims)                                                      # Bm x Tq x Tk, Bm = 1 or B
    batch = _Batched.of(qk, pv, q)
    if batch is not None:
        batch.run(q, k, v, bias, scale, step, vector, rnd, dims, out)
        return out
    for b in range(dims.B):
        bias_b = None if bias is None else bias[b if bias.shape[0] > 1 else 0]
        for h in range(dims.Hkv):
            ops = _KVOperands.quantize(k[b, h], v[b, h], qk, pv, bias_b is not None)
            for hs, s0, e0 in _calls(range(h * dims.group, (h + 1) * dims.group), dims.Tq, step, rows):
                _one_call(q[b], ops, bias_b, scale, qk, pv, vector, rnd, dims, hs, s0, e0, out[b])
    return out


@dataclass
class _KVOperands:
    """One KV head's quantized K^T (D x Tk) and V (Tk x D), and K's per-row code maxima for the skip bound."""
    KT_P: torch.Tensor
    KT_X: torch.Tensor
    V_P: torch.Tensor
    V_X: torch.Tensor
    k_amax: Optional[torch.Tensor]

    @staticmethod
    def quantize(k_h, v_h, qk: Scheme, pv: Scheme, masked: bool) -> "_KVOperands":
        KT_P, KT_X = qk.b(k_h.to(torch.float32).t().contiguous())
        V_P, V_X = pv.b(v_h.to(torch.float32).contiguous())
        return _KVOperands.checked(KT_P, KT_X, V_P, V_X, qk, pv, masked)

    @staticmethod
    def checked(KT_P, KT_X, V_P, V_X, qk: Scheme, pv: Scheme, masked: bool) -> "_KVOperands":
        qk.check_scales(KT_X, KT_P.shape[0], "b (Kᵀ)")
        pv.check_scales(V_X, V_P.shape[0], "b (V)")
        return _KVOperands(KT_P, KT_X, V_P, V_X, _code_amax(KT_P, KT_X, qk.block_size) if masked else None)


def _one_call(q_b, ops: _KVOperands, bias, scale, qk: Scheme, pv: Scheme, vector, rnd, dims: _Dims, hs: range,
              s0: int, e0: int, out_b) -> None:
    """One call of the reference's loop: query heads hs, queries [s0, e0) against one KV head."""
    Tk, D = dims.Tk, dims.D
    bv = pv.block_size
    n, m = len(hs), e0 - s0
    Q_T = q_b[hs.start:hs.stop, s0:e0].to(torch.float32).reshape(n * m, D).t().contiguous()
    A_P, A_X = qk.a(Q_T)
    lo, hi = 0, Tk
    rows_bias = None
    if bias is not None:
        rows_bias = bias[s0:e0]                                                   # m x Tk
        bound = SLACK * abs(scale) * float((_code_amax(A_P, A_X, qk.block_size) * ops.k_amax).sum())
        lo, hi = _live_span(rows_bias, max(bound, torch.finfo(torch.float32).tiny), bv)
    S_live = rnd(qk.reduce(A_P, A_X, ops.KT_P[:, lo:hi], ops.KT_X[:, lo:hi]) * scale)   # n*m x (hi - lo)
    if rows_bias is not None:
        S_live = rnd(S_live.view(n, m, hi - lo) + rows_bias[:, lo:hi]).view(n * m, hi - lo)
    if hi - lo == Tk:
        S = S_live
    else:
        S = rnd(rows_bias).repeat(n, 1)                                           # absorbed keys: the mask
        S.view(n, m, Tk)[:, :, lo:hi] = S_live.view(n, m, hi - lo)
    P = softmax(S, vector)
    if hi - lo != Tk and (P[:, :lo].any() or P[:, hi:].any()):
        lo, hi = 0, Tk                                                            # some row has no live key
    PT_P, PT_X = pv.a(P.t().contiguous())                                         # Tk x n*m, blocks along keys
    blocks = slice(lo // bv, -(-hi // bv))
    O = pv.reduce(PT_P[lo:hi], PT_X[blocks], ops.V_P[lo:hi], ops.V_X[blocks])     # n*m x D
    out_b[s0:e0, hs.start:hs.stop] = O.view(n, m, D).transpose(0, 1).to(out_b.dtype)


# ------------------------------------------------------------------------------------------ batched path
#: score entries per batched launch (problems x n*m x Tk float32): 4 GiB
ELEMENTS_PER_LAUNCH = 1 << 30

#: bytes of prepared query codes and scales (Q^T of the chunks waiting for their launches) held at once
PREPARED_BYTES = 1 << 28


def _columnwise(quantizer, block_size: int) -> bool:
    """A library block quantizer with blocks along axis 0: every column is quantized on its own, so the columns
    of many calls quantized side by side get exactly the codes and scales each call would get."""
    from ..block import mxgemmini, mxquant, ocp
    if not isinstance(quantizer, partial) or quantizer.args:
        return False
    if quantizer.func not in (mxgemmini.quantize, mxquant.quantize, ocp.quantize):
        return False
    kw = quantizer.keywords
    return "fmt" in kw and kw.get("axis", 0) in (0, -2) and kw.get("block_size", block_size) == block_size


def _systolic_reducer(reduce, block_size: int):
    """(arith, schedule, size) when `reduce` is matmul.systolic bound to an Arithmetic the kernel runs."""
    from ..matmul import _systolic
    if not isinstance(reduce, partial) or reduce.args or reduce.func is not _systolic.systolic:
        return None
    kw = reduce.keywords
    if set(kw) - {"arith", "schedule", "size", "block_size"} or "arith" not in kw or "schedule" not in kw:
        return None
    size = kw.get("size", 16)
    if getattr(kw["arith"], "kernel", None) is None or kw.get("block_size", 32) != block_size:
        return None
    if size > 64 or 32 % size or block_size % size or len(kw["schedule"]) != size:
        return None
    return kw["arith"], kw["schedule"], size


def _group_amax(codes: torch.Tensor, scales: torch.Tensor, block_size: int, groups: int) -> torch.Tensor:
    """_code_amax of each of `groups` equal column groups side by side, one kernel: K x groups, float64."""
    from .. import _lib
    K, cols = codes.shape
    out = torch.empty(K, groups, dtype=torch.float64, device=codes.device)
    with _lib.on(codes.device):
        _lib.run("mxq_group_amax", _lib.ptr(codes.contiguous()), _lib.ptr(scales.contiguous()), K, cols, groups,
                 block_size, _lib.ptr(out), _lib.stream(codes.device))
    return out


def _mask_rows(bias: torch.Tensor, z0: int, Hkv: int, s0: int):
    """(pointer tensor, batch-row stride, row stride) of mask row s0 of pair z0, keys contiguous."""
    if bias.stride(2) != 1:
        bias = bias.contiguous()
    batched = bias.shape[0] > 1
    return bias[z0 // Hkv if batched else 0, s0], bias.stride(0) if batched else 0, bias.stride(1)


def _windows(a_amax: torch.Tensor, k_amax: torch.Tensor, z0: int, Zc: int, scale: float, bias: torch.Tensor,
             Hkv: int, s0: int, m: int, block: int) -> torch.Tensor:
    """Per pair z0..z0+Zc, words whose OR is 3 when its call keeps every key: the reference's bound (SLACK *
    |scale| * sum over D of the two amax factors, at least FLT_MIN) and its live-key span == (0, Tk)
    (mxq/nn/_attention.py:117-127), as Zc x ceil(m/64) int32 words on the device (one per 64 query rows, each
    written whole; no host synchronisation)."""
    from .. import _lib
    D, Tk = a_amax.shape[0], bias.shape[2]
    flags = torch.empty(Zc, -(-m // 64), dtype=torch.int32, device=a_amax.device)
    mask, b_stride, r_stride = _mask_rows(bias, z0, Hkv, s0)
    with _lib.on(a_amax.device):
        _lib.run("mxq_attend_windows", _lib.ptr(a_amax), a_amax.shape[1], _lib.ptr(k_amax[:, z0:]), k_amax.shape[1],
                 D, Zc, SLACK * abs(scale), _lib.ptr(mask), b_stride, r_stride, z0, Hkv, m, Tk, block,
                 _lib.ptr(flags), _lib.stream(a_amax.device))
    return flags


def _hints(a_amax: torch.Tensor, k_amax: torch.Tensor, z0: int, Zc: int, scale: float, bias: torch.Tensor,
           Hkv: int, s0: int, m: int, rows: int, Tk: int, with_tail: bool = False):
    """The two batched launches' hints from the mask rows s0.. of pairs z0..z0+Zc and each call's bound
    (include/mxq_hip.h mxq_attend_hints): the 32 x 32 score groups whose mask absorbs every score the call can
    produce, where a +0 score gives the reference's r(r(s * scale) + mask) (skip, for Q K^T), and per 64 rows
    the end of the keys some row still sees (k_end, for P V; checked by the kernel, so a row whose every key
    is masked, where softmax is uniform, costs time, not bits).  with_tail: also the largest mask value past
    k_end per 64 rows (tail_max, for the softmax's tail), else None."""
    from .. import _lib
    D = a_amax.shape[0]
    mask, b_stride, r_stride = _mask_rows(bias, z0, Hkv, s0)
    batched = bias.shape[0] > 1
    batches = (z0 + Zc - 1) // Hkv - z0 // Hkv + 1 if batched else 1
    rg, kg, tg = -(-rows // 32), -(-Tk // 32), -(-rows // 64)
    dev = a_amax.device
    minabs = torch.empty(batches, rg, kg, dtype=torch.float32, device=dev)
    maxval = torch.empty(batches, rg, kg, dtype=torch.float32, device=dev) if with_tail else None
    skip = torch.empty(Zc, rg, kg, dtype=torch.uint8, device=dev)
    k_end = torch.empty(Zc, tg, dtype=torch.int32, device=dev)
    tail_max = torch.empty(Zc, tg, dtype=torch.float32, device=dev) if with_tail else None
    with _lib.on(dev):
        _lib.run("mxq_mask_minabs", _lib.ptr(mask), b_stride, r_stride, batches, rows, m, Tk, _lib.ptr(minabs),
                 _lib.ptr(maxval), _lib.stream(dev))
        _lib.run("mxq_attend_hints", _lib.ptr(a_amax), a_amax.shape[1], _lib.ptr(k_amax[:, z0:]), k_amax.shape[1],
                 D, Zc, SLACK * abs(scale), _lib.ptr(minabs), z0, Hkv, int(batched), rows, Tk, _lib.ptr(skip),
                 _lib.ptr(k_end), _lib.ptr(maxval), _lib.ptr(tail_max), _lib.stream(dev))
    return skip, k_end, tail_max


@dataclass
class _Prepared:
    """One chunk of the batched path between its preparation and its launches."""
    z0: int
    z1: int
    s0: int
    e0: int
    A_P: torch.Tensor
    A_X: torch.Tensor
    flags: Optional[torch.Tensor]
    skip: Optional[torch.Tensor]
    k_end: Optional[torch.Tensor]
    tail_max: Optional[torch.Tensor]


@dataclass
class _Batched:
    """attend built from the library's own pieces (column-wise block quantizers, matmul.systolic with a kernel
    Arithmetic, no LUT rows) runs a query chunk of every (batch row, KV head) pair as one quantize call per
    operand and one launch per matmul.  Each pair's codes, scales, scores and outputs are those its own call
    gives: the quantizers treat columns independently, a batched launch computes each problem as a single one,
    and softmax works row by row.  A chunk in which some pair would skip masked keys goes through the
    reference's per-pair loop instead, on the same codes."""
    qk: Scheme
    pv: Scheme
    qk_red: tuple
    pv_red: tuple
    pv_fast: bool    # the P V launch runs the fast kernel, which never reads P^T past k_end where it is +0

    @staticmethod
    def of(qk: Scheme, pv: Scheme, q: torch.Tensor) -> Optional["_Batched"]:
        if q.device.type != "cuda" or qk.rows != 1 or pv.rows != 1:
            return None
        if not all(_columnwise(f, s.block_size) for s, f in ((qk, qk.a), (qk, qk.b), (pv, pv.a), (pv, pv.b))):
            return None
        qk_red, pv_red = _systolic_reducer(qk.reduce, qk.block_size), _systolic_reducer(pv.reduce, pv.block_size)
        if qk_red is None or pv_red is None:
            return None
        from ..matmul._systolic import fast_lanes
        arith, sched, size = pv_red
        return _Batched(qk, pv, qk_red, pv_red, fast_lanes(arith, sched, size))

    def run(self, q, k, v, bias, scale, step, vector, rnd, dims: _Dims, out) -> None:
        qk, pv = self.qk, self.pv
        B, Hkv, Tk, D, n = dims.B, dims.Hkv, dims.Tk, dims.D, dims.group
        Z = B * Hkv
        # pair z = b * Hkv + h: its K^T in columns [z*Tk, (z+1)*Tk) (a transposed view of k: no copy), its V the
        # z-th Tk x D slab (blocks along the keys, every column on its own, so the same codes as V alone)
        KT_P, KT_X = qk.b(k.to(torch.float32).permute(3, 0, 1, 2).reshape(D, Z * Tk))
        V_P, V_X = pv.b.func(v.to(torch.float32).reshape(Z, Tk, D), **{**pv.b.keywords, "axis": 1})
        qk.check_scales(KT_X, D, "b (Kᵀ)")
        pv.check_scales(V_X.transpose(0, 1), Tk, "b (V)")                         # Z x nb x D
        kv = (KT_P, KT_X, V_P, V_X)
        k_amax = _group_amax(KT_P, KT_X, qk.block_size, Z) if bias is not None else None
        qg = q.reshape(Z, n, dims.Tq, D)
        # chunks are prepared (Q^T's codes, flags, hints) in batches that stop once they hold PREPARED_BYTES of
        # codes and scales, so the prepared operands stay bounded (by that plus one chunk) however long the input
        batch, held = [], 0
        for s0 in range(0, dims.Tq, step):
            e0 = min(s0 + step, dims.Tq)
            for z0, z1 in _launch_ranges(B, Hkv, max(1, ELEMENTS_PER_LAUNCH // (n * (e0 - s0) * Tk))):
                c = self._prepare(qg, bias, kv, k_amax, scale, vector, dims, z0, z1, s0, e0)
                batch.append(c)
                held += (c.A_P.numel() + c.A_X.numel()) * 4
                if held >= PREPARED_BYTES:
                    self._launch(batch, q, qg, bias, kv, scale, vector, rnd, dims, out)
                    batch, held = [], 0
        if batch:
            self._launch(batch, q, qg, bias, kv, scale, vector, rnd, dims, out)

    def _launch(self, chunks, q, qg, bias, kv, scale, vector, rnd, dims: _Dims, out) -> None:
        """Prepared chunks' launches.  Their flags come over in one transfer into pinned memory, queued ahead of
        the matmuls with an event behind it, so the host queues the matmuls while the GPU works, then waits for
        the copy alone and returns without waiting for the matmuls."""
        if bias is not None:
            flags = chunks[0].flags.view(-1) if len(chunks) == 1 else torch.cat([c.flags.view(-1) for c in chunks])
            host = torch.empty(flags.shape, dtype=flags.dtype, pin_memory=True)
            host.copy_(flags, non_blocking=True)
            copied = torch.cuda.Event()
            copied.record(torch.cuda.current_stream(flags.device))
        for c in chunks:
            self._chunk(c, qg, bias, kv, scale, vector, dims, out)
        if bias is None:
            return
        copied.synchronize()
        words = host.numpy()
        # a pair that would skip masked keys gets the reference's own call, on the same codes, over its outputs
        at = 0
        for c in chunks:
            zc, w = c.flags.shape
            every = np.bitwise_or.reduce(words[at:at + zc * w].reshape(zc, w), axis=1)
            for z in range(zc):
                if every[z] != 3:
                    self._per_pair(q, bias, kv, scale, vector, rnd, dims, c.z0 + z, c.z0 + z + 1, c.s0, c.e0, out)
            at += zc * w

    def _prepare(self, qg, bias, kv, k_amax, scale, vector, dims: _Dims, z0, z1, s0, e0) -> "_Prepared":
        """Pairs z0..z1, queries s0..e0: Q^T's codes and, with a mask, each pair's flag (int32 on the device: 3
        when its call keeps every key, so the batched result is the reference's; otherwise the caller redoes it
        through the reference's call) and the two launches' hints."""
        qk, pv = self.qk, self.pv
        Zc, n, m, Tk, D, Hkv = z1 - z0, dims.group, e0 - s0, dims.Tk, dims.D, dims.Hkv
        cols = n * m                                                              # one call's columns
        A_P, A_X = qk.a(qg[z0:z1, :, s0:e0].to(torch.float32).permute(3, 0, 1, 2).reshape(D, Zc * cols))
        flags = skip = k_end = tail_max = None
        if bias is not None:
            a_amax = _group_amax(A_P, A_X, qk.block_size, Zc)
            flags = _windows(a_amax, k_amax, z0, Zc, scale, bias, Hkv, s0, m, pv.block_size)
            skip, k_end, tail_max = _hints(a_amax, k_amax, z0, Zc, scale, bias, Hkv, s0, m, cols, Tk,
                                           self._tail_ok(cols, Tk, vector))
        return _Prepared(z0, z1, s0, e0, A_P, A_X, flags, skip, k_end, tail_max)

    def _tail_ok(self, cols: int, Tk: int, vector) -> bool:
        """Whether the scores past each 64-row group's k_end may go unstored and P^T unwritten there: the
        softmax kernel takes them from the mask, and the P V launch's fast kernel reads P^T only below k_end
        where the softmax's stage bytes say the rest is +0 (64-row groups inside one call: cols % 64 == 0)."""
        return (self.pv_fast and cols % 64 == 0 and
                _softmax_pt_spec(self.pv.a, self.pv.block_size, vector, Tk) is not None)

    def _chunk(self, c: "_Prepared", qg, bias, kv, scale, vector, dims: _Dims, out) -> None:
        """A prepared chunk as two batched launches, its outputs into `out`."""
        from .. import _lib
        from ..matmul._systolic import systolic_batched
        qk, pv = self.qk, self.pv
        KT_P, KT_X, V_P, V_X = kv
        z0, z1, s0, e0, A_P, A_X, skip, k_end = c.z0, c.z1, c.s0, c.e0, c.A_P, c.A_X, c.skip, c.k_end
        Zc, n, m, Tk, D, Hkv = z1 - z0, dims.group, e0 - s0, dims.Tk, dims.D, dims.Hkv
        cols = n * m                                                              # one call's columns
        arith, sched, size = self.qk_red
        S = torch.empty(Zc, cols, Tk, dtype=torch.float32, device=qg.device)
        # the score step r(r(S * scale) + mask row) is applied as the scores are stored (_scale_mask's step)
        mask, b_stride, r_stride = (None, 0, 0) if bias is None else _mask_rows(bias, z0, Hkv, s0)
        epi = _lib.SystolicEpilogue(scale=float(scale), bf16=int(vector == "bf16"), mask=_lib.ptr(mask),
                                    mask_b_stride=b_stride, mask_row_stride=r_stride, z0=z0, z_per_b=Hkv, m=m)
        # with a tail, the scores past each 64-row group's k_end are never stored: the softmax reads what it
        # needs of them from the mask through the same score step
        tail = None
        if c.tail_max is not None:
            tail = _lib.SoftmaxTail(k_end=_lib.ptr(k_end), tail_max=_lib.ptr(c.tail_max), score=epi)
        systolic_batched((A_P, A_X, KT_P[:, z0 * Tk:], KT_X[:, z0 * Tk:]),
                         _lib.SystolicLayout(ld_a=Zc * cols, batch_a=cols, ld_xa=Zc * cols, batch_xa=cols,
                                             ld_b=KT_P.shape[1], batch_b=Tk, ld_xb=KT_X.shape[1], batch_xb=Tk,
                                             ld_c=Tk, batch_c=cols * Tk),
                         Zc, D, cols, Tk, S, arith, sched, size, qk.block_size, skip=skip,
                         c_end=None if tail is None else k_end, epilogue=epi)
        # every call's P^T side by side: softmax and the quantizer in one kernel where they are torch's persistent
        # softmax and an MX-Gemmini quantizer; else P, quantized as it lies (a transposed view: no copy)
        PT = _softmax_pt(S, pv.a, pv.block_size, vector, cols if k_end is not None and cols % 32 == 0 else None,
                         tail)
        assert tail is None or PT is not None, "a tail needs the softmax kernel"
        a_live = None
        if PT is None:
            P = softmax(S, vector)
            PT_P, PT_X = pv.a(P.contiguous().view(Zc * cols, Tk).t())
        else:
            PT_P, PT_X, a_live = PT
        arith, sched, size = self.pv_red
        # one query head per KV head, float32 out, the chunk's pairs in one batch row: the products go straight
        # into out (query j of pair z at out[b, s0 + j, z - b * Hkv]), no copy; else into O, copied below
        b0 = z0 // Hkv
        direct = n == 1 and out.dtype == torch.float32 and out.is_contiguous() and (z1 - 1) // Hkv == b0
        if direct:
            O = out[b0, s0:e0, z0 - b0 * Hkv:z1 - b0 * Hkv]
            ld_c, batch_c = out.stride(1), out.stride(2)
        else:
            O = torch.empty(Zc, cols, D, dtype=torch.float32, device=qg.device)
            ld_c, batch_c = D, cols * D
        systolic_batched((PT_P, PT_X, V_P[z0:], V_X[z0:]),
                         _lib.SystolicLayout(ld_a=Zc * cols, batch_a=cols, ld_xa=Zc * cols, batch_xa=cols,
                                             ld_b=D, batch_b=Tk * D, ld_xb=D, batch_xb=V_X.shape[1] * D,
                                             ld_c=ld_c, batch_c=batch_c),
                         Zc, Tk, cols, D, O, arith, sched, size, pv.block_size, k_end=k_end, a_live=a_live)
        if direct:
            return
        O = O.view(Zc, n, m, D)
        for b in range(z0 // Hkv, (z1 - 1) // Hkv + 1):                          # pairs into B x Tq x H x D
            h0, h1 = max(z0, b * Hkv) - b * Hkv, min(z1, (b + 1) * Hkv) - b * Hkv
            part = O[b * Hkv + h0 - z0:b * Hkv + h1 - z0]                         # (h1 - h0) x n x m x D
            out[b, s0:e0, h0 * n:h1 * n] = part.permute(2, 0, 1, 3).reshape(m, (h1 - h0) * n, D).to(out.dtype)

    def _per_pair(self, q, bias, kv, scale, vector, rnd, dims: _Dims, z0, z1, s0, e0, out) -> None:
        KT_P, KT_X, V_P, V_X = kv
        Tk, D, n = dims.Tk, dims.D, dims.group
        for z in range(z0, z1):
            b, h = divmod(z, dims.Hkv)
            ops = _KVOperands.checked(KT_P[:, z * Tk:(z + 1) * Tk], KT_X[:, z * Tk:(z + 1) * Tk], V_P[z], V_X[z],
                                      self.qk, self.pv, bias is not None)
            bias_b = None if bias is None else bias[b if bias.shape[0] > 1 else 0]
            _one_call(q[b], ops, bias_b, scale, self.qk, self.pv, vector, rnd, dims, range(h * n, (h + 1) * n),
                      s0, e0, out[b])


def _softmax_pt_spec(quantizer, block_size: int, vector: Optional[str], T: int):
    """The kernel's block spec when mxq_softmax_quantize_t computes softmax over T keys and `quantizer`'s P^T
    (torch's persistent softmax, for 32 < T <= 2048 keys, and an MX-Gemmini quantizer of blocks of 32 along the
    keys), else None."""
    from ..block import mxgemmini
    from ..element_quant.formats import get
    from ..scale_factor import MXQUANT_FLOOR
    if vector is not None or not 32 < T <= 2048 or block_size != 32:
        return None
    if not isinstance(quantizer, partial) or quantizer.func is not mxgemmini.quantize or \
            quantizer.keywords.get("block_size", 32) != 32:
        return None
    kw = quantizer.keywords
    f = get(kw["fmt"])
    if f is None:
        return None
    return mxgemmini.spec(f, kw.get("rounding_mode", "ties_away"), kw.get("scale_floor", MXQUANT_FLOOR), kw.get("via"))


def _softmax_pt(S: torch.Tensor, quantizer, block_size: int, vector: Optional[str], live_cols: Optional[int] = None,
                tail: Optional["_lib.SoftmaxTail"] = None):
    """(P^T codes, scales, stage bytes) of softmax(S) over its last dim through `quantizer`
    (mxq/nn/_attention.py:136-139), as one kernel (mxq_softmax_quantize_t): for float32 rows of 32 < T <= 2048
    keys, where torch.softmax runs its persistent softmax, which the kernel reproduces bit for bit, and an
    MX-Gemmini quantizer of blocks of 32 along the keys.  With live_cols (P^T's columns per problem), the third
    item is the P V product's a_live hint for these codes, else None.  With a tail (include/mxq_hip.h
    mxq_softmax_tail), S holds each 64-row group's keys below its k_end only.  None where the kernel does not
    apply."""
    from .. import _lib
    T = S.shape[-1]
    spec = _softmax_pt_spec(quantizer, block_size, vector, T) if S.dtype == torch.float32 else None
    if spec is None:
        return None
    Sc = S.contiguous()
    R = Sc.numel() // T
    PT_P = torch.empty((T, R), dtype=torch.float32, device=S.device)
    PT_X = torch.empty((-(-T // 32), R), dtype=torch.float32, device=S.device)
    live = None
    if live_cols is not None:
        live = torch.empty((R // live_cols, -(-T // 32), live_cols // 32), dtype=torch.uint8, device=S.device)
    with _lib.on(S.device):
        _lib.run("mxq_softmax_quantize_t", _lib.ptr(Sc), R, T, _lib.ptr(PT_P), _lib.ptr(PT_X), spec, _lib.ptr(live),
                 live_cols or 0, None if tail is None else ctypes.byref(tail), _lib.stream(S.device))
    return PT_P, PT_X, live


def _launch_ranges(B: int, Hkv: int, per_launch: int):
    """Pair ranges [z0, z1) of at most per_launch pairs: whole batch rows when a launch holds one or more,
    else pieces of one batch row."""
    if per_launch >= Hkv:
        per_launch -= per_launch % Hkv
        return [(z0, min(B * Hkv, z0 + per_launch)) for z0 in range(0, B * Hkv, per_launch)]
    return [(b * Hkv + h0, b * Hkv + min(Hkv, h0 + per_launch)) for b in range(B) for h0 in range(0, Hkv, per_launch)]


def _scale_mask(S: torch.Tensor, bias: Optional[torch.Tensor], scale: float, vector: Optional[str], n: int, m: int,
                z0: int, Hkv: int, s0: int) -> None:
    """S (Zc x n*m x Tk scores of pairs z0.., queries s0..) <- r(r(S * scale) + mask rows) in place, one pass:
    the reference's `r(S * scale)` and `r(S + mask)` (mxq/nn/_attention.py:128-135), float32 multiply and add
    with the scale as float32, r the vector rounding.  Pair z's mask is bias[z // Hkv] (bias[0] when the mask has
    one batch row), rows s0.., keys contiguous.  The batched path applies the same step inside the systolic
    launch's stores (mxq_systolic_epilogue); this is its standalone form, against which that one is tested."""
    from .. import _lib
    Zc, _, Tk = S.shape
    mask, b_stride, r_stride = (None, 0, 0) if bias is None else _mask_rows(bias, z0, Hkv, s0)
    with _lib.on(S.device):
        _lib.run("mxq_scores_scale_mask", _lib.ptr(S), Zc, n, m, Tk, float(scale), _lib.ptr(mask), b_stride,
                 r_stride, z0, Hkv, int(vector == "bf16"),
                 _lib.stream(S.device))


def _mxq_attention(module, query, key, value, attention_mask, dropout: float = 0.0, scaling: Optional[float] = None,
                   **kwargs):
    """transformers' attention-function signature.  A module patch() gave no core runs sdpa unchanged."""
    core = getattr(module, "_mxq_core", None)
    if core is None:
        from transformers.integrations.sdpa_attention import sdpa_attention_forward
        return sdpa_attention_forward(module, query, key, value, attention_mask, dropout=dropout, scaling=scaling,
                                      **kwargs)
    if dropout:
        raise ValueError("mxq attention is inference only: dropout must be 0")
    scale = query.shape[-1] ** -0.5 if scaling is None else scaling
    out = attend(query, key, value, attention_mask, scale, *core, vector=getattr(module, "_mxq_vector", None))
    return out, None


def register() -> None:
    """Install NAME as a transformers attention implementation using eager's additive mask; repeatable."""
    from transformers import AttentionInterface
    from transformers.masking_utils import AttentionMaskInterface, eager_mask
    AttentionInterface.register(NAME, _mxq_attention)
    AttentionMaskInterface.register(NAME, eager_mask)
