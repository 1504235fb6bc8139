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
from dataclasses import dataclass
from typing import Iterator, Optional, Tuple

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
    for b in range(dims.B):
        bias = None
        if mask is not None:
            bias = mask[b if mask.shape[0] > 1 else 0, 0, :, :dims.Tk].to(torch.float32)
            bias = bias.expand(dims.Tq, dims.Tk) if bias.shape[0] == 1 else bias
        for h in range(dims.Hkv):
            _one_kv_head(q[b], k[b, h], v[b, h], bias, scale, qk, pv, step, rows, vector, rnd, dims,
                         range(h * dims.group, (h + 1) * dims.group), out[b])
    return out


def _one_kv_head(q_b, k_h, v_h, bias, scale, qk: Scheme, pv: Scheme, step, rows, vector, rnd, dims: _Dims,
                 heads: range, out_b):
    Tk, D = dims.Tk, dims.D
    KT_P, KT_X = qk.b(k_h.to(torch.float32).t().contiguous())                    # D x Tk
    V_P, V_X = pv.b(v_h.to(torch.float32).contiguous())                          # Tk x D
    qk.check_scales(KT_X, D, "b (Kᵀ)")
    pv.check_scales(V_X, Tk, "b (V)")
    k_amax = _code_amax(KT_P, KT_X, qk.block_size) if bias is not None else None
    bv = pv.block_size
    tiny = torch.finfo(torch.float32).tiny
    for hs, s0, e0 in _calls(heads, dims.Tq, step, rows):
        n, m = len(hs), e0 - s0
        Q_T = q_b[hs.start:hs.stop, s0:e0].to(torch.float32).reshape(n * m, D).t().contiguous()
        A_P, A_X = qk.a(Q_T)
        lo, hi = 0, Tk
        rows_bias = None
        if bias is not None:
            rows_bias = bias[s0:e0]                                               # m x Tk
            bound = SLACK * abs(scale) * float((_code_amax(A_P, A_X, qk.block_size) * k_amax).sum())
            lo, hi = _live_span(rows_bias, max(bound, tiny), bv)
        S_live = rnd(qk.reduce(A_P, A_X, KT_P[:, lo:hi], KT_X[:, lo:hi]) * scale)  # n*m x (hi - lo)
        if rows_bias is not None:
            S_live = rnd(S_live.view(n, m, hi - lo) + rows_bias[:, lo:hi]).view(n * m, hi - lo)
        if hi - lo == Tk:
            S = S_live
        else:
            S = rnd(rows_bias).repeat(n, 1)                                       # absorbed keys: the mask
            S.view(n, m, Tk)[:, :, lo:hi] = S_live.view(n, m, hi - lo)
        P = softmax(S, vector)
        if hi - lo != Tk and (P[:, :lo].any() or P[:, hi:].any()):
            lo, hi = 0, Tk                                                        # some row has no live key
        PT_P, PT_X = pv.a(P.t().contiguous())                                     # Tk x n*m, blocks along keys
        blocks = slice(lo // bv, -(-hi // bv))
        O = pv.reduce(PT_P[lo:hi], PT_X[blocks], V_P[lo:hi], V_X[blocks])         # n*m x D
        out_b[s0:e0, hs.start:hs.stop] = O.view(n, m, D).transpose(0, 1).to(out_b.dtype)


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
