"""Oracle attention core: mxq.nn.attend restated in numpy, with the softmax passed in.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

`attend` follows mxq/nn/_attention.py:70-143 (vector None or "bf16"): per batch row and KV head, K^T and V
quantized once; queries taken `step` at a time, the query heads of one KV head side by side (head-major columns)
up to a multiple of `rows` and the rest head by head; S = fl(reduce * scale), + mask, softmax, P^T quantized,
O = reduce over the key blocks some query still sees (mxq/nn/_attention.py:108-141, the SLACK bound of :60-62
and _amax of :65-67).

The quantizers, reducers and softmax are callables on numpy float32 arrays, so the same loop runs with the
oracle's block quantizers and systolic reducer, and with whichever softmax produced the probabilities under
test (torch.softmax on a given device): S and O are then pinned bit for bit, the softmax itself is torch's.

Pins: the reference's own outputs on four shapes (tests/golden/attend.npz: chunking, GQA, padding-free and
causal masks, the key-block skip) with torch's CPU softmax, and on three with vector="bf16"
(tests/golden/vector.npz) with oracle/vector.py's rounded softmax over torch's CPU exp and sum; with no mask
and one chunk it reduces to softmax(A^T B * scale) V over the oracle reducers, which the tests check directly.
"""
import math

import numpy as np

F32, F64 = np.float32, np.float64

SLACK = 2.0 ** 16                    # mxq/nn/_attention.py:60-62
ELEMENTS_PER_STEP = 1 << 26          # mxq/nn/_attention.py:55-58
TINY = float(np.finfo(F32).tiny)


class Side:
    """One Scheme as numpy callables: a, b: V -> (P, X); reduce: (P_A, X_A, P_B, X_B) -> Y."""

    def __init__(self, a, b, reduce, rows=1, block_size=32):
        self.a, self.b, self.reduce, self.rows, self.block_size = a, b, reduce, rows, block_size


def amax_rows(P, X, block_size):
    """mxq/nn/_attention.py:65-67."""
    Xr = np.repeat(X, block_size, axis=0)[:P.shape[0]]
    with np.errstate(all="ignore"):
        return (np.abs(P) * Xr).astype(F32).max(axis=1).astype(F64)


def attend(q, k, v, mask, scale, qk, pv, softmax, chunk=None, vector=None):
    """mxq/nn/_attention.py:70-143.  q: B x H x Tq x D, k, v: B x Hkv x Tk x D.  vector=None or "bf16": with
    "bf16" the score steps S * scale and + mask are rounded to bf16 (oracle/vector.py's rounder), and `softmax`
    is expected to be the rounded one (oracle.vector.softmax_bf16 with the device's exp and row sum)."""
    from .vector import rounder
    r = rounder(vector)
    q, k, v = (np.asarray(t, F32) for t in (q, k, v))
    B, H, Tq, D = q.shape
    Hkv, Tk = k.shape[1], k.shape[2]
    assert H % Hkv == 0
    rows = max(qk.rows, pv.rows)
    group = H // Hkv
    bq, bv = qk.block_size, pv.block_size
    step = chunk or max(rows, ELEMENTS_PER_STEP // (group * Tk) // rows * rows)
    sc = F32(scale)
    out = np.zeros((B, Tq, H, D), F32)
    for b in range(B):
        mb = None
        if mask is not None:
            mb = np.asarray(mask[b if mask.shape[0] > 1 else 0, 0, :, :Tk], F32)
            if mb.shape[0] == 1:
                mb = np.broadcast_to(mb, (Tq, Tk))
        for h in range(Hkv):
            KP, KX = qk.b(np.ascontiguousarray(k[b, h].T))
            VP, VX = pv.b(np.ascontiguousarray(v[b, h]))
            kmax = amax_rows(KP, KX, bq) if mb is not None else None
            heads = list(range(h * group, (h + 1) * group))
            for s in range(0, Tq, step):
                e = min(s + step, Tq)
                whole = s + (e - s) // rows * rows
                parts = [(heads, s, whole)] if whole > s else []
                if whole < e:
                    parts += [([hq], whole, e) for hq in heads]
                for hs, s0, e0 in parts:
                    n, m = len(hs), e0 - s0
                    Q = q[b, hs[0]:hs[-1] + 1, s0:e0].reshape(n * m, D)
                    AP, AX = qk.a(np.ascontiguousarray(Q.T))
                    lo, hi = 0, Tk
                    if mb is not None:
                        bound = max(SLACK * abs(scale) * float((amax_rows(AP, AX, bq) * kmax).sum()), TINY)
                        mc = mb[s0:e0]
                        with np.errstate(all="ignore"):
                            bf = F32(bound)
                            absorbed = ((mc + bf) == mc) & ((mc - bf) == mc)
                        seen = np.nonzero(~absorbed.all(axis=0))[0]
                        if seen.size:
                            lo = int(seen[0]) // bv * bv
                            hi = min(Tk, -(-(int(seen[-1]) + 1) // bv) * bv)
                        else:
                            hi = min(Tk, bv)
                    with np.errstate(all="ignore"):
                        live = r((qk.reduce(AP, AX, KP[:, lo:hi], KX[:, lo:hi]) * sc).astype(F32))
                        if mb is not None:
                            live = r((live.reshape(n, m, hi - lo) + mb[s0:e0, lo:hi]).astype(F32)).reshape(n * m, -1)
                    if lo == 0 and hi == Tk:
                        S = live
                    else:
                        S = np.tile(r(np.asarray(mb[s0:e0], F32)), (n, 1))
                        S.reshape(n, m, Tk)[:, :, lo:hi] = live.reshape(n, m, hi - lo)
                    P = np.asarray(softmax(S), F32)
                    if (lo or hi < Tk) and (P[:, :lo].any() or P[:, hi:].any()):
                        lo, hi = 0, Tk
                    PP, PX = pv.a(np.ascontiguousarray(P.T))
                    blk = slice(lo // bv, math.ceil(hi / bv))
                    O = pv.reduce(PP[lo:hi], PX[blk], VP[lo:hi], VX[blk])
                    out[b, s0:e0, hs[0]:hs[-1] + 1] = O.reshape(n, m, D).transpose(1, 0, 2)
    return out
