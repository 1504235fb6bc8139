"""Oracle MX-Gemmini look-up tables: formats (code values, finder fixed points, finder-safe values), tables
(weighted k-means per column group), pick, lookup, finder, and block.lut.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

Follows mxq/lut/formats.py:29-159 and mxq/lut/kmeans.py:27-152 step for step in numpy (float64 k-means, the
same seeding, argmin-first tie rules, dedupe, convergence test, snap and pad order).

Pins: fixtures the reference wrote for tables, finder and the safe-value sets (tests/golden/), which are
functions only an import of the reference pins; pick and lookup against brute-force nearest-entry search.
"""
import math

import numpy as np

from . import block as ob

SIZE = 16
FORMATS = ("MXFP6_E3M2", "MXFP6_E2M3", "MXFP8_E5M2", "MXFP8_E4M3")
_EM = {"MXFP6_E3M2": (3, 2), "MXFP6_E2M3": (2, 3), "MXFP8_E5M2": (5, 2), "MXFP8_E4M3": (4, 3)}
_RTOL, _ATOL = 1e-5, 1e-8


def _fx_e3m2(v):
    """mxq/lut/formats.py:35-42"""
    sign, exp, mant = (v >> 5) & 1, (v >> 2) & 0x7, v & 0x3
    if exp == 0 and mant == 0:
        return 0
    s_exp = -2 if exp == 0 else exp - 3
    sig = (0 if exp == 0 else 4) | mant
    mag = ((sig << ((s_exp + 2) & 0b111)) & 0x1FF) & 0xFF
    return -mag if sign else mag


def _fx_e2m3(v):
    """mxq/lut/formats.py:45-48"""
    sign, exp, mant = (v >> 5) & 1, (v >> 3) & 0x3, v & 0x7
    mag = mant if exp == 0 else ((8 + mant) << (exp - 1))
    return -mag if sign else mag


def _fx_e5m2(v):
    """mxq/lut/formats.py:51-58"""
    sign, exp, mant = (v >> 7) & 1, (v >> 2) & 0x1F, v & 0x3
    if exp == 0 and mant == 0:
        return 0
    sig = (0 if exp == 0 else 4) | mant
    s_exp = (1 - 15) if exp == 0 else exp - 15
    mag = (sig << ((s_exp + 14) & 0x1F)) & 0xFFFFFFFF
    return -mag if sign else mag


def _fx_e4m3(v):
    """mxq/lut/formats.py:61-68"""
    sign, exp, mant = (v >> 7) & 1, (v >> 3) & 0xF, v & 0x7
    if exp == 0 and mant == 0:
        return 0
    sig = (0 if exp == 0 else 8) | mant
    s_exp = (1 - 7) if exp == 0 else exp - 7
    mag = (sig << ((s_exp + 6) & 0xF)) & 0x3FFFF
    return -mag if sign else mag


FINDER = {(3, 2): (_fx_e3m2, 0x1FF), (2, 3): (_fx_e2m3, None), (5, 2): (_fx_e5m2, 0x1FFFFFFFF), (4, 3): (_fx_e4m3, 0x7FFFF)}


def tables_of(name):
    """mxq/lut/formats.py:83-111: (code values float32, code fixed points int64, safe values float32 ascending)."""
    e, m = _EM[name]
    n = 1 << (1 + e + m)
    b = (1 << (e - 1)) - 1
    vals = []
    for c in range(n):
        s, ex, man = (c >> (e + m)) & 1, (c >> m) & ((1 << e) - 1), c & ((1 << m) - 1)
        if (e, m) == (5, 2) and ex == 0x1F:
            v = float("nan") if man else float("inf")
        elif ex == 0:
            v = man * 2.0 ** (1 - b - m)
        else:
            v = (1.0 + man / (1 << m)) * 2.0 ** (ex - b)
        vals.append(-v if s else v)
    fx = [FINDER[(e, m)][0](c) for c in range(n)]
    seen = {}
    for c in range(n):
        v = vals[c]
        if v != v or v in (float("inf"), float("-inf")):
            continue
        if fx[c] not in seen or abs(v) < abs(seen[fx[c]]):
            seen[fx[c]] = v
    safe = sorted(set(seen.values()))
    return np.array(vals, dtype=np.float32), np.array(fx, dtype=np.int64), np.array(safe, dtype=np.float32)


def _dedupe(C):
    """mxq/lut/kmeans.py:37-42"""
    C = np.sort(C, axis=1)
    dup = np.zeros_like(C, dtype=bool)
    dup[:, 1:] = C[:, 1:] == C[:, :-1]
    return np.sort(np.where(dup, np.inf, C), axis=1)


def tables(P, fmt, group, max_iters):
    """mxq/lut/kmeans.py:46-122"""
    all_vals, _, safe = tables_of(fmt)
    P = np.asarray(P, dtype=np.float32)
    K, n = P.shape
    ng = (n + (1 << group) - 1) >> group
    grid = np.unique(all_vals[np.isfinite(all_vals)])
    nv = grid.size
    b = np.searchsorted(grid, P)
    if (b >= nv).any() or not np.array_equal(grid[np.minimum(b, nv - 1)], P):
        raise ValueError(f"mxq.lut: P holds a value that is not a {fmt} code; quantize it first")
    gid = np.broadcast_to(np.arange(n) >> group, P.shape)
    counts = np.bincount((gid * nv + b).reshape(-1), minlength=ng * nv).reshape(ng, nv)
    present = counts > 0
    npres = present.sum(axis=1)
    x = grid.astype(np.float64)
    C = np.full((ng, SIZE), np.inf)
    few = npres <= SIZE
    for g in np.nonzero(few)[0]:
        v = x[present[g]]
        C[g, :v.size] = v
    many = ~few
    if many.any():
        cnt = counts[many]
        cdf = np.cumsum(cnt, axis=1).astype(np.float64) / cnt.sum(axis=1, keepdims=True).astype(np.float64)
        probes = (np.arange(SIZE, dtype=np.float64) + 0.5) / SIZE
        seeds = np.stack([np.searchsorted(cdf[i], probes, side="left") for i in range(cnt.shape[0])])
        seeds = np.minimum(seeds, nv - 1)
        C[many] = _dedupe(x[seeds])
        Cm, w = C[many].copy(), cnt.astype(np.float64)
        live = np.ones(Cm.shape[0], dtype=bool)
        for _ in range(max_iters):
            if not live.any():
                break
            idx = np.nonzero(live)[0]
            Cl, wl = Cm[idx], w[idx]
            with np.errstate(invalid="ignore"):
                lab = np.abs(x.reshape(1, -1, 1) - Cl[:, None, :]).argmin(axis=2)
            sums = np.zeros_like(Cl)
            wsum = np.zeros_like(Cl)
            rows = np.repeat(np.arange(Cl.shape[0])[:, None], nv, axis=1)
            np.add.at(sums, (rows, lab), wl * x)
            np.add.at(wsum, (rows, lab), wl)
            with np.errstate(invalid="ignore", divide="ignore"):
                new = _dedupe(np.where(wsum > 0, sums / wsum, Cl))
                valid = np.isfinite(Cl)
                same = (np.isfinite(new) == valid).all(axis=1) & \
                    ((np.abs(new - Cl) <= _ATOL + _RTOL * np.abs(Cl)) | ~valid).all(axis=1)
            Cm[idx[~same]] = new[~same]
            live[idx[same]] = False
        C[many] = Cm
    s = safe.astype(np.float64)
    valid = np.isfinite(C)
    with np.errstate(invalid="ignore"):
        near = np.abs(C[:, :, None] - s[None, None, :]).argmin(axis=2)
    member = np.zeros((ng, s.size), dtype=bool)
    for g in range(ng):
        member[g, near[g][valid[g]]] = True
    order = np.array(sorted(range(s.size), key=lambda i: abs(float(safe[i]))))
    free = ~member[:, order]
    take = free & (np.cumsum(free, axis=1) <= (SIZE - member.sum(axis=1, keepdims=True)))
    member[:, order] |= take
    T = np.sort(np.where(member, safe[None, :], np.float32(np.inf)), axis=1)[:, :SIZE]
    return np.ascontiguousarray(T, dtype=np.float32)


def pick(P, T, group):
    """mxq/lut/kmeans.py:125-138"""
    P = np.asarray(P, dtype=np.float32)
    n = P.shape[1]
    size = T.shape[1]
    rows = T.astype(np.float32)[np.arange(n) >> group]
    v = P.T
    hi = np.stack([np.searchsorted(rows[j], v[j], side="left") for j in range(n)])
    hi = np.clip(hi, 1, size - 1)
    lo = hi - 1
    d_lo = np.abs(v - np.take_along_axis(rows, lo, 1))
    d_hi = np.abs(np.take_along_axis(rows, hi, 1) - v)
    return np.ascontiguousarray(np.where(d_lo <= d_hi, lo, hi).T.astype(np.int64))


def lookup(I, T, group):
    """mxq/lut/kmeans.py:141-146"""
    n = I.shape[1]
    rows = T.astype(np.float32)[np.arange(n) >> group]
    return np.ascontiguousarray(np.take_along_axis(rows, I.T, 1).T.astype(np.float32))


def encode(T, fmt):
    """mxq/lut/formats.py:125-137"""
    vals = tables_of(fmt)[0]
    lk = {}
    for c, bits in enumerate(vals.view(np.int32).tolist()):
        lk.setdefault(bits, c)
    flat = np.asarray(T, dtype=np.float32).reshape(-1).view(np.int32).tolist()
    return np.array([lk[b] for b in flat], dtype=np.int64).reshape(np.shape(T))


def finder(codes, T, fmt, group):
    """mxq/lut/formats.py:140-159"""
    e, m = _EM[fmt]
    mask = FINDER[(e, m)][1]
    fx_all = tables_of(fmt)[1]
    n = codes.shape[1]
    fx = fx_all[np.asarray(codes, dtype=np.int64)]
    lut_fx = fx_all[encode(T, fmt)]
    cols = np.arange(n) >> group
    d = np.abs(fx[:, :, None] - lut_fx[cols][None, :, :])
    if mask is not None:
        d = d & mask
    return d.argmin(axis=-1).astype(np.int64)


def lut_quantize(V, fmt, axis, block_size, rounding_mode, scale_floor, group, max_iters):
    """mxq/block/lut.py:23-34"""
    P, X = ob.mxgemmini_quantize(V, fmt, axis, block_size, rounding_mode, scale_floor)
    Pk = P if axis % 2 == 0 else P.T
    T = tables(Pk, fmt, group, max_iters)
    P_lut = lookup(pick(Pk, T, group), T, group)
    return np.ascontiguousarray(P_lut if axis % 2 == 0 else P_lut.T), X


def nv_of(fmt):
    vals = tables_of(fmt)[0]
    return np.unique(vals[np.isfinite(vals)]).size


def ceil_groups(n, group):
    return math.ceil(n / (1 << group))
