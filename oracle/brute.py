"""Brute-force and exact-rational models that pin the oracle's numerics on small inputs.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

Nothing here shares a formula with oracle/numerics.py: rounding is a search for the nearest member of an
enumerated grid (ties by the grid index, which alternates parity exactly as the significand's last bit does),
sums are exact (float64 where every operand sits on a narrow grid, fractions.Fraction otherwise), and the
systolic, adder-tree and anchor-tree models walk one output at a time in Python scalars.  A slip in the oracle's step, exponent, tie or
sign handling makes one of them disagree.
"""
from fractions import Fraction
from functools import lru_cache

import numpy as np

F32, F64 = np.float32, np.float64


@lru_cache(maxsize=None)
def _grid(e, m, top_exp):
    b = (1 << (e - 1)) - 1
    emin = 1 - b
    top = b if top_exp is None else top_exp
    vals = [k * 2.0 ** (emin - m) for k in range(1 << m)]                            # zero and subnormals
    for E in range(emin, top + 1):
        vals += [(1 + j / (1 << m)) * 2.0 ** E for j in range(1 << m)]
    vals.append(2.0 ** (top + 1))
    out = np.array(vals, dtype=F64)
    out.flags.writeable = False
    return out


def grid(e, m, top_exp=None):
    """Non-negative values of a float with e exponent bits (bias 2^(e-1)-1, subnormals) and m fraction bits,
    ascending, through binade top_exp (default: the format's emax = bias), plus the next power of two as the
    overflow sentinel.  float64, exact."""
    return _grid(e, m, top_exp)


def nearest(ax, g, mode):
    """Round non-negative exact values `ax` (float64) onto ascending grid `g`: truncate = the largest member not
    above; otherwise the nearer neighbour, ties to the even index (rne) or to the larger (ties_away).
    Values above the grid's last member map to it."""
    ax = np.asarray(ax, F64)
    hi_i = np.clip(np.searchsorted(g, ax, side="left"), 0, len(g) - 1)
    exact = g[hi_i] == ax
    lo_i = np.where(exact, hi_i, np.maximum(hi_i - 1, 0))
    lo, hi = g[lo_i], g[hi_i]
    if mode == "truncate":
        return np.where(ax >= g[-1], g[-1], np.where(exact, hi, lo))
    d_lo, d_hi = ax - lo, hi - ax
    tie = d_lo == d_hi
    pick_hi = d_hi < d_lo
    if mode == "rne":
        pick_hi = pick_hi | (tie & (hi_i % 2 == 0))
    elif mode == "ties_away":
        pick_hi = pick_hi | tie
    else:
        raise ValueError(mode)
    out = np.where(exact, hi, np.where(pick_hi, hi, lo))
    return np.where(ax >= g[-1], g[-1], out)


def _f32_ties_away(ax, r, g, mode, e):
    """The one place float32 ties_away (floor(k + 0.5) computed in float32) leaves the nearest value:
    k = 0.5 - 2^-25 of the subnormal step, where k + 0.5 rounds to 1.0 before the floor.  Narrow formats
    only; e = 8 rounds in float64, where the same point is not a float32 input."""
    if mode != "ties_away" or e >= 8:
        return r
    return np.where(ax == (0.5 - 2.0 ** -25) * g[1], g[1], r)


def ieee_em(x, e, m, mode):
    """float_em's ieee grid by search: nearest value, results at or past 2^(emax+1) become Inf, a nonzero value
    of a narrow format (e < 8) that rounds to zero becomes +0; NaN, +-Inf and +-0 pass through."""
    x = np.asarray(x, F64)
    g = grid(e, m)
    nz = np.isfinite(x) & (x != 0)
    ax = np.where(nz, np.abs(x), 0)
    r = _f32_ties_away(ax, nearest(ax, g, mode), g, mode, e)
    r = np.where(r >= g[-1], np.inf, r)
    out = np.where(nz, np.copysign(r, x), x)
    if e < 8:
        out = np.where(nz & (r == 0), 0.0, out)
    return out


def ocp_em(x, e, m, mode, max_norm):
    """float_em's ocp grid by search: nearest on the unbounded-above grid, clamped at max_norm, zeros +0,
    NaN and +-Inf pass through."""
    x = np.asarray(x, F64)
    g = grid(e, m, top_exp=40)
    fin = np.isfinite(x)
    ax = np.where(fin, np.abs(x), 0)
    r = np.minimum(_f32_ties_away(ax, nearest(ax, g, mode), g, mode, e), max_norm)
    out = np.where(fin, np.copysign(r, x), x)
    return np.where(x == 0, 0.0, out)


def round_significand_bits(x32, keep, mode):
    """A finite float32 rounded to `keep` fraction bits on float32's own exponent range (subnormals at the
    float32 subnormal step), by search on the ieee(8, keep) grid."""
    return ieee_em(np.asarray(x32, F32).astype(F64), 8, keep, mode)


def truncate_bits(x32, m):
    """Keep m fraction bits toward zero by clearing bit-pattern bits; subnormals are normalised first by
    scaling with 2^64 (exact), so their leading 1 counts as the implicit bit."""
    x = np.asarray(x32, F32)
    out = np.empty_like(x)
    for i, v in enumerate(x.reshape(-1)):
        if not np.isfinite(v) or v == 0:
            out.reshape(-1)[i] = v
            continue
        scale = 1.0
        if abs(v) < 2.0 ** -126:
            v = F32(v * F32(2.0 ** 64))
            scale = 2.0 ** -64
        u = np.array(v, F32).view(np.uint32)
        u = np.uint32(u & np.uint32(~((1 << (23 - m)) - 1) & 0xFFFFFFFF))
        out.reshape(-1)[i] = F32(float(np.array(u, np.uint32).view(F32)) * scale)
    return out


def exact_round_fraction(q, e, m, mode="rne"):
    """An exact rational q rounded to the ieee(e, m) grid (nearest, ties even), Inf past 2^(emax+1); float."""
    if q == 0:
        return 0.0
    g = grid(e, m)
    a = abs(q)
    i = int(np.searchsorted(g, float(a), side="left"))
    cand = [j for j in (i - 2, i - 1, i, i + 1) if 0 <= j < len(g)]
    best = min(cand, key=lambda j: (abs(Fraction(g[j]) - a), 0 if (mode == "rne" and j % 2 == 0) else 1))
    v = g[best]
    if v >= g[-1]:
        v = float("inf")
    return -v if q < 0 else v


def exact_add(a, b, e, m):
    """mxq arith.exact_add by exact rationals: a + b with one rounding (ties even), a zero operand returns
    the other operand unchanged."""
    a, b = float(a), float(b)
    if a == 0:
        return b
    if b == 0:
        return a
    if not (np.isfinite(a) and np.isfinite(b)):
        return a + b
    r = exact_round_fraction(Fraction(a) + Fraction(b), e, m)
    return 0.0 if r == 0 else r


def mxgemmini_product(a, b, prod_m=3, floor_exp=-16, limit=448.0, value=448.0):
    """One MXGEMMINI product in exact scalars: a*b truncated to prod_m fraction bits, flushed to +0 below
    2^floor_exp, saturated to sign*value above limit."""
    p = Fraction(float(a)) * Fraction(float(b))
    if p == 0:
        return 0.0
    s = -1 if p < 0 else 1
    ap = abs(p)
    E = ap.numerator.bit_length() - ap.denominator.bit_length()
    while Fraction(2) ** E > ap:
        E -= 1
    while Fraction(2) ** (E + 1) <= ap:
        E += 1
    step = Fraction(2) ** (E - prod_m)
    t = (ap // step) * step
    if floor_exp is not None and t < Fraction(2) ** floor_exp:
        return 0.0
    if t > Fraction(limit):
        t = Fraction(value)
    return s * float(t)


def systolic_mxgemmini(P_A, X_A, P_B, X_B, schedule, size=16, block_size=32):
    """The MXGEMMINI PE column one output at a time: per block, per run of `size` k, lane sums in the
    schedule's formats (lane = round to the lane grid, zeros unsigned), then the block's sum times its two
    scales (one float32 rounding) added into a bf16 accumulator."""
    P_A, X_A, P_B, X_B = (np.asarray(t, F32) for t in (P_A, X_A, P_B, X_B))
    K, M = P_A.shape
    N = P_B.shape[1]

    def lane(x, e, m):
        r = exact_round_fraction(Fraction(float(x)), e, m) if np.isfinite(x) else float(x)
        return 0.0 if r == 0 else r

    C = np.zeros((M, N), F32)
    for i in range(M):
        for j in range(N):
            c = 0.0
            for g0 in range(0, K, block_size):
                sc = F32(X_A[g0 // block_size, i]) * F32(X_B[g0 // block_size, j])
                for k0 in range(g0, min(g0 + block_size, K), size):
                    S = 0.0
                    for k in range(k0, min(k0 + size, g0 + block_size, K)):
                        e, m = schedule[k % size]
                        p = mxgemmini_product(P_A[k, i], P_B[k, j])
                        S = exact_add(lane(S, e, m), lane(p, e, m), e, m)
                    tile = float(F32(F32(S) * sc))
                    c = exact_add(lane(c, 8, 7), lane(tile, 8, 7), 8, 7)
            C[i, j] = c
    return C


def _mxg_lane(x, e, m):
    """An MXGEMMINI lane value: x on the ieee(e, m) grid, nearest, ties even; zeros unsigned."""
    r = exact_round_fraction(Fraction(float(x)), e, m) if np.isfinite(x) else float(x)
    return 0.0 if r == 0 else r


def _mxg_acc(a, b, e, m):
    return exact_add(_mxg_lane(a, e, m), _mxg_lane(b, e, m), e, m)


def _bf16_tile(c, S, sc):
    tile = float(F32(F32(S) * sc))
    return exact_add(_mxg_lane(c, 8, 7), _mxg_lane(tile, 8, 7), 8, 7)


def _blocks(K, size, block_size):
    """(first k of the block, first k of the reduction, its product count) in the reducers' order."""
    for g0 in range(0, K, block_size):
        for k0 in range(g0, min(g0 + block_size, K), size):
            yield g0, k0, min(k0 + size, g0 + block_size, K) - k0


def adder_tree_mxgemmini(P_A, X_A, P_B, X_B, schedule, size=16, block_size=32):
    """The MXGEMMINI adder tree one output at a time: a reduction's `size` exact-scalar products (zeros past a
    tail) halved level by level, each pair summed exactly and rounded once to its level's format."""
    P_A, X_A, P_B, X_B = (np.asarray(t, F32) for t in (P_A, X_A, P_B, X_B))
    K, M = P_A.shape
    N = P_B.shape[1]
    C = np.zeros((M, N), F32)
    for i in range(M):
        for j in range(N):
            c = 0.0
            for g0, k0, n in _blocks(K, size, block_size):
                sc = F32(X_A[g0 // block_size, i]) * F32(X_B[g0 // block_size, j])
                vals = [mxgemmini_product(P_A[k, i], P_B[k, j]) for k in range(k0, k0 + n)] + [0.0] * (size - n)
                for e, m in schedule:
                    vals = [_mxg_acc(vals[2 * q], vals[2 * q + 1], e, m) for q in range(len(vals) // 2)]
                c = _bf16_tile(c, vals[0], sc)
            C[i, j] = c
    return C


def _exp_label(x):
    """floor(log2|x|) of a finite nonzero float from its exact binary expansion; -1 for zero and non-finite
    values (they never decide an anchor through it)."""
    x = float(x)
    if x == 0 or not np.isfinite(x):
        return -1
    q = abs(Fraction(x))
    E = q.numerator.bit_length() - q.denominator.bit_length()
    while Fraction(2) ** E > q:
        E -= 1
    while Fraction(2) ** (E + 1) <= q:
        E += 1
    return E


def _drop_to_int(q, drop):
    """An exact rational made an integer: toward zero, or nearest with ties to even."""
    if drop == "truncate":
        return Fraction(int(q))                       # int() of a Fraction truncates toward zero
    fl = q.numerator // q.denominator
    rem = q - fl
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and fl % 2 == 1):
        fl += 1
    return Fraction(fl)


def anchor_tree_mxgemmini(P_A, X_A, P_B, X_B, schedule, size, width, bits_of, drop, headroom, emin=None,
                          block_size=32):
    """The MXGEMMINI anchor tree one output at a time in exact rationals.  bits_of(m) gives a tree's level
    widths.  Per tree: the anchor is the largest label among its nonzero products (code-exponent sum, at least
    emin per code when given) and the running sum c (its exponent minus one), plus headroom; every term is cut
    to an integer multiple of 2^(anchor + 2 - bits[0]); terms are summed in adjacent pairs, products first and
    c last, an odd one carried up, and cut again where the level width falls; the root is rounded to float32,
    then to the tree's lane."""
    P_A, X_A, P_B, X_B = (np.asarray(t, F32) for t in (P_A, X_A, P_B, X_B))
    K, M = P_A.shape
    N = P_B.shape[1]

    def label(x):
        lab = _exp_label(x)
        return lab if emin is None else max(lab, emin)

    C = np.zeros((M, N), F32)
    for i in range(M):
        for j in range(N):
            cacc = 0.0
            for g0, k0, n in _blocks(K, size, block_size):
                sc = F32(X_A[g0 // block_size, i]) * F32(X_B[g0 // block_size, j])
                c = 0.0
                for t, (e, m) in enumerate(schedule):
                    bits = bits_of(m)
                    ks = [k for k in range(k0 + t * width, k0 + (t + 1) * width) if k < k0 + n]
                    prods = [mxgemmini_product(P_A[k, i], P_B[k, j]) for k in ks]
                    labs = [label(P_A[k, i]) + label(P_B[k, j]) for k in ks]
                    cands = [lb for pv, lb in zip(prods, labs) if pv != 0]
                    if c != 0:
                        cands.append(_exp_label(c) - 1)
                    anchor = (max(cands) if cands else 0) + headroom
                    step = Fraction(2) ** (anchor + 2 - bits[0])
                    terms = prods + [0.0] * (width - len(prods)) + [c]
                    x = [_drop_to_int(Fraction(float(v)) / step, drop) for v in terms]
                    for lvl in range(1, len(bits)):
                        nxt = [x[2 * q] + x[2 * q + 1] for q in range(len(x) // 2)]
                        if len(x) % 2:
                            nxt.append(x[-1])
                        if bits[lvl] != bits[lvl - 1]:
                            nxt = [_drop_to_int(v / Fraction(2) ** (bits[lvl - 1] - bits[lvl]), drop) for v in nxt]
                        x = nxt
                    root = x[0] * Fraction(2) ** (anchor + 2 - bits[-1])
                    assert Fraction(float(root)) == root            # an integer below 2^53 times a power of two
                    c = _mxg_lane(float(F32(float(root))), e, m)   # one rounding to float32, then the lane
                cacc = _bf16_tile(cacc, c, sc)
            C[i, j] = cacc
    return C


def pick(P, T, group):
    """Nearest table entry per element by exhaustive comparison, ties to the lower index."""
    P = np.asarray(P, F64)
    K, n = P.shape
    out = np.zeros((K, n), np.int64)
    for j in range(n):
        row = np.asarray(T[j >> group], F64)
        d = np.abs(P[:, j:j + 1] - row[None, :])
        out[:, j] = np.argmin(d, axis=1)                                             # first minimum
    return out
