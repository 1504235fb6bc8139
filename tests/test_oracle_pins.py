"""What pins the oracle, on the CPU: torch's own kernels where the reference calls them (log2, exp2, bf16 and
float8 casts, softmax is torch's by construction), brute-force grid searches and exact rationals
(oracle/brute.py) for the rounding grids, exact_add, truncate, the MXGEMMINI product and the systolic column,
closed-form boundary values for flush/saturate/scale rules, exhaustive nearest search for pick."""
import numpy as np
import pytest
import torch

from _util import assert_bits_equal
from oracle import block as ob
from oracle import brute
from oracle import lut as ol
from oracle import numerics as nx
from oracle import systolic as osys

F32, F64 = np.float32, np.float64
RNG = np.random.default_rng(20261202)


def _random_finite_f32(n, lo_exp=-149, hi_exp=127):
    e = RNG.integers(lo_exp, hi_exp, n)
    v = np.ldexp(RNG.uniform(1, 2, n), e) * RNG.choice([-1.0, 1.0], n)
    return v.astype(F32)


def _near_grid(g, n_each=3):
    """Grid members, midpoints and their float32 neighbours (where ties and carries live)."""
    g = g[:-1]
    mids = (g[:-1] + g[1:]) / 2
    pts = np.concatenate([g, mids]).astype(F32)
    return np.concatenate([pts, np.nextafter(pts, F32(np.inf)), np.nextafter(pts, F32(0))])


# ---- torch pins -----------------------------------------------------------------------------------------

def test_log2_matches_torch():
    """floor of the oracle's log2 (float64 log2 rounded once) is floor of torch.log2 on float32, the only way
    the reference uses log2, including the round-up band just below every power of two where both give the
    upper binade.  (Away from integers torch's float32 log2 is off by an ulp now and then: 2 in 200000.)"""
    pows = np.ldexp(np.ones(277, F32), np.arange(-149, 128)).astype(F32)
    x = np.concatenate([pows, *(np.nextafter(pows, F32(0)) for _ in range(1)), _random_finite_f32(200000)])
    band = pows.copy()
    for _ in range(40):                                                   # 40 ulps below each power of two
        band = np.nextafter(band, F32(0))
        x = np.concatenate([x, band])
    x = np.abs(x[np.isfinite(x) & (x != 0)])
    mine, theirs = nx.log2_f32(x), torch.log2(torch.from_numpy(x)).numpy()
    assert_bits_equal(np.floor(mine), np.floor(theirs), "floor(log2)")


def test_exp2_int_matches_torch():
    t = np.arange(-160, 140).astype(F32)
    assert_bits_equal(nx.exp2_int(t), torch.exp2(torch.from_numpy(t)).numpy(), "exp2")
    assert_bits_equal(nx.exp2_int(t), torch.pow(2.0, torch.from_numpy(t)).numpy(), "pow")


def test_bf16_matches_torch_cast_and_search():
    bits = RNG.integers(0, 1 << 32, 400000, dtype=np.int64).astype(np.uint32)
    x = bits.view(F32)
    x = x[~np.isnan(x)]
    assert_bits_equal(nx.bf16(x), torch.from_numpy(x).to(torch.bfloat16).float().numpy(), "bf16 vs torch")
    fin = x[np.isfinite(x)][:50000]
    assert_bits_equal(nx.bf16(fin), brute.round_significand_bits(fin, 7, "rne").astype(F32), "bf16 vs search")


@pytest.mark.parametrize("mode", ["rne", "ties_away", "truncate"])
def test_round_bits_is_nearest_on_the_grid(mode):
    x = np.concatenate([_random_finite_f32(6000), _random_finite_f32(2000, -149, -120)])
    for keep in (1, 2, 3, 5, 7, 10):                                       # grids up to 260k members
        got = nx.from_bits(nx.round_bits(nx.bits_of(x), keep, mode))
        want = brute.round_significand_bits(x, keep, mode).astype(F32)
        assert_bits_equal(got, want, f"round_bits keep={keep} {mode}")


def test_round_int_rules():
    k = np.array([0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 0.49999997, 2.4999998, 1e8 + 0.0, 3.0], F32)
    assert list(nx.round_int(k, "rne")) == [0, 2, 2, -0, -2, -2, 0, 2, 1e8, 3]
    # ties_away is sign * floor(|k| + 0.5) in float32: 0.5 - 2^-25 + 0.5 rounds to 1.0 before the floor
    assert list(nx.round_int(k, "ties_away")) == [1, 2, 3, -1, -2, -3, 1, 2, 1e8, 3]
    assert list(nx.round_int(k, "truncate")) == [0, 1, 2, -0, -1, -2, 0, 2, 1e8, 3]
    # torch.round is half-even, as the reference's rne integer rounding calls it
    z = np.concatenate([k, _random_finite_f32(10000, -3, 30)])
    assert_bits_equal(nx.round_int(z, "rne"), torch.round(torch.from_numpy(z)).numpy(), "rne vs torch.round")


def test_float8_casts():
    """ocp E4M3 rne is torch's float8_e4m3fn cast inside +-448; ieee E5M2 rne is torch's float8_e5m2 cast
    (overflow to Inf included).  Zero signs differ by rule: the ocp grid makes an input of -0 into +0 (a
    negative value that rounds to zero stays -0), the ieee grid of a narrow format makes a nonzero value that
    rounds to zero +0 (an input of -0 stays -0)."""
    x = np.concatenate([_near_grid(brute.grid(4, 3, 8)), _random_finite_f32(50000, -12, 9)])
    x = np.concatenate([x, -x])
    x = x[np.abs(x) <= 448]
    t = torch.from_numpy(x).to(torch.float8_e4m3fn).float().numpy()
    t = np.where(x == 0, F32(0), t)
    assert_bits_equal(nx.float_em(x, 4, 3, "rne", "ocp"), t, "E4M3 vs torch")
    y = np.concatenate([_near_grid(brute.grid(5, 2)), _random_finite_f32(50000, -20, 17)])
    y = np.concatenate([y, -y])
    t = torch.from_numpy(y).to(torch.float8_e5m2).float().numpy()
    t = np.where((t == 0) & (y != 0), F32(0), t)
    assert_bits_equal(nx.float_em(y, 5, 2, "rne", "ieee"), t, "E5M2 vs torch")


# ---- grid searches --------------------------------------------------------------------------------------

IEEE_FORMATS = [(4, 3), (4, 4), (4, 5), (4, 6), (5, 2), (3, 2), (2, 3), (2, 1), (5, 10), (6, 9), (8, 7)]


@pytest.mark.parametrize("em", IEEE_FORMATS, ids=lambda em: f"e{em[0]}m{em[1]}")
@pytest.mark.parametrize("mode", ["rne", "ties_away", "truncate"])
def test_ieee_grid_is_nearest(em, mode):
    e, m = em
    b = (1 << (e - 1)) - 1
    x = np.concatenate([_near_grid(brute.grid(e, m)), _random_finite_f32(20000, -b - m - 3, b + 3),
                        np.array([0.0, -0.0, np.inf, -np.inf, np.nan], F32)])
    x = np.concatenate([x, -x])
    got = nx.float_em(x, e, m, mode, "ieee")
    want = brute.ieee_em(x.astype(F64), e, m, mode).astype(F32)
    assert_bits_equal(got, want, f"ieee e{e}m{m} {mode}")


@pytest.mark.parametrize("fmt", list(nx.FORMATS))
@pytest.mark.parametrize("mode", ["rne", "ties_away", "truncate"])
def test_ocp_grid_is_nearest_then_clamped(fmt, mode):
    e, m, emax, mn = nx.FORMATS[fmt][:4]
    x = np.concatenate([_near_grid(brute.grid(e, m, emax + 2)), _random_finite_f32(20000, -12, emax + 4),
                        np.array([0.0, -0.0, np.inf, -np.inf, np.nan], F32)])
    x = np.concatenate([x, -x])
    got = nx.float_em(x, e, m, mode, "ocp")
    want = brute.ocp_em(x.astype(F64), e, m, mode, mn).astype(F32)
    assert_bits_equal(got, want, f"ocp {fmt} {mode}")


@pytest.mark.parametrize("em", [(4, 3), (5, 2), (3, 2), (2, 3), (2, 1), (4, 5)], ids=lambda em: f"e{em[0]}m{em[1]}")
def test_qtorch_grid_in_range(em):
    """qtorch keeps normals only, binades 2^-b .. 2^b (b = bias): inside them it is nearest with ties away,
    past the top it saturates to the largest normal, and the underflow rule sends a rounded magnitude above
    2^(-b-1) to 2^-b and anything else to +0."""
    e, m = em
    b = (1 << (e - 1)) - 1
    normals = np.array([(1 + j / (1 << m)) * 2.0 ** E for E in range(-b, b + 1) for j in range(1 << m)]
                       + [2.0 ** (b + 1)])
    x = np.concatenate([_near_grid(normals), _random_finite_f32(20000, -b, b + 1)])
    x = x[(np.abs(x) >= 2.0 ** -b)]
    x = np.concatenate([x, -x])
    got = nx.float_em(x, e, m, "ties_away", "qtorch").astype(F64)
    want = brute.nearest(np.abs(x).astype(F64), normals, "ties_away")
    top = normals[-2]
    want = np.copysign(np.where(want >= normals[-1], top, want), x)
    assert np.array_equal(got, want)
    under = np.array([2.0 ** (-b - 1) * 1.25, 2.0 ** (-b - 1), 2.0 ** (-b - 3), -2.0 ** (-b - 1) * 1.5, 1e30], F32)
    out = nx.float_em(under, e, m, "ties_away", "qtorch")
    assert list(out.astype(F64)) == [2.0 ** -b, 0.0, 0.0, -(2.0 ** -b), top]


def test_microsoft_nearest_is_ocp_grid_ties_away():
    """microxcaling's element step with 'nearest' is the OCP grid with ties away, clamped at max_norm; 'floor'
    is truncation, except in the log2 round-up band below each power of two, where torch.log2 picks the
    upper binade and truncation lands one step lower."""
    for fmt, (e, m, emax, mn, ms) in nx.FORMATS.items():
        x = np.concatenate([_near_grid(brute.grid(e, m, emax + 1)), _random_finite_f32(20000, -10, emax + 2)])
        x = np.concatenate([x, -x])
        got = nx.microsoft_fmt(x, fmt, "nearest")
        assert_bits_equal(got, brute.ocp_em(x.astype(F64), e, m, "ties_away", mn).astype(F32), f"{fmt} nearest")
        fl = nx.microsoft(x, ms[0], ms[1], mn, "floor")
        band = np.floor(nx.log2_f32(np.abs(x))) != (np.frexp(np.abs(x))[1] - 1)
        want = brute.ocp_em(x.astype(F64), e, m, "truncate", mn).astype(F32)
        assert_bits_equal(fl[~band], want[~band], f"{fmt} floor")


@pytest.mark.parametrize("fmt", list(nx.FORMATS))
def test_microsoft_dither_pins(fmt):
    """microxcaling's dither (floor(|A| + u)) pinned without retyping it: u = 0.5 everywhere is its "nearest";
    u = 0 is its "floor"; every result is the floor or the next value up (the floor with u just below 1); and
    stochastic rounding is unbiased, the mean over uniform draws of u being A itself (within 6 standard errors of
    the grid step) for values inside the format's range."""
    eb, mb, _, mn = nx.FORMATS[fmt][4]
    rng = np.random.default_rng(7)
    A = (rng.standard_normal(4000) * np.exp2(rng.integers(-10, 6, 4000))).astype(np.float32)
    A = A[np.abs(A) < mn / 2]
    half, zero = np.full(A.shape, 0.5, np.float32), np.zeros(A.shape, np.float32)
    top = np.full(A.shape, np.nextafter(np.float32(1), np.float32(0)), np.float32)
    assert_bits_equal(nx.microsoft(A, eb, mb, mn, "dither", True, half), nx.microsoft(A, eb, mb, mn, "nearest"), "u=1/2")
    assert_bits_equal(nx.microsoft(A, eb, mb, mn, "dither", True, zero), nx.microsoft(A, eb, mb, mn, "floor"), "u=0")
    lo, hi = nx.microsoft(A, eb, mb, mn, "floor"), nx.microsoft(A, eb, mb, mn, "dither", True, top)
    u = rng.random(A.shape).astype(np.float32)
    d = nx.microsoft(A, eb, mb, mn, "dither", True, u)
    assert np.all((d == lo) | (d == hi)) and np.all(np.abs(hi) >= np.abs(lo))
    draws = 400
    mean = np.mean([nx.microsoft(A, eb, mb, mn, "dither", True, rng.random(A.shape).astype(np.float32))
                    for _ in range(draws)], axis=0, dtype=np.float64)
    step = np.abs(hi.astype(np.float64) - lo.astype(np.float64))
    assert np.all(np.abs(mean - A) <= 6 * step * 0.5 / np.sqrt(draws) + 1e-30)


# ---- exact rationals ------------------------------------------------------------------------------------

@pytest.mark.parametrize("em", [(4, 3), (4, 4), (4, 6), (6, 9), (5, 10), (8, 7)], ids=lambda em: f"e{em[0]}m{em[1]}")
def test_exact_add_is_one_rounding(em):
    """The three paths of exact_add (fp32, TwoSum pair, float64) against exact rational sums."""
    e, m = em
    g = brute.grid(e, m)[:-1]
    n = 4000
    if e == 8:
        a = nx.bf16(_random_finite_f32(n, -133, 127))
        b = nx.bf16(np.where(RNG.random(n) < 0.5, _random_finite_f32(n, -133, 127),
                             a * RNG.uniform(-1.01, -0.99, n).astype(F32)))
    else:
        a = (RNG.choice(g, n) * RNG.choice([-1, 1], n)).astype(F32)
        b = (RNG.choice(g, n) * RNG.choice([-1, 1], n)).astype(F32)
        b[:200] = -a[:200]                                                  # exact cancellations
        b[200:300] = 0
    got = nx.exact_add(a, b, e, m)
    want = np.array([brute.exact_add(x, y, e, m) for x, y in zip(a, b)], F32)
    assert_bits_equal(got, want, f"exact_add e{e}m{m}")


def test_truncate_significand_by_bits():
    x = np.concatenate([_random_finite_f32(3000), _random_finite_f32(1000, -149, -126),
                        np.array([0.0, -0.0, np.inf, -np.inf], F32)])
    for m in (1, 3, 5, 7, 10):
        assert_bits_equal(nx.truncate_significand(x, m), brute.truncate_bits(x, m), f"truncate m={m}")


def test_flush_and_saturate_boundaries():
    t = F32(2.0 ** -16)
    x = np.array([t, np.nextafter(t, F32(0)), -t, -np.nextafter(t, F32(0)), 0.0, -0.0, 1.0], F32)
    assert list(nx.flush_product(x, -16)) == [t, 0, -t, 0, 0, 0, 1]
    assert np.signbit(nx.flush_product(np.array([-1e-30], F32), -16)[0]) == False  # noqa: E712 (+0)
    s = nx.saturate(np.array([448, 449, -449, 1e30, -0.0, np.inf, np.nan], F32), 448.0, 448.0)
    assert list(s[:6]) == [448, 448, -448, 448, 0, 448] and np.isnan(s[6]) and not np.signbit(s[4])
    assert nx.saturation(4, 3) == (448.0, 448.0)
    assert nx.saturation(5, 2)[0] == 57344.0


def test_mxgemmini_product_exact():
    a = np.concatenate([RNG.choice(brute.grid(4, 3)[:-1], 3000), [448, 448, 2.0 ** -9]]).astype(F32)
    b = np.concatenate([RNG.choice(brute.grid(4, 3)[:-1], 3000), [448, -2, 2.0 ** -9]]).astype(F32)
    b = b * RNG.choice([-1, 1], b.size).astype(F32)
    a = a * np.exp2(RNG.integers(-8, 6, a.size)).astype(F32)
    got = nx.MXGEMMINI().product(a, b)
    want = np.array([brute.mxgemmini_product(x, y) for x, y in zip(a, b)], F32)
    assert_bits_equal(got, want, "product")


# ---- the systolic column and pick ------------------------------------------------------------------------

@pytest.mark.parametrize("K,M,N,scale_b", [(64, 3, 4, 0.05), (40, 2, 3, 0.05), (32, 2, 2, 30.0)])
def test_systolic_against_scalar_model(K, M, N, scale_b):
    A = (RNG.standard_normal((K, M)) * 2).astype(F32)
    B = (RNG.standard_normal((K, N)) * scale_b).astype(F32)
    A[:, 0] *= 1e-6                                                       # products flushed
    PA, XA = ob.mxgemmini_quantize(A, "MXFP8_E4M3", 0)
    PB, XB = ob.mxgemmini_quantize(B, "MXFP8_E4M3", 0)
    got = osys.systolic(PA, XA, PB, XB, nx.MXGEMMINI(), osys.HW_FINAL)
    want = brute.systolic_mxgemmini(PA, XA, PB, XB, osys.HW_FINAL)
    assert_bits_equal(got, want, f"systolic {K}x{M}x{N}")


def test_systolic_columns_independent_and_zero_blocks():
    A = RNG.standard_normal((96, 6)).astype(F32)
    B = (RNG.standard_normal((96, 8)) * 0.1).astype(F32)
    PA, XA = ob.mxgemmini_quantize(A, "MXFP8_E4M3", 0)
    PB, XB = ob.mxgemmini_quantize(B, "MXFP8_E4M3", 0)
    full = osys.systolic(PA, XA, PB, XB, nx.MXGEMMINI(), osys.HW_FINAL)
    part = osys.systolic(PA, XA, PB[:, 2:5], XB[:, 2:5], nx.MXGEMMINI(), osys.HW_FINAL)
    assert_bits_equal(full[:, 2:5], part, "column slice")
    PA0 = PA.copy()
    PA0[32:64] = 0
    z = osys.systolic(PA0, XA, PB, XB, nx.MXGEMMINI(), osys.HW_FINAL)
    drop = osys.systolic(np.concatenate([PA[:32], PA[64:]]), np.concatenate([XA[:1], XA[2:]]),
                         np.concatenate([PB[:32], PB[64:]]), np.concatenate([XB[:1], XB[2:]]),
                         nx.MXGEMMINI(), osys.HW_FINAL)
    assert_bits_equal(z, drop, "an all-zero block adds nothing")


@pytest.mark.parametrize("fmt", ol.FORMATS)
def test_pick_is_exhaustive_nearest(fmt):
    V = (RNG.standard_t(4, (300, 20))).astype(F32)
    P, _ = ob.mxgemmini_quantize(V, fmt, 0, 32, "rne", 2.0 ** -23)
    T = ol.tables(P, fmt, 1, 20)
    assert np.array_equal(ol.pick(P, T, 1), brute.pick(P, T, 1))
    I = ol.pick(P, T, 1)
    assert_bits_equal(ol.lookup(I, T, 1), np.take_along_axis(T[np.arange(20) >> 1], I.T, axis=1).T, "lookup")


def test_fp64_accum_is_float64_dot():
    from fractions import Fraction
    A = RNG.standard_normal((64, 3)).astype(F32)
    B = RNG.standard_normal((64, 4)).astype(F32)
    PA, XA = ob.mxgemmini_quantize(A, "MXFP8_E4M3", 0)
    PB, XB = ob.mxgemmini_quantize(B, "MXFP8_E4M3", 0)
    Y = osys.fp64_accum(PA, XA, PB, XB)
    dA, dB = ob.dequantize(PA, XA), ob.dequantize(PB, XB)
    for i in range(3):
        for j in range(4):
            exact = sum(Fraction(float(x)) * Fraction(float(y)) for x, y in zip(dA[:, i], dB[:, j]))
            assert Y[i, j] == F32(float(exact))                                  # products of codes: exact sums


def test_scale_mxquant_properties():
    amax = np.concatenate([_random_finite_f32(20000, -140, 127), np.array([0.0, 1e-39, 2.0 ** -23], F32)])
    amax = np.abs(amax)
    X = nx.scale_mxquant(amax, 1e-38)
    ex = np.frexp(np.maximum(amax, F32(1e-38)))[1] - 1
    band = nx.log2_f32(np.maximum(amax, F32(1e-38))) == ex + 1
    want = np.maximum(np.ldexp(np.ones_like(amax), np.where(band, ex + 1, ex)), F32(1e-38)).astype(F32)
    assert_bits_equal(X, want, "mxquant scale")
    H = nx.scale_mxquant(amax, 2.0 ** -23)
    assert (H >= F32(2.0 ** -23)).all()


def test_compose_layout_invariants():
    """Shapes, the zero-padded last block, P * expand(X) == dequantize, FP32 pass-through (X = 1, P = V), and
    step 2 applied to V / X per block."""
    V = (RNG.standard_normal((5, 70, 3)) * 3).astype(F32)
    V[0, 64:, 0] = 100.0                                                    # the short last block's own amax
    P, X = ob.compose(V, lambda a: nx.scale_mxquant(a), None, axis=1, block_size=32)
    assert P.shape == V.shape and X.shape == (5, 3, 3)
    amax_last = np.abs(V[:, 64:, :]).max(axis=1)
    assert_bits_equal(X[:, 2, :], nx.scale_mxquant(amax_last), "last block scaled by its own 6 rows")
    Xe = np.repeat(X, 32, axis=1)[:, :70, :]
    assert_bits_equal(P, (V / Xe).astype(F32), "P = V / X without a step 2")
    assert_bits_equal(ob.dequantize(P, X, axis=1), (P * Xe).astype(F32), "dequantize = P * expand(X)")
    P1, X1 = ob.mxgemmini_quantize(V[0], None, 0)
    assert_bits_equal(P1, V[0], "FP32 pass-through codes") and (X1 == 1).all()
    P2, X2 = ob.mxquant_quantize(V[0], "MXFP8_E4M3", 0)
    Xe2 = np.repeat(X2, 32, axis=0)[:70]
    assert_bits_equal(P2, nx.float_em((V[0] / Xe2).astype(F32), 4, 3, "ties_away", "qtorch"), "mxquant = qtorch(V/X)")


def test_scale_ocp_properties():
    """shared = floor(log2 amax) - emax as an exponent (E8M0): NaN above 127, clamped at -127; amax 0 reads
    the float32 minimum normal."""
    amax = np.abs(np.concatenate([_random_finite_f32(20000, -140, 127), np.array([0.0], F32)]))
    for emax in (8, 15, 2, 4):
        X = nx.scale_ocp(amax, emax)
        a = np.where(amax == 0, F32(2.0 ** -126), amax)
        ex = np.frexp(a)[1] - 1
        ex = np.where(nx.log2_f32(a) == ex + 1, ex + 1, ex) - emax
        want = np.where(ex > 127, np.nan, np.ldexp(np.ones_like(a, dtype=F64), np.maximum(ex, -127))).astype(F32)
        assert_bits_equal(X, want, f"scale_ocp emax={emax}")
        assert_bits_equal(nx.scale_ocp_below_top(amax, emax + 1), X, "below_top is emax - 1")
