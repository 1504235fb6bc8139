"""Oracle numerics: rounding, float_em grids, the microxcaling element step, scale factors and arith.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

Each function restates one reference function in numpy, in the reference's operation order, on float32
(or float64 where the reference uses float64).  numpy float32 arithmetic, floor, trunc, rint, frexp, ldexp
and remainder round exactly as torch's CPU kernels do.  Two torch calls have no exact numpy twin and are
restated:
  * torch.log2 on float32, which the reference only ever floors: taken as the correctly rounded log2
    (float64 log2 rounded to float32); its floor is pinned against torch.log2's, with the round-up band
    below every power of two (tests/test_oracle_pins.py).
  * torch.exp2 / torch.pow(2, .) of integer-valued floats: exact powers of two, via ldexp; pinned against torch.

Pins: rounding.* and bf16 against torch casts; float_em ieee/ocp against brute-force nearest-value search over
the enumerated grid and torch float8 casts; qtorch by its grid properties; exact_add, truncate, flush and
saturate against exact rationals (oracle/brute.py); microsoft "even", ocp_no_clip by fixtures the reference
wrote (tests/golden/); all in tests/test_oracle_pins.py and tests/test_oracle_golden.py.
"""
import numpy as np

F32, F64, I64 = np.float32, np.float64, np.int64
MODES = ("ties_away", "rne", "truncate")
GRIDS = ("qtorch", "ieee", "ocp")
_U32 = 0xFFFFFFFF

# (name) -> (e, m, emax, max_norm, microxcaling (ebits, mbits, emax, max_norm))
# mxq/element_quant/formats.py:23-29 and mxq/microxcaling/formats.py:61-125
FORMATS = {
    "MXFP8_E4M3": (4, 3, 8, 448.0, (4, 5, 8, 448.0)),
    "MXFP8_E5M2": (5, 2, 15, 57344.0, (5, 4, 15, 57344.0)),
    "MXFP6_E3M2": (3, 2, 4, 28.0, (3, 4, 4, 28.0)),
    "MXFP6_E2M3": (2, 3, 2, 7.5, (2, 5, 2, 7.5)),
    "MXFP4": (2, 1, 2, 6.0, (2, 3, 2, 6.0)),
}


def f32(x):
    return np.asarray(x, dtype=F32)


def bits_of(x):
    """float32 array -> int64 array holding the uint32 pattern (mxq/rounding/__init__.py:82)."""
    return f32(x).view(np.int32).astype(I64) & _U32


def from_bits(q):
    """int64 array of uint32 patterns -> float32 (mxq/rounding/__init__.py:84)."""
    q = np.asarray(q, dtype=I64)
    q = np.where(q >= 1 << 31, q - (1 << 32), q).astype(np.int32)
    return q.view(F32)


def canon_nan(x):
    """NaN payloads are outside the spec: a NaN made by arithmetic becomes the quiet NaN 0x7FC00000 before a
    rounding that reads its bits (the qtorch grid)."""
    x = f32(x)
    return np.where(np.isnan(x), np.array(0x7FC00000, dtype=np.uint32).view(F32), x).astype(F32)


def tsign(x):
    """torch.sign: (0 < x) - (x < 0); 0 for +-0 and NaN."""
    return ((x > 0).astype(x.dtype) - (x < 0).astype(x.dtype))


def log2_f32(x):
    """torch.log2 on float32 (correctly rounded): float64 log2 rounded once to float32."""
    x = f32(x)
    with np.errstate(divide="ignore", invalid="ignore"):
        return np.log2(x.astype(F64)).astype(F32)


def exp2_int(t, dtype=F32):
    """torch.exp2 / pow(2, t) of integer-valued floats (NaN and +-inf included), exact."""
    t = np.asarray(t, dtype=dtype)
    out = np.empty_like(t)
    fin = np.isfinite(t)
    out[~fin] = np.exp2(t[~fin])                       # inf -> inf, -inf -> 0, nan -> nan
    ti = np.clip(np.where(fin, t, 0), -2000, 2000).astype(np.int64)
    out[fin] = np.ldexp(np.ones_like(t)[fin], ti[fin])
    return out


# ------------------------------------------------------------------------------------------- rounding
def round_bits(bits, keep, mode):
    """mxq/rounding/__init__.py:34-55 (+ rne.py:6-8, ties_away.py:5-6, truncate.py:5-6)."""
    bits = np.asarray(bits, dtype=I64)
    keep = np.asarray(keep, dtype=I64)
    drop = 23 - keep
    mask = (np.int64(1) << drop) - 1
    half = np.int64(1) << (drop - 1)
    if mode == "ties_away":
        r = (bits + half) & ~mask
    elif mode == "rne":
        r = (bits + half - 1 + ((bits >> drop) & 1)) & ~mask
    elif mode == "truncate":
        r = bits & ~mask
    else:
        raise ValueError(mode)
    return r & _U32


def round_int(k, mode):
    """mxq/rounding/rne.py:11-12, ties_away.py:9-10, truncate.py:9-10 (in k's own dtype)."""
    k = np.asarray(k)
    if mode == "rne":
        return np.rint(k)
    if mode == "ties_away":
        return tsign(k) * np.floor(np.abs(k) + k.dtype.type(0.5))
    if mode == "truncate":
        return np.trunc(k)
    raise ValueError(mode)


def bf16(x):
    """mxq/rounding/__init__.py:64-85."""
    x32 = f32(x)
    q = from_bits(round_bits(bits_of(x32), 7, "rne"))
    return np.where(np.isnan(x32), x32, q)


# ------------------------------------------------------------------------------------------- float_em
def bias(e):
    return (1 << (e - 1)) - 1


def float_em(z, e, m, rounding_mode="ties_away", grid="qtorch"):
    """mxq/element_quant/float_em.py:39-50."""
    z = np.asarray(z)
    if (e, m) == (8, 23):
        if z.dtype == F64:
            return _ieee(z, 8, 23, rounding_mode)
        return f32(z).copy()
    return {"qtorch": _qtorch, "ieee": _ieee, "ocp": _ocp}[grid](z, e, m, rounding_mode)


def _qtorch(z, e, m, rounding_mode):
    """mxq/element_quant/float_em.py:53-73."""
    z32 = f32(z)
    bits = bits_of(z32)
    q = round_bits(bits, m, rounding_mode)
    L = bias(e)
    min_store, max_store = 127 - L, 127 + L
    exp_store = (q >> 23) & 0xFF
    sign = bits & 0x80000000
    max_num = sign | (max_store << 23) | (0x007FFFFF & ~((1 << (23 - m)) - 1))
    min_num = sign | (min_store << 23)
    middle = (min_store - 1) << 23
    q_mag = q & 0x7FFFFFFF
    q = np.where(exp_store > max_store, max_num, q)
    below = exp_store < min_store
    q = np.where(below & (q_mag > middle), min_num, q)
    q = np.where(below & ~(q_mag > middle), 0, q)
    return from_bits(q)


def _ieee(z, e, m, rounding_mode):
    """mxq/element_quant/float_em.py:76-99."""
    x = np.asarray(z)
    x = x if x.dtype == F64 else x.astype(F64 if e == 8 else F32)
    dt = x.dtype.type
    b = bias(e)
    emin, emax = 1 - b, b
    ax = np.abs(x)
    finite_nz = np.isfinite(x) & (ax != 0)
    _, ex = np.frexp(np.where(finite_nz, ax, np.ones_like(ax)))
    E = (ex - 1).astype(x.dtype)
    step = exp2_int(np.maximum(E, dt(emin)) - dt(m), x.dtype)
    with np.errstate(invalid="ignore", over="ignore"):
        k = round_int(ax / step, rounding_mode)
        val = k * step
    val = np.where(val >= dt(2.0 ** (emax + 1)), dt(np.inf), val)
    out = np.where(finite_nz, np.copysign(val, x), x)
    if e < 8:
        out = np.where(finite_nz & (val == 0), np.zeros_like(out), out)
    return out.astype(F32)


def _ocp(z, e, m, rounding_mode):
    """mxq/element_quant/float_em.py:102-123."""
    f = next((v for v in FORMATS.values() if (v[0], v[1]) == (e, m)), None)
    if f is None:
        raise ValueError(f"grid='ocp' is defined only for the OCP element formats, not (e={e}, m={m})")
    x = np.asarray(z)
    x = x if x.dtype == F64 else x.astype(F32)
    dt = x.dtype.type
    emin = 1 - bias(e)
    ax = np.abs(x)
    finite_nz = np.isfinite(x) & (ax != 0)
    _, ex = np.frexp(np.where(finite_nz, ax, np.ones_like(ax)))
    E = (ex - 1).astype(x.dtype)
    step = exp2_int(np.maximum(E, dt(emin)) - dt(m), x.dtype)
    with np.errstate(invalid="ignore", over="ignore"):
        val = round_int(ax / step, rounding_mode) * step
    val = np.minimum(val, dt(f[3]))
    out = np.where(finite_nz, np.copysign(val, x), x)
    out = np.where(x == 0, np.zeros_like(out), out)
    return out.astype(F32)


# --------------------------------------------------------------------------- microxcaling element step
def _ms_round_mantissa(A, mode, u=None):
    """mxq/microxcaling/elemwise.py:29-60 (names: nearest = ties_away, even = rne, floor = truncate).  "dither"
    (:41-43) rounds with u, the uniforms torch.rand_like drew for A (float32, A's shape)."""
    if mode == "dither":
        return tsign(A) * np.floor(np.abs(A) + f32(u).reshape(A.shape))
    if mode == "floor":
        return tsign(A) * np.floor(np.abs(A))
    if mode == "nearest":
        return tsign(A) * np.floor(np.abs(A) + F32(0.5))
    if mode == "even":
        absA = np.abs(A)
        maskA = (np.remainder(absA - F32(0.5), F32(2)) == np.zeros_like(A)).astype(A.dtype)
        return tsign(A) * (np.floor(absA + F32(0.5)) - maskA)
    raise ValueError(mode)


def microsoft(A, ebits, mbits, max_norm, mode="even", saturate_normals=True, u=None):
    """mxq/microxcaling/elemwise.py:63-151 `_quantize_elemwise_core` (float formats, allow_denorm=True) on float32;
    u: the draws for mode "dither"."""
    A = f32(A)
    with np.errstate(all="ignore"):
        private_exp = np.floor(log2_f32(np.abs(A) + (A == 0).astype(F32)))
        min_exp = -(2 ** (ebits - 1)) + 2
        private_exp = np.maximum(private_exp, F32(min_exp))          # torch clip(min): NaN stays NaN
        p2 = exp2_int(private_exp)
        out = A / p2 * F32(2 ** (mbits - 2))
        out = _ms_round_mantissa(out, mode, u)
        out = out / F32(2 ** (mbits - 2)) * p2
        if saturate_normals:
            out = np.clip(out, F32(-max_norm), F32(max_norm))
        else:
            out = np.where(np.abs(out) > F32(max_norm), tsign(out) * F32(np.inf), out)
    out = np.where(A == np.inf, F32(np.inf), out)
    out = np.where(A == -np.inf, F32(-np.inf), out)
    return out.astype(F32)


def microsoft_fmt(z, fmt, rounding_mode="even", u=None):
    """mxq/element_quant/microsoft.py:18-23."""
    eb, mb, _, mn = FORMATS[fmt][4]
    return microsoft(z, eb, mb, mn, rounding_mode, True, u)


# ---------------------------------------------------------------------------------------- scale factors
MXQUANT_FLOOR = 1e-38
HARDWARE_FLOOR = 2.0 ** -23
FP32_MIN_NORMAL = 2.0 ** -126


def scale_mxquant(amax, floor=MXQUANT_FLOOR):
    """mxq/scale_factor.py:40-44 (torch clamp keeps NaN; the Python floor becomes a float32 scalar)."""
    amax = f32(amax)
    fl = F32(floor)
    with np.errstate(all="ignore"):
        a = np.where(np.isnan(amax), amax, np.maximum(amax, fl))
        sc = exp2_int(np.floor(log2_f32(a)))
        return np.where(np.isnan(sc), sc, np.maximum(sc, fl)).astype(F32)


def scale_ocp(amax, emax, scale_bits=8):
    """mxq/scale_factor.py:47-59."""
    amax = f32(amax)
    with np.errstate(all="ignore"):
        shared = np.floor(log2_f32(amax + F32(FP32_MIN_NORMAL) * (amax == 0).astype(F32)))
        shared = shared - F32(emax)
        scale_emax = 2 ** (scale_bits - 1) - 1
        shared = np.where(shared > scale_emax, F32(np.nan), shared)
        shared = np.where(shared < -scale_emax, F32(-scale_emax), shared)
        return exp2_int(shared)


def scale_ocp_below_top(amax, emax, scale_bits=8):
    """mxq/scale_factor.py:62-65."""
    return scale_ocp(amax, emax - 1, scale_bits)


def scale_ocp_no_clip(amax, fmt, rounding_mode="even", scale_bits=8, u=None):
    """mxq/scale_factor.py:68-81 (u: the draws for rounding_mode "dither", one per maximum)."""
    e, m, emax, mn, (eb, mb, _, _) = FORMATS[fmt]
    X = scale_ocp(amax, emax, scale_bits)
    with np.errstate(all="ignore"):
        rounded = microsoft(f32(amax) / X, eb, mb, mn, rounding_mode, saturate_normals=False, u=u)
        return np.where(np.isinf(rounded), X * F32(2), X).astype(F32)


# ------------------------------------------------------------------------------------------------ arith
def fits_float32(e, m):
    """mxq/arith.py:21-30."""
    return 2 ** e - 1 + m <= 24


def two_sum(a, b):
    """mxq/arith.py:33-38."""
    with np.errstate(all="ignore"):
        s = a + b
        bb = s - a
        return s, (a - (s - bb)) + (b - bb)


def round_pair(s, t, e, m):
    """mxq/arith.py:41-65."""
    b = bias(e)
    emin, emax = 1 - b, b
    ax = np.abs(s)
    finite_nz = np.isfinite(s) & (ax != 0)
    _, ex = np.frexp(np.where(finite_nz, ax, np.ones_like(ax)))
    E = (ex - 1).astype(F32)
    step = exp2_int(np.maximum(E, F32(emin)) - F32(m))
    with np.errstate(all="ignore"):
        k = ax / step
        kf = np.floor(k)
        tie = (k - kf) == F32(0.5)
        up = (tsign(s) * t) > 0
        k_out = np.where(tie & (t != 0), np.where(up, kf + F32(1), kf), np.rint(k))
        val = k_out * step
    val = np.where(val >= F32(2.0 ** (emax + 1)), F32(np.inf), val)
    out = np.where(finite_nz, np.copysign(val, s), s)
    return np.where(finite_nz & (val == 0), np.zeros_like(out), out).astype(F32)


def exact_add(a, b, e, m, rounding_mode="rne", grid="ieee"):
    """mxq/arith.py:68-103."""
    a, b = f32(a), f32(b)
    if rounding_mode == "rne" and grid == "ieee" and fits_float32(e, m):
        with np.errstate(all="ignore"):
            q = float_em(a + b, e, m, "rne", "ieee")
        return np.where(a == 0, b, np.where(b == 0, a, q)).astype(F32)
    if rounding_mode == "rne" and grid == "ieee" and e <= 7:
        q = round_pair(*two_sum(a, b), e, m)
        return np.where(a == 0, b, np.where(b == 0, a, q)).astype(F32)
    a64, b64 = a.astype(F64), b.astype(F64)
    with np.errstate(all="ignore"):
        q = float_em(a64 + b64, e, m, rounding_mode, grid)
    return np.where(a64 == 0, b, np.where(b64 == 0, a, q)).astype(F32)


def truncate_significand(x, m):
    """mxq/arith.py:106-117."""
    x = f32(x)
    ax = np.abs(x)
    nz = np.isfinite(x) & (ax != 0)
    mant, ex = np.frexp(np.where(nz, ax, np.ones_like(ax)))
    k = round_int(mant * F32(1 << (m + 1)), "truncate")
    t = np.ldexp(k / F32(1 << m), ex - 1).astype(F32)
    return np.where(nz, np.copysign(t, x), x).astype(F32)


def flush_product(x, floor_exp):
    """mxq/arith.py:120-124 (the Python threshold compares as a float32 scalar)."""
    x = f32(x)
    return np.where(np.abs(x) < F32(2.0 ** floor_exp), F32(0), x).astype(F32)


def saturate(x, limit, value):
    """mxq/arith.py:127-137."""
    x = f32(x)
    ax = np.abs(x)
    with np.errstate(all="ignore"):
        return (tsign(x) * np.where(ax > F32(limit), F32(value), ax)).astype(F32)


# ------------------------------------------------------------------------------------------ Arithmetics
PROD_FLOOR = -16


def saturation(prod_e, prod_m):
    """mxq/matmul/_arithmetic.py:88-102."""
    b = bias(prod_e)
    fp8 = (prod_e, prod_m) == (4, 3)
    limit = 2.0 ** (b + 1 if fp8 else b) * (1 + ((2 ** prod_m - 2) if fp8 else (2 ** prod_m - 1)) / 2 ** prod_m)
    value = 2.0 ** (b + 1) * (1 + (2 ** prod_m - 2) / 2 ** prod_m)
    if value > float(np.finfo(np.float32).max):
        value = float("inf")
    return limit, value


def unsigned_zero(x):
    """mxq/matmul/_arithmetic.py:105-108."""
    return np.where(x == 0, np.zeros_like(x), x)


class MXGEMMINI:
    """mxq/matmul/_arithmetic.py:111-134."""

    def __init__(self, prod_e=4, prod_m=3, prod_floor=PROD_FLOOR):
        self.prod_e, self.prod_m, self.prod_floor = prod_e, prod_m, prod_floor
        self.limit, self.value = saturation(prod_e, prod_m)
        self.name = f"mxgemmini(prod=e{prod_e}m{prod_m})"

    def rne(self, x, e, m):
        return bf16(x) if (e, m) == (8, 7) else float_em(x, e, m, "rne", "ieee")

    def lane(self, x, e, m):
        return unsigned_zero(self.rne(x, e, m))

    def product(self, a, b):
        with np.errstate(all="ignore"):
            t = truncate_significand(f32(a) * f32(b), self.prod_m)
        if self.prod_floor is not None:
            t = flush_product(t, self.prod_floor)
        return saturate(t, self.limit, self.value)

    def acc_add(self, S, p, e, m):
        return exact_add(self.lane(S, e, m), self.lane(p, e, m), e, m)

    def tile_add(self, C, tile):
        return exact_add(self.lane(C, 8, 7), self.lane(tile, 8, 7), 8, 7)


class MXQUANT:
    """mxq/matmul/_arithmetic.py:64-73."""

    def __init__(self, prod_e, prod_m):
        self.prod_e, self.prod_m = prod_e, prod_m
        self.name = f"mxquant(prod=e{prod_e}m{prod_m})"

    @staticmethod
    def q(x, e, m):
        return float_em(x, e, m, "ties_away", "qtorch")

    def product(self, a, b):
        with np.errstate(all="ignore"):
            return self.q(canon_nan(f32(a) * f32(b)), self.prod_e, self.prod_m)

    def acc_add(self, S, p, e, m):
        with np.errstate(all="ignore"):
            return self.q(canon_nan(f32(S) + f32(p)), e, m)

    def tile_add(self, C, tile):
        with np.errstate(all="ignore"):
            return (f32(C) + f32(tile)).astype(F32)
