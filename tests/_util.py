"""Shared test helpers: seeded edge-value corpora, bit-exact comparison, the host numerics library."""
import ctypes

import numpy as np

F32 = np.float32


def bits(x):
    return np.asarray(x, dtype=F32).view(np.uint32)


def assert_bits_equal(got, want, what=""):
    """Bit-for-bit equality, with any NaN matching any NaN (payloads and NaN signs are not part of the spec)."""
    got = np.asarray(got)
    want = np.asarray(want)
    assert got.shape == want.shape, f"{what}: shape {got.shape} != {want.shape}"
    if got.dtype.kind == "f":
        gn, wn = np.isnan(got), np.isnan(want)
        bad = (gn != wn) | (~gn & (got.view(np.uint32 if got.dtype == F32 else np.uint64)
                                   != want.view(np.uint32 if want.dtype == F32 else np.uint64)))
    else:
        bad = got != want
    if bad.any():
        idx = np.argwhere(bad)[:8]
        rows = [f"  at {tuple(i)}: got {got[tuple(i)]!r} want {want[tuple(i)]!r}" for i in idx]
        raise AssertionError(f"{what}: {int(bad.sum())} of {bad.size} differ\n" + "\n".join(rows))


def special_f32():
    """Signed zeros, infinities, NaN, subnormal edges, powers of two and their neighbours, max values."""
    vals = [0.0, -0.0, np.inf, -np.inf, np.nan, 1.0, -1.0, 2.0, 0.5, 448.0, 480.0, 57344.0, 1e-38, 2.0 ** -126,
            2.0 ** -149, 3 * 2.0 ** -149, 2.0 ** -127, float(np.finfo(F32).max), 6.0, 7.5, 28.0, 1.75, 1.875]
    base = np.array(vals, dtype=F32)
    u = base.view(np.uint32)
    around = np.concatenate([u, u + 1, u - 1]).astype(np.uint32)
    pw = np.arange(-149, 128)
    p2 = np.ldexp(np.ones(pw.shape, dtype=F32), pw).astype(F32).view(np.uint32)
    p2n = np.concatenate([p2, p2 - 1, p2 + 1, p2 - 2, p2 - 40, p2 - 44, p2 - 45]).astype(np.uint32)
    allu = np.concatenate([around, p2n]).view(F32)
    return np.concatenate([allu, -allu]).astype(F32)


def random_f32(rng, n, lo=-40, hi=40):
    """Random float32 values with log-uniform magnitudes in [2^lo, 2^hi), random signs, plus random bit patterns."""
    mag = np.exp2(rng.uniform(lo, hi, n)).astype(F32)
    sgn = np.where(rng.random(n) < 0.5, -1, 1).astype(F32)
    raw = rng.integers(0, 2 ** 32, n // 4, dtype=np.uint64).astype(np.uint32).view(F32)
    return np.concatenate([mag * sgn, raw]).astype(F32)


def grid_values(e, m):
    """Every finite value of the ieee float(e, m) grid (both signs, one zero), as float64."""
    b = (1 << (e - 1)) - 1
    emin, emax = 1 - b, b
    vals = [k * 2.0 ** (emin - m) for k in range(1 << m)]                   # subnormals and 0
    for E in range(emin, emax + 1):
        vals += [(1 + j / (1 << m)) * 2.0 ** E for j in range(1 << m)]
    v = np.array(sorted(set(vals)), dtype=np.float64)
    return np.unique(np.concatenate([-v, v]))


class HostNumerics:
    """ctypes front of tests/host/numerics_host.cpp (the kernels' header built for the host)."""

    def __init__(self, lib):
        self.lib = lib

    @staticmethod
    def _p(a):
        return a.ctypes.data_as(ctypes.c_void_p)

    def _un(self, fn, x, *args, out_dtype=F32, in_dtype=F32):
        x = np.ascontiguousarray(x, dtype=in_dtype)
        out = np.empty(x.shape, dtype=out_dtype)
        getattr(self.lib, fn)(self._p(x), self._p(out), ctypes.c_int64(x.size), *args)
        return out

    def float_em(self, z, e, m, mode, grid, max_norm=0.0):
        z = np.asarray(z)
        if z.dtype == np.float64:
            return self._un("h_float_em64", z, e, m, mode, grid, ctypes.c_float(max_norm), in_dtype=np.float64)
        return self._un("h_float_em32", z, e, m, mode, grid, ctypes.c_float(max_norm))

    def ocp_grid_fast(self, z, e, m, mode, max_norm):
        return self._un("h_ocp_grid_fast", z, e, m, mode, ctypes.c_float(max_norm))

    def microsoft(self, z, ebits, mbits, max_norm, mode, sat=True):
        return self._un("h_microsoft", z, ebits, mbits, ctypes.c_float(max_norm), mode, int(sat))

    def bf16(self, x):
        return self._un("h_bf16", x)

    def div_inv(self, x):
        return self._un("h_div_inv", x)

    def floor_log2(self, x):
        return self._un("h_floor_log2", x, out_dtype=np.int32)

    def round_bits(self, b, keep, mode):
        return self._un("h_round_bits", b, keep, mode, out_dtype=np.int64, in_dtype=np.int64)

    def truncate(self, x, m):
        return self._un("h_truncate", x, m)

    def flush(self, x, thr):
        return self._un("h_flush", x, ctypes.c_float(thr))

    def saturate(self, x, limit, value):
        return self._un("h_saturate", x, ctypes.c_float(limit), ctypes.c_float(value))

    def exact_add(self, a, b, e, m, mode, grid, max_norm=0.0):
        a = np.ascontiguousarray(a, dtype=F32)
        b = np.ascontiguousarray(b, dtype=F32)
        out = np.empty(a.shape, dtype=F32)
        self.lib.h_exact_add(self._p(a), self._p(b), self._p(out), ctypes.c_int64(a.size), e, m, mode, grid,
                             ctypes.c_float(max_norm))
        return out

    def scale(self, a, spec):
        a = np.ascontiguousarray(a, dtype=F32)
        out = np.empty(a.shape, dtype=F32)
        self.lib.h_scale(self._p(a), self._p(out), ctypes.c_int64(a.size), ctypes.byref(spec))
        return out

    def block_quantize(self, V3, bs, spec):
        V3 = np.ascontiguousarray(V3, dtype=F32)
        outer, n, inner = V3.shape
        nb = -(-n // bs)
        P = np.empty(V3.shape, dtype=F32)
        X = np.empty((outer, nb, inner), dtype=F32)
        self.lib.h_block_quantize(self._p(V3), self._p(P), self._p(X), ctypes.c_int64(outer), ctypes.c_int64(n),
                                  ctypes.c_int64(inner), ctypes.c_int64(bs), ctypes.byref(spec))
        return P, X

    def mx_encode(self, q, e, m):
        q = np.ascontiguousarray(q, dtype=F32)
        codes = np.empty(q.shape, dtype=np.uint8)
        ok = np.empty(q.shape, dtype=np.uint8)
        self.lib.h_mx_encode(self._p(q), self._p(codes), self._p(ok), ctypes.c_int64(q.size), e, m)
        return codes, ok.astype(bool)

    def mx_decode(self, codes, e, m):
        return self._un("h_mx_decode", codes, e, m, in_dtype=np.uint8)

    def e8m0_encode(self, x, zero):
        x = np.ascontiguousarray(x, dtype=F32)
        z = np.ascontiguousarray(np.broadcast_to(zero, x.shape), dtype=np.uint8)
        b = np.empty(x.shape, dtype=np.uint8)
        ok = np.empty(x.shape, dtype=np.uint8)
        self.lib.h_e8m0_encode(self._p(x), self._p(z), self._p(b), self._p(ok), ctypes.c_int64(x.size))
        return b, ok.astype(bool)

    def e8m0_decode(self, b):
        return self._un("h_e8m0_decode", b, in_dtype=np.uint8)
