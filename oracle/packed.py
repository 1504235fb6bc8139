"""Oracle packed wire formats: element-code bytes and E8M0 scale bytes of block-quantized tensors, and 4-bit LUT
indices two to a byte.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

The reference keeps codes and scales as float32 tensors; these byte forms have no counterpart there.  They
follow the OCP Microscaling Formats (MX) v1.0 specification: an element code is sign | e exponent bits |
m mantissa bits with bias 2^(e-1) - 1 (subnormal when the exponent field is 0), which is the numbering of the
reference's element codes on every finite value (mxq/lut/formats.py:87-99 decodes code c the same way); E5M2
keeps IEEE Inf and NaN, E4M3's only special is NaN (S.1111.111), FP6 and FP4 have none.  A scale is E8M0:
2^k is the byte k + 127 for k in [-127, 127], NaN is 0xFF.

Method: table lookup, not bit manipulation.  `code_table` enumerates every code's value from the formula
above; `encode` searches a value's float32 bit pattern in that table, sorted.

Pins (tests/test_oracle_packed.py): the reference's own decode tables for E4M3, E5M2, E3M2, E2M3 written by
the reference (tests/golden/lut_*.npz; every code but E4M3's 0x7F/0xFF, which MX-Gemmini's decoders read as
±480 and OCP as NaN); torch's float8_e4m3fn and float8_e5m2 casts of every value; the OCP spec's FP4 value
list and each format's max_norm in mxq/element_quant/formats.py.
"""
import math

import numpy as np

F32 = np.float32
FORMATS = {"MXFP8_E4M3": (4, 3), "MXFP8_E5M2": (5, 2), "MXFP6_E3M2": (3, 2), "MXFP6_E2M3": (2, 3),
           "MXFP4": (2, 1)}
ERR_CODE, ERR_SCALE = 1, 2


def code_table(e, m):
    """float32 value of each code 0 .. 2^(1 + e + m) - 1."""
    bias = (1 << (e - 1)) - 1
    vals = []
    for c in range(1 << (1 + e + m)):
        s, ex, man = (c >> (e + m)) & 1, (c >> m) & ((1 << e) - 1), c & ((1 << m) - 1)
        if (e, m) == (5, 2) and ex == 31:
            v = math.nan if man else math.inf
        elif (e, m) == (4, 3) and ex == 15 and man == 7:
            v = math.nan
        elif ex == 0:
            v = man * 2.0 ** (1 - bias - m)
        else:
            v = (1.0 + man / (1 << m)) * 2.0 ** (ex - bias)
        vals.append(-v if s else v)
    return np.array(vals, dtype=F32)


def _sorted_table(e, m):
    """(bit patterns of the finite and infinite values, ascending; their codes)."""
    table = code_table(e, m)
    keep = ~np.isnan(table)
    bits = table.view(np.uint32)[keep]
    codes = np.arange(table.size)[keep]
    order = np.argsort(bits, kind="stable")
    return bits[order], codes[order]


def encode(q, e, m):
    """float32 values -> (uint8 codes, ok): ok is False where a value is not one of the format's."""
    q = np.asarray(q, dtype=F32)
    bits, codes_of = _sorted_table(e, m)
    u = q.view(np.uint32)
    at = np.clip(np.searchsorted(bits, u), 0, bits.size - 1)
    found = bits[at] == u
    codes = np.where(found, codes_of[at], 0).astype(np.uint8)
    ok = found.copy()
    nan = np.isnan(q)
    if (e, m) in ((4, 3), (5, 2)):                    # the NaN code, with the value's sign
        codes = np.where(nan, ((u >> 31) << (e + m)) | 0x7F, codes).astype(np.uint8)
        ok |= nan
    return codes, ok


def decode(codes, e, m):
    return code_table(e, m)[np.asarray(codes, dtype=np.int64)]


def e8m0_encode(x, zero_block):
    """Block scales -> (uint8 bytes, ok).  A scale E8M0 lacks is 0 (2^-127) for an all-zero block, else not ok."""
    x = np.asarray(x, dtype=F32)
    zero_block = np.broadcast_to(np.asarray(zero_block, dtype=bool), x.shape)
    x64 = x.astype(np.float64)
    fr, ex = np.frexp(np.where(np.isfinite(x64) & (x64 > 0), x64, 0.0))
    k = ex.astype(np.int64) - 1
    pow2 = (fr == 0.5) & (k >= -127) & (k <= 127)
    nan = np.isnan(x)
    out = np.where(nan, 0xFF, np.where(pow2, k + 127, 0)).astype(np.uint8)
    ok = nan | pow2 | zero_block
    return out, ok


def e8m0_decode(b):
    b = np.asarray(b, dtype=np.int64)
    x = np.ldexp(np.ones(b.shape, dtype=F32), np.minimum(b, 254) - 127).astype(F32)
    return np.where(b == 0xFF, F32(np.nan), x)


def pack(P, X, fmt, axis=0, block_size=32):
    """Float32 codes P and scales X (block.quantize's outputs) -> (code bytes, scale bytes, error bits)."""
    e, m = FORMATS[fmt]
    P = np.asarray(P, dtype=F32)
    X = np.asarray(X, dtype=F32)
    codes, ok = encode(P, e, m)
    Pt = np.moveaxis(P, axis, -1)
    n = Pt.shape[-1]
    nb = -(-n // block_size)
    pad = np.zeros(Pt.shape[:-1] + (nb * block_size - n,), dtype=F32)
    blocks = np.concatenate([Pt, pad], axis=-1).reshape(Pt.shape[:-1] + (nb, block_size))
    zero = np.moveaxis((blocks.view(np.uint32) & 0x7FFFFFFF).max(axis=-1) == 0, -1, axis)
    scales, sok = e8m0_encode(X, zero)
    err = (0 if ok.all() else ERR_CODE) | (0 if sok.all() else ERR_SCALE)
    return codes, scales, err


def unpack(codes, scales, fmt):
    e, m = FORMATS[fmt]
    return decode(codes, e, m), e8m0_decode(scales)


def pack_indices(I):
    """K x n indices in [0, 16) -> K x ceil(n / 2) bytes: column j in the low nibble (j even), j + 1 high."""
    I = np.asarray(I, dtype=np.int64)
    K, n = I.shape
    if n % 2:
        I = np.concatenate([I, np.zeros((K, 1), dtype=np.int64)], axis=1)
    return (I[:, 0::2] | (I[:, 1::2] << 4)).astype(np.uint8)


def unpack_indices(B, n):
    B = np.asarray(B, dtype=np.int64)
    both = np.stack([B & 0xF, B >> 4], axis=-1).reshape(B.shape[0], -1)
    return both[:, :n]
