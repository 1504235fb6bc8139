"""Oracle block quantization: compose, dequantize and the named quantizers.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

Pins: layout invariants (shapes, zero padding, P * expand(X) == dequantize, FP32 pass-through gives X = 1)
and the numerics pins of oracle/numerics.py; block.ocp's `no_clip` placement by fixtures the reference wrote.
"""
import math

import numpy as np

from . import numerics as nx

F32 = np.float32
BLOCK = 32


def _to_blocks(V, axis, block_size):
    """mxq/block/_driver.py:23-32: move the axis last, zero-pad to a multiple of block_size, split."""
    if not -V.ndim <= axis < V.ndim:
        raise IndexError(f"axis {axis} out of range for {V.ndim}-D tensor")
    axis = axis % V.ndim
    Vt = np.moveaxis(V, axis, -1)
    n = Vt.shape[-1]
    pad = (-n) % block_size
    if pad:
        Vt = np.concatenate([Vt, np.zeros(Vt.shape[:-1] + (pad,), dtype=Vt.dtype)], axis=-1)
    return Vt.reshape(*Vt.shape[:-1], -1, block_size), axis, n


def compose(V, scale, elem, axis=0, block_size=BLOCK):
    """mxq/block/_driver.py:45-66.  scale(amax) and elem(z) are numpy callables or None."""
    V = np.asarray(V).astype(F32)
    data, axis, n = _to_blocks(V, axis, block_size)
    if scale is None:
        X = np.ones(data.shape[:-1] + (1,), dtype=F32)
        z = data
    else:
        with np.errstate(all="ignore"):
            amax = np.abs(data).max(axis=-1, keepdims=True) if data.shape[-1] else np.zeros(data.shape[:-1] + (1,), F32)
            X = scale(amax).astype(F32)
            z = (data / X).astype(F32)
    P = z.copy() if elem is None else elem(z)
    P = np.moveaxis(P.reshape(*P.shape[:-2], -1)[..., :n], -1, axis)
    X = np.moveaxis(X[..., 0], -1, axis)
    return np.ascontiguousarray(P, dtype=F32), np.ascontiguousarray(X, dtype=F32)


def dequantize(P, X, axis=0, block_size=BLOCK):
    """mxq/block/_driver.py:69-72."""
    axis = axis % P.ndim
    Xe = np.repeat(X, block_size, axis=axis)
    Xe = np.take(Xe, np.arange(P.shape[axis]), axis=axis)
    with np.errstate(all="ignore"):
        return (P * Xe).astype(F32)


def _fmt(fmt):
    if fmt is None:
        return None
    key = fmt.strip().upper()
    return None if key == "FP32" else key


def mxquant_quantize(V, fmt, axis=0, block_size=BLOCK):
    """mxq/block/mxquant.py:26-32."""
    f = _fmt(fmt)
    if f is None:
        return compose(V, None, None, axis, block_size)
    e, m = nx.FORMATS[f][:2]
    return compose(V, nx.scale_mxquant, lambda z: nx.float_em(nx.canon_nan(z), e, m), axis, block_size)


def mxgemmini_quantize(V, fmt, axis=0, block_size=BLOCK, rounding_mode="ties_away",
                       scale_floor=nx.MXQUANT_FLOOR, via=None):
    """mxq/block/mxgemmini.py:37-59."""
    f = _fmt(fmt)
    if f is None:
        return compose(V, None, None, axis, block_size)
    e, m = nx.FORMATS[f][:2]

    def elem(z):
        if via is not None:
            z = nx.float_em(z, via[0], via[1], rounding_mode, "ieee")
        return nx.float_em(z, e, m, rounding_mode, "ocp")

    return compose(V, lambda a: nx.scale_mxquant(a, scale_floor), elem, axis, block_size)


def ocp_quantize(V, fmt, axis=0, block_size=BLOCK, rounding_mode="even", scale_bits=8, placement="top",
                 draws=None):
    """mxq/block/ocp.py:35-49.  draws = (u_amax, u) for rounding_mode "dither": the uniforms rand_like drew for
    the block maxima (no_clip only, else None) and for the blocked tensor (..., nblocks, block_size), flat in
    those tensors' order."""
    f = _fmt(fmt)
    if f is None:
        return compose(V, None, None, axis, block_size)
    u_amax, u = draws if draws is not None else (None, None)
    emax = nx.FORMATS[f][2]
    if placement == "top":
        scale = lambda a: nx.scale_ocp(a, emax, scale_bits)                       # noqa: E731
    elif placement == "below_top":
        scale = lambda a: nx.scale_ocp_below_top(a, emax, scale_bits)             # noqa: E731
    else:
        scale = lambda a: nx.scale_ocp_no_clip(a, f, rounding_mode, scale_bits, u_amax)   # noqa: E731
    return compose(V, scale, lambda z: nx.microsoft_fmt(z, f, rounding_mode, u), axis, block_size)


def nblocks(n, block_size=BLOCK):
    return math.ceil(n / block_size)
