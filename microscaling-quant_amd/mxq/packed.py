"""Packed wire formats of block-quantized tensors.  Not in the reference, whose codes and scales are float32
tensors: this is what the hardware moves, a quarter of those bytes (include/mxq_hip.h declares the kernels).

    codes, scales = quantize(V, fmt, method="mxgemmini", axis=0, block_size=32, **options)   one pass, bytes out
    codes, scales = pack(P, X, fmt, axis=0, block_size=32)       float32 codes and scales -> bytes
    P, X = unpack(codes, scales, fmt, axis=0, block_size=32)      bytes -> float32 codes and scales
    V_hat = dequantize(codes, scales, fmt, axis=0, block_size=32) bytes -> P * expand(X), float32
    I4 = pick(P, T, group=G)                                      lut.pick's indices, two 4-bit nibbles a byte
    P_lut = lookup(I4, T, group=G, n=n)                           lut.lookup of those

An element code is one byte in the OCP MX layout: sign | e exponent bits | m mantissa bits, bias 2^(e-1) - 1,
the numbering of the reference's element codes (mxq/lut/formats.py:87-99) on every finite value; E5M2 keeps
Inf and NaN, E4M3's NaN is S.1111.111, FP6 and FP4 have no specials.  Codes are shaped like P.  A scale is an
E8M0 byte: 2^k is k + 127 (k in [-127, 127]), NaN 0xFF; scales are shaped like X.  A block whose codes are all
zero has the value 0 under any scale, so its scale may be one E8M0 lacks (block.mxgemmini's 1e-38 floor) and
packs as 2^-127: unpack then reads 2^-127 there, and dequantize gives the same zeros.

`quantize` takes the quantizer `method` ("mxgemmini", "ocp" or "mxquant") and that quantizer's options with
its defaults; it writes exactly the bytes `pack` makes of that quantizer's (P, X).  mxquant's qtorch grid has
values below some formats' smallest subnormal: such a code raises ValueError, as does any code or scale with
no byte.  Checking reads back one error word (a host synchronisation); check=False skips it.

Nibbles: row k's byte j // 2 holds column j's index in its low nibble for even j, column j + 1's in its high
one (0 past n); tables of at most 16 entries.
"""
from typing import Tuple, Union

import torch

from . import _lib
from .block import _driver, mxgemmini, mxquant, ocp
from .element_quant.formats import Format, get
from .lut.kmeans import _check, _check_tables
from .lut.formats import SIZE
from .scale_factor import MXQUANT_FLOOR

__all__ = ["quantize", "pack", "unpack", "dequantize", "pick", "lookup", "METHODS"]

METHODS = ("mxgemmini", "ocp", "mxquant")


def _format(fmt: Union[str, Format]) -> Format:
    f = get(fmt)
    if f is None:
        raise ValueError("mxq.packed: FP32 has no byte format; name an MX element format")
    return f


def _check_err(err: torch.Tensor, who: str, f: Format) -> None:
    bits = int(err.item())
    if bits & 1:
        raise ValueError(f"mxq.packed.{who}: a code is not a {f.name} value (off its grid or range, or a special "
                         f"the format lacks)")
    if bits & 2:
        raise ValueError(f"mxq.packed.{who}: a block scale that is not a power of two in [2^-127, 2^127] (E8M0) "
                         f"belongs to a block with nonzero codes")


def _spec(f: Format, method: str, options: dict) -> _lib.BlockSpec:
    if method == "mxgemmini":
        allowed = {"rounding_mode": "ties_away", "scale_floor": MXQUANT_FLOOR, "via": None}
    elif method == "ocp":
        allowed = {"rounding_mode": "even", "scale_bits": 8, "placement": "top"}
    elif method == "mxquant":
        allowed = {}
    else:
        raise ValueError(f"mxq.packed.quantize: method must be one of {METHODS}, got {method!r}")
    unknown = set(options) - set(allowed)
    if unknown:
        raise TypeError(f"mxq.packed.quantize: {method} takes no option {sorted(unknown)[0]!r}")
    o = {**allowed, **options}
    if method == "mxgemmini":
        return mxgemmini.spec(f, o["rounding_mode"], o["scale_floor"], o["via"])
    if method == "ocp":
        if o["placement"] not in ocp.PLACEMENTS:
            raise ValueError(f"placement must be one of {ocp.PLACEMENTS}, got {o['placement']!r}")
        return ocp.spec(f, o["rounding_mode"], o["scale_bits"], o["placement"])
    return mxquant.spec(f)


def _shapes(shape, axis: int, block_size: int):
    outer, n, inner = _driver._view3(shape, axis)
    xshape = list(shape)
    xshape[axis] = -(-n // block_size)
    return outer, n, inner, xshape


def quantize(V: torch.Tensor, fmt: Union[str, Format], method: str = "mxgemmini", axis: int = 0,
             block_size: int = _driver.BLOCK, *, check: bool = True, **options) -> Tuple[torch.Tensor, torch.Tensor]:
    """Block-quantize V along `axis` straight to (code bytes, E8M0 scale bytes), uint8 on V's device."""
    f = _format(fmt)
    axis = _driver._axis(V, axis)
    spec = _spec(f, method, options)
    _driver._check_block(block_size)
    dev = _lib.compute_device(V)
    Vd = _lib.to_device(V.detach(), dev)
    if Vd.dtype not in _driver._NATIVE:
        Vd = Vd.to(torch.float32)
    Vd = Vd.contiguous()
    outer, n, inner, xshape = _shapes(Vd.shape, axis, block_size)
    codes = torch.empty(Vd.shape, dtype=torch.uint8, device=dev)
    scales = torch.empty(xshape, dtype=torch.uint8, device=dev)
    err = torch.zeros(1, dtype=torch.int32, device=dev)
    with _lib.on(dev):
        _lib.run("mxq_block_quantize_packed", _lib.ptr(Vd), _driver._NATIVE[Vd.dtype], _lib.ptr(codes),
                 _lib.ptr(scales), _lib.ptr(err), outer, n, inner, block_size, spec, _lib.stream(dev))
    if check:
        _check_err(err, "quantize", f)
    return _lib.back(codes, V), _lib.back(scales, V)


def pack(P: torch.Tensor, X: torch.Tensor, fmt: Union[str, Format], axis: int = 0,
         block_size: int = _driver.BLOCK, *, check: bool = True) -> Tuple[torch.Tensor, torch.Tensor]:
    """float32 codes P and scales X of `fmt` (a block quantizer's outputs) -> (code bytes, scale bytes)."""
    f = _format(fmt)
    axis = _driver._axis(P, axis)
    _driver._check_block(block_size)
    outer, n, inner, xshape = _shapes(P.shape, axis, block_size)
    if list(X.shape) != xshape:
        raise ValueError(f"mxq.packed.pack: X has shape {tuple(X.shape)}, expected {tuple(xshape)}")
    dev = _lib.compute_device(P, X)
    Pd = _lib.to_device(P.detach(), dev).to(torch.float32).contiguous()
    Xd = _lib.to_device(X.detach(), dev).to(torch.float32).contiguous()
    codes = torch.empty(Pd.shape, dtype=torch.uint8, device=dev)
    scales = torch.empty(xshape, dtype=torch.uint8, device=dev)
    err = torch.zeros(1, dtype=torch.int32, device=dev)
    with _lib.on(dev):
        _lib.run("mxq_pack", _lib.ptr(Pd), _lib.ptr(Xd), _lib.ptr(codes), _lib.ptr(scales), _lib.ptr(err), outer, n,
                 inner, block_size, f.e, f.m, _lib.stream(dev))
    if check:
        _check_err(err, "pack", f)
    return _lib.back(codes, P), _lib.back(scales, P)


def _byte_operands(codes, scales, axis, block_size, who):
    if codes.dtype != torch.uint8 or scales.dtype != torch.uint8:
        raise ValueError(f"mxq.packed.{who}: codes and scales must be uint8, got {codes.dtype} and {scales.dtype}")
    axis = _driver._axis(codes, axis)
    _driver._check_block(block_size)
    outer, n, inner, xshape = _shapes(codes.shape, axis, block_size)
    if list(scales.shape) != xshape:
        raise ValueError(f"mxq.packed.{who}: scales have shape {tuple(scales.shape)}, expected {tuple(xshape)}")
    dev = _lib.compute_device(codes, scales)
    return (_lib.to_device(codes.detach(), dev).contiguous(), _lib.to_device(scales.detach(), dev).contiguous(),
            dev, outer, n, inner, xshape)


def unpack(codes: torch.Tensor, scales: torch.Tensor, fmt: Union[str, Format], axis: int = 0,
           block_size: int = _driver.BLOCK) -> Tuple[torch.Tensor, torch.Tensor]:
    """(code bytes, scale bytes) -> (P, X) float32."""
    f = _format(fmt)
    Cd, Sd, dev, outer, n, inner, xshape = _byte_operands(codes, scales, axis, block_size, "unpack")
    P = torch.empty(Cd.shape, dtype=torch.float32, device=dev)
    X = torch.empty(xshape, dtype=torch.float32, device=dev)
    with _lib.on(dev):
        _lib.run("mxq_unpack", _lib.ptr(Cd), _lib.ptr(Sd), _lib.ptr(P), _lib.ptr(X), outer, n, inner, block_size,
                 f.e, f.m, _lib.stream(dev))
    return _lib.back(P, codes), _lib.back(X, codes)


def dequantize(codes: torch.Tensor, scales: torch.Tensor, fmt: Union[str, Format], axis: int = 0,
               block_size: int = _driver.BLOCK) -> torch.Tensor:
    """(code bytes, scale bytes) -> P * expand(X), float32, bit-identical to block.dequantize of the float32
    codes and scales the bytes hold."""
    f = _format(fmt)
    Cd, Sd, dev, outer, n, inner, _ = _byte_operands(codes, scales, axis, block_size, "dequantize")
    out = torch.empty(Cd.shape, dtype=torch.float32, device=dev)
    with _lib.on(dev):
        _lib.run("mxq_dequantize_packed", _lib.ptr(Cd), _lib.ptr(Sd), _lib.ptr(out), outer, n, inner, block_size,
                 f.e, f.m, _lib.stream(dev))
    return _lib.back(out, codes)


def pick(P: torch.Tensor, T: torch.Tensor, *, group: int) -> torch.Tensor:
    """lut.pick's indices as nibbles: K x ceil(n / 2) uint8."""
    ng = _check(P, group)
    _check_tables(T, ng, P.shape[1], group, "pick")
    if T.shape[1] > SIZE:
        raise ValueError(f"mxq.packed.pick: a 4-bit index names at most {SIZE} entries, tables have {T.shape[1]}")
    dev = _lib.compute_device(P, T)
    Pd = _lib.to_device(P.detach(), dev).to(torch.float32).contiguous()
    Td = _lib.to_device(T.detach(), dev).to(torch.float32).contiguous()
    K, n = Pd.shape
    out = torch.empty((K, (n + 1) // 2), dtype=torch.uint8, device=dev)
    with _lib.on(dev):
        _lib.run("mxq_lut_pick_packed", _lib.ptr(Pd), K, n, group, _lib.ptr(Td), Td.shape[1], _lib.ptr(out),
                 _lib.stream(dev))
    return _lib.back(out, P)


def lookup(I4: torch.Tensor, T: torch.Tensor, *, group: int, n: int) -> torch.Tensor:
    """The table values the nibbles name: K x n float32 (n columns; the bytes hold ceil(n / 2))."""
    if I4.dtype != torch.uint8 or I4.ndim != 2 or I4.shape[1] != (n + 1) // 2:
        raise ValueError(f"mxq.packed.lookup: {n} columns need K x {(n + 1) // 2} uint8 nibbles, got "
                         f"{tuple(I4.shape)} {I4.dtype}")
    if not isinstance(group, int) or isinstance(group, bool) or group < 0:
        raise ValueError(f"mxq.lut: group {group!r} must be a non-negative integer")
    ng = (n + (1 << group) - 1) >> group
    _check_tables(T, ng, n, group, "lookup")
    dev = _lib.compute_device(I4, T)
    Id = _lib.to_device(I4.detach(), dev).contiguous()
    Td = _lib.to_device(T.detach(), dev).to(torch.float32).contiguous()
    width = Td.shape[1]
    if width > SIZE:
        raise ValueError(f"mxq.packed.lookup: a 4-bit index names at most {SIZE} entries, tables have {width}")
    both = torch.stack([Id & 0xF, Id >> 4], dim=-1).reshape(Id.shape[0], -1)[:, :n]
    if both.numel() and bool((both >= width).any()):
        raise IndexError(f"mxq.packed.lookup: index out of range for tables of width {width}")
    K = Id.shape[0]
    out = torch.empty((K, n), dtype=torch.float32, device=dev)
    with _lib.on(dev):
        _lib.run("mxq_lut_lookup_packed", _lib.ptr(Id), K, n, group, _lib.ptr(Td), width, _lib.ptr(out),
                 _lib.stream(dev))
    return _lib.back(out, I4)
