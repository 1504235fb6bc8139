"""Block quantization driver (mxq/block/_driver.py:1-72): `compose`, `dequantize` and the block layout helpers
`Blocks`, `to_blocks`, `codes_from_blocks`, `scales_from_blocks`.

Layout contract (MXQuant's mx_block32_quantize):
    quantize(V, axis) -> (P, X)   P: V's shape, the codes (float32)
                                  X: V's shape with axis of length ceil(len / block_size), the scales (float32)
    V_hat = P * expand(X), each scale repeated block_size times along axis (the last block zero-padded).

The named quantizers (block.mxquant, block.mxgemmini, block.ocp) hand `quantize_fused` a step-1/step-2 spec and
run as one gfx950 kernel: V is viewed as (outer, n, inner) with the block axis n in the middle, so no
transpose, padding or reassembly copy is made.  `compose` with arbitrary Python callables keeps the
reference's generic composition: the layout steps are torch views and copies on the tensor's device, the
callables run as given.
"""
from typing import Callable, NamedTuple, Optional, Tuple

import torch

from .. import _lib

BLOCK = 32

_NATIVE = {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2}


def _axis(V: torch.Tensor, axis: int) -> int:
    if not -V.ndim <= axis < V.ndim:
        raise IndexError(f"axis {axis} out of range for {V.ndim}-D tensor")
    return axis % V.ndim


def _check_block(block_size: int) -> None:
    if block_size == 0:
        raise ZeroDivisionError("integer division or modulo by zero")
    if block_size < 0:
        raise ValueError(f"block_size must be positive, got {block_size}")


class Blocks(NamedTuple):
    """A tensor cut into blocks along one axis (mxq/block/_driver.py:17-20).  `data` is (..., nblocks,
    block_size): the axis moved last and cut into rows of block_size, the last one zero-padded.  `axis`
    (non-negative) and `n` (the axis' length) are what undoing the cut needs."""
    data: torch.Tensor
    axis: int
    n: int


def to_blocks(V: torch.Tensor, axis: int, block_size: int) -> Blocks:
    """V's blocks along `axis` (mxq/block/_driver.py:23-32), in V's dtype and on its device.  IndexError for an
    axis out of range."""
    axis = _axis(V, axis)
    _check_block(block_size)
    last = V.movedim(axis, -1)
    n = last.shape[-1]
    nb = -(-n // block_size)
    data = last.new_zeros(*last.shape[:-1], nb * block_size)
    data[..., :n] = last
    return Blocks(data.view(*last.shape[:-1], nb, block_size), axis, n)


def codes_from_blocks(P: torch.Tensor, b: Blocks) -> torch.Tensor:
    """Codes in block form (..., nblocks, block_size) back in the layout of the tensor `b` was cut from, the
    padding dropped, contiguous (mxq/block/_driver.py:35-37)."""
    rows = P.flatten(-2)
    return rows.narrow(-1, 0, b.n).movedim(-1, b.axis).contiguous()


def scales_from_blocks(X: torch.Tensor, b: Blocks) -> torch.Tensor:
    """Scales in block form (..., nblocks, 1) in the layout of that tensor with its axis nblocks long,
    contiguous (mxq/block/_driver.py:40-42)."""
    return X.squeeze(-1).movedim(-1, b.axis).contiguous()


def _view3(shape, axis: int):
    outer = _lib.numel(shape[:axis])
    inner = _lib.numel(shape[axis + 1:])
    return outer, int(shape[axis]), inner


def quantize_fused(V: torch.Tensor, axis: int, block_size: int, spec: _lib.BlockSpec) -> Tuple[torch.Tensor, torch.Tensor]:
    """One kernel: amax, scale, divide, element rule, for every block of V along `axis` (already validated)."""
    axis = _axis(V, axis)
    _check_block(block_size)
    if V.is_cuda:
        dev, Vd = V.device, V                           # only its memory is read: no autograd record needed
    else:
        dev = _lib.compute_device(V)
        Vd = V.detach().to(dev)
    if Vd.dtype not in _NATIVE:
        Vd = Vd.to(torch.float32)                       # the reference's V.to(float32) (RNE from float64)
    if not Vd.is_contiguous():
        if _transposed_view(Vd, axis, block_size):
            return _quantize_transposed(Vd, dev, spec, V)
        Vd = Vd.contiguous()
    n = Vd.shape[axis]
    if n > 1 and Vd.numel():
        inner = Vd.stride(axis)                         # contiguous, numel > 0, length > 1: the inner size
        outer = Vd.numel() // (n * inner)
    else:
        outer, n, inner = _view3(Vd.shape, axis)
    nb = -(-n // block_size)
    xshape = list(Vd.shape)
    xshape[axis] = nb
    # torch.empty_like and new_empty skip the device and dtype parsing of torch.empty (half a microsecond each)
    P = torch.empty_like(Vd, dtype=torch.float32)
    X = Vd.new_empty(xshape, dtype=torch.float32)
    with _lib.on(dev):
        _lib.run("mxq_block_quantize", _lib.ptr(Vd), _NATIVE[Vd.dtype], _lib.ptr(P), _lib.ptr(X), outer, n, inner,
                 block_size, spec, _lib.stream(dev))
    if V.is_cuda:
        return P, X
    return _lib.back(P, V), _lib.back(X, V)


def quantize_dither(V: torch.Tensor, axis: int, block_size: int, spec: _lib.BlockSpec) -> Tuple[torch.Tensor, torch.Tensor]:
    """quantize_fused for microxcaling's element step rounding by dither (mxq_block_quantize_dither).  The
    uniforms are drawn on V's device in the reference's order: one per block maximum when the scale rule rounds
    the maximum (ocp_no_clip), then one per element of the blocked tensor (..., nblocks, block_size), padding
    included."""
    from ..element_quant.microsoft import draws
    axis = _axis(V, axis)
    _check_block(block_size)
    outer, n, inner = _view3(V.shape, axis)
    nb = -(-n // block_size)
    u_amax = draws(V, outer * inner * nb) if spec.scale_rule == _lib.SCALE_OCP_NO_CLIP else None
    u = draws(V, outer * inner * nb * block_size)
    dev = _lib.compute_device(V)
    Vd = _lib.to_device(V.detach(), dev)
    if Vd.dtype not in _NATIVE:
        Vd = Vd.to(torch.float32)
    Vd = Vd.contiguous()
    xshape = list(Vd.shape)
    xshape[axis] = nb
    P = torch.empty(Vd.shape, dtype=torch.float32, device=dev)
    X = torch.empty(xshape, dtype=torch.float32, device=dev)
    u_amax = None if u_amax is None else _lib.to_device(u_amax, dev)
    u = _lib.to_device(u, dev)
    with _lib.on(dev):
        _lib.run("mxq_block_quantize_dither", _lib.ptr(Vd), _NATIVE[Vd.dtype], _lib.ptr(u_amax), _lib.ptr(u),
                 _lib.ptr(P), _lib.ptr(X), outer, n, inner, block_size, spec, _lib.stream(dev))
    return _lib.back(P, V), _lib.back(X, V)


def _transposed_view(V: torch.Tensor, axis: int, block_size: int) -> bool:
    """V (n x inner) is the transpose of a row-major matrix and is quantized along axis 0 in blocks of 32."""
    return (V.ndim == 2 and axis == 0 and block_size == 32 and not V.is_contiguous()
            and V.stride() == (1, V.shape[0]) and V.shape[0] > 1 and V.shape[1] > 1)


def _quantize_transposed(Vd: torch.Tensor, dev: torch.device, spec: _lib.BlockSpec, V: torch.Tensor):
    """quantize_fused of a transposed view, read as it lies (no copy of the input)."""
    n, inner = Vd.shape
    P = torch.empty((n, inner), dtype=torch.float32, device=dev)
    X = torch.empty((-(-n // 32), inner), dtype=torch.float32, device=dev)
    with _lib.on(dev):
        _lib.run("mxq_block_quantize_t", _lib.ptr(Vd), _NATIVE[Vd.dtype], _lib.ptr(P), _lib.ptr(X), n, inner, 32,
                 spec, _lib.stream(dev))
    return _lib.back(P, V), _lib.back(X, V)


def compose(V: torch.Tensor, *, scale: Optional[Callable[[torch.Tensor], torch.Tensor]],
            elem: Optional[Callable[[torch.Tensor], torch.Tensor]],
            axis: int = 0, block_size: int = BLOCK) -> Tuple[torch.Tensor, torch.Tensor]:
    """Block quantization from its two steps; returns (P codes, X scales), float32.

    scale(amax) -> X   step 1: amax is each block's max |value|, shape (..., nblocks, 1); X the same shape
    elem(z) -> P       step 2: z = block / X, shape (..., nblocks, block_size); P the same shape
    Either may be None: no scale step means X = 1, no element step means P = V / X; both None is FP32
    pass-through (one kernel)."""
    if scale is None and elem is None:
        return quantize_fused(V, axis, block_size, _lib.BlockSpec())
    V = V.to(torch.float32)
    b = to_blocks(V, axis, block_size)
    if scale is None:
        X = torch.ones(b.data.shape[:-1] + (1,), dtype=torch.float32, device=V.device)
        z = b.data
    else:
        X = scale(b.data.abs().amax(dim=-1, keepdim=True))
        z = b.data / X
    P = z.clone() if elem is None else elem(z)
    return codes_from_blocks(P, b), scales_from_blocks(X, b)


def dequantize(P: torch.Tensor, X: torch.Tensor, axis: int = 0, block_size: int = BLOCK) -> torch.Tensor:
    """V_hat = P * expand(X): each scale repeated block_size times along `axis`, cut to P's length."""
    axis = axis % P.ndim
    _check_block(block_size)
    n = P.shape[axis]
    nb = -(-n // block_size)
    want = list(P.shape)
    want[axis] = nb
    if P.dtype == torch.float32 and X.dtype == torch.float32 and list(X.shape) == want and P.device == X.device:
        dev = _lib.compute_device(P)
        Pd = _lib.to_device(P.detach(), dev).contiguous()
        Xd = _lib.to_device(X.detach(), dev).contiguous()
        out = torch.empty_like(Pd)
        outer, n, inner = _view3(Pd.shape, axis)
        with _lib.on(dev):
            _lib.run("mxq_block_dequantize", _lib.ptr(Pd), _lib.ptr(Xd), _lib.ptr(out), outer, n, inner, block_size,
                     _lib.stream(dev))
        return _lib.back(out, P)
    # any other dtype or a broadcasting X: the reference's expression, on the tensors' device
    Xe = torch.repeat_interleave(X, block_size, dim=axis).narrow(axis, 0, P.shape[axis])
    return P * Xe
