"""Fitting the tables and picking indices for a K x n tensor of block codes, one table per 2^G columns
(mxq/lut/kmeans.py:1-152), on the GPU.

    T = tables(P, fmt, group=G, max_iters=50)   ceil(n / 2^G) x SIZE values, each row ascending
    I = pick(P, T, group=G)                     K x n int64: each code's nearest entry, ties to the lower index
    P_lut = lookup(I, T, group=G)

A table is fitted to its group's codes: the distinct codes weighted by how often they occur; 16 or fewer are
the centres, else 16 quantile seeds refined by weighted Lloyd passes in float64 (an empty cluster keeps its
centre, equal centres merge) until two passes agree to numpy.allclose or max_iters; each centre snapped to
the nearest finder-safe value; duplicates dropped; padded to 16 with unused safe values of smallest
magnitude; sorted.  Every sum is exact, so the GPU's summation order gives the same tables.
"""
import torch

from .. import _lib
from .formats import SIZE, _format, _grid, _tables

__all__ = ["tables", "pick", "lookup"]


def _check(P: torch.Tensor, group: int) -> int:
    if P.ndim != 2:
        raise ValueError(f"mxq.lut: expects a K×n tensor, got shape {tuple(P.shape)}")
    if not isinstance(group, int) or isinstance(group, bool) or group < 0:
        raise ValueError(f"mxq.lut: group {group!r} must be a non-negative integer")
    return (P.shape[1] + (1 << group) - 1) >> group


def _check_tables(T: torch.Tensor, ng: int, n: int, group: int, who: str) -> None:
    if T.ndim != 2 or T.shape[0] != ng or T.shape[1] < 2:
        raise ValueError(f"mxq.lut.{who}: {n} columns at group {group} need ({ng}, width) tables with width >= 2, "
                         f"got {tuple(T.shape)}")


_DEVICE_GRIDS = {}


def _device_grid(name: str, dev: torch.device):
    """(value grid, safe values, safe order) of a format on `dev`, copied there once per process."""
    key = (name, dev)
    if key not in _DEVICE_GRIDS:
        grid, order = _grid(name)
        _DEVICE_GRIDS[key] = (grid.to(dev), _tables(name)[2].to(dev), order.to(dev))
    return _DEVICE_GRIDS[key]


def _not_a_code(fmt_name: str) -> ValueError:
    return ValueError(f"mxq.lut: P holds a value that is not a {fmt_name} code; quantize it first")


def fit(P: torch.Tensor, fmt, group: int, max_iters: int):
    """(T, err): the tables of `tables` and, on P's compute device, the int32 word the kernels set when P holds
    a value that is not a code of fmt (read it to raise as `tables` does).  No host synchronisation."""
    f = _format(fmt)
    ng = _check(P, group)
    if not isinstance(max_iters, int) or isinstance(max_iters, bool) or max_iters < 0:
        raise ValueError(f"mxq.lut: max_iters {max_iters!r} must be a non-negative integer")
    dev = _lib.compute_device(P)
    Pd = _lib.to_device(P.detach(), dev).to(torch.float32).contiguous()
    g_d, s_d, o_d = _device_grid(f.name, dev)
    K, n = Pd.shape
    nv = g_d.numel()
    T = torch.empty((ng, SIZE), dtype=torch.float32, device=dev)
    work = torch.empty(ng * nv + 1, dtype=torch.int32, device=dev)
    if n == 0:
        work.zero_()
    with _lib.on(dev):
        _lib.run("mxq_lut_tables", _lib.ptr(Pd), K, n, group, max_iters, _lib.ptr(g_d), nv, _lib.ptr(s_d),
                 s_d.numel(), _lib.ptr(o_d), f.e, f.m, _lib.ptr(T), _lib.ptr(work), _lib.stream(dev))
    return T, work[-1:]


def tables(P: torch.Tensor, fmt, *, group: int, max_iters: int) -> torch.Tensor:
    """One SIZE-entry table per 2^group columns of P (K x n block codes, each a value of fmt)."""
    f = _format(fmt)
    T, err = fit(P, fmt, group, max_iters)
    if int(err.item()):
        raise _not_a_code(f.name)
    return _lib.back(T, P)


def _pick(P: torch.Tensor, T: torch.Tensor, group: int, values: bool) -> torch.Tensor:
    dev = _lib.compute_device(P, T)
    Pd = _lib.to_device(P.detach(), dev).to(torch.float32).contiguous()
    Td = _lib.to_device(T.detach(), dev).to(torch.float32).contiguous()
    K, n = Pd.shape
    out = torch.empty((K, n), dtype=torch.float32 if values else torch.int64, device=dev)
    with _lib.on(dev):
        _lib.run("mxq_lut_pick", _lib.ptr(Pd), K, n, group, _lib.ptr(Td), Td.shape[1],
                 _lib.ptr(None if values else out), _lib.ptr(out if values else None), _lib.stream(dev))
    return _lib.back(out, P)


def pick(P: torch.Tensor, T: torch.Tensor, *, group: int) -> torch.Tensor:
    """Each code's nearest entry in its column group's table, ties to the lower index: K x n int64.  Any table
    width of two or more (one ascending row per group); the chip's is SIZE."""
    ng = _check(P, group)
    _check_tables(T, ng, P.shape[1], group, "pick")
    return _pick(P, T, group, values=False)


def pick_values(P: torch.Tensor, T: torch.Tensor, *, group: int) -> torch.Tensor:
    """lookup(pick(P, T), T) in one kernel, without the int64 indices: K x n float32."""
    ng = _check(P, group)
    _check_tables(T, ng, P.shape[1], group, "pick")
    return _pick(P, T, group, values=True)


def lookup(I: torch.Tensor, T: torch.Tensor, *, group: int) -> torch.Tensor:
    """The values the indices name: K x n float32.  Any table width (one row per group)."""
    ng = _check(I, group)
    _check_tables(T, ng, I.shape[1], group, "lookup")
    dev = _lib.compute_device(I, T)
    Id = _lib.to_device(I.detach(), dev).long().contiguous()
    Td = _lib.to_device(T.detach(), dev).to(torch.float32).contiguous()
    width = Td.shape[1]
    if Id.numel() and (bool((Id < 0).any()) or bool((Id >= width).any())):
        raise IndexError(f"mxq.lut.lookup: index out of range for tables of width {width}")
    K, n = Id.shape
    out = torch.empty((K, n), dtype=torch.float32, device=dev)
    with _lib.on(dev):
        _lib.run("mxq_lut_lookup", _lib.ptr(Id), K, n, group, _lib.ptr(Td), width, _lib.ptr(out), _lib.stream(dev))
    return _lib.back(out, I)
