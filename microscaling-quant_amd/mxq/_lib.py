"""Loader and call plumbing for libmxq_hip.so, the gfx950 kernels behind every mxq operation.

The library is a plain C ABI (include/mxq_hip.h) loaded with ctypes.  torch is imported first, so the
library's libamdhip64.so.7 dependency resolves to the HIP runtime torch already loaded: one runtime, one set
of streams and device pointers.  Tensors are passed as device pointers; outputs are allocated by torch on the
input's device; kernels run on torch's current stream of that device.

There is no CPU implementation behind this package.  CPU tensors are copied to the current GPU, computed
there, and copied back (the reference returns outputs on the input's device).  Without a GPU, or without the
built library, every computing call raises RuntimeError.
"""
import contextlib
import ctypes
import functools
import os
import threading
from typing import Optional, Sequence

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get("MXQ_HIP_LIB", os.path.join(_HERE, "libmxq_hip.so"))

_lock = threading.Lock()
_lib: Optional[ctypes.CDLL] = None
_FN = {}            # entry point name -> its ctypes function, filled by load()

#: the MXQ_ABI_VERSION of include/mxq_hip.h these signatures follow; a library reporting another is refused
ABI_VERSION = 4

c_i32, c_i64, c_f32, c_f64, c_ptr = ctypes.c_int32, ctypes.c_int64, ctypes.c_float, ctypes.c_double, ctypes.c_void_p


class BlockSpec(ctypes.Structure):
    """mxq_block_spec (include/mxq_hip.h)."""
    _fields_ = [("scale_rule", c_i32), ("scale_floor", c_f32), ("scale_emax", c_i32), ("scale_bits", c_i32),
                ("elem", c_i32), ("e", c_i32), ("m", c_i32), ("rounding", c_i32), ("max_norm", c_f32),
                ("via_e", c_i32), ("via_m", c_i32)]


class ArithSpec(ctypes.Structure):
    """mxq_arith_spec (include/mxq_hip.h)."""
    _fields_ = [("kind", c_i32), ("prod_e", c_i32), ("prod_m", c_i32), ("has_floor", c_i32), ("flush_thr", c_f32),
                ("sat_limit", c_f32), ("sat_value", c_f32)]


class SystolicHints(ctypes.Structure):
    """include/mxq_hip.h mxq_systolic_hints: device pointers (0 for none) to the skip map, the k_end bounds, the
    caller's suffix bytes of A and the column bounds past which skipped tiles are not stored."""
    _fields_ = [("skip", c_ptr), ("k_end", c_ptr), ("a_live", c_ptr), ("c_end", c_ptr)]


class SystolicEpilogue(ctypes.Structure):
    """include/mxq_hip.h mxq_systolic_epilogue: R(R(C * scale) + mask value) on every stored output."""
    _fields_ = [("scale", ctypes.c_float), ("bf16", ctypes.c_int32), ("mask", c_ptr),
                ("mask_b_stride", ctypes.c_int64), ("mask_row_stride", ctypes.c_int64), ("z0", ctypes.c_int64),
                ("z_per_b", ctypes.c_int64), ("m", ctypes.c_int64)]


class SoftmaxTail(ctypes.Structure):
    """include/mxq_hip.h mxq_softmax_tail: per 64-row group the keys S holds (k_end) and the largest score past
    them (tail_max), and the score step that gives those scores from the mask."""
    _fields_ = [("k_end", c_ptr), ("tail_max", c_ptr), ("score", SystolicEpilogue)]


class SystolicLayout(ctypes.Structure):
    """mxq_systolic_layout (include/mxq_hip.h): row and problem strides of the five operands, in elements."""
    _fields_ = [(n, c_i64) for n in ("ld_a", "batch_a", "ld_xa", "batch_xa", "ld_b", "batch_b", "ld_xb", "batch_xb",
                                     "ld_c", "batch_c")]


class AnchorSpec(ctypes.Structure):
    """mxq_anchor_spec (include/mxq_hip.h)."""
    _fields_ = [(n, c_i32) for n in ("width", "drop", "headroom", "has_emin", "emin", "nbits")]


# exported symbol -> (restype, argtypes); every symbol include/mxq_hip.h declares
SIGNATURES = {
    "mxq_last_error": (ctypes.c_char_p, []),
    "mxq_version": (c_i32, []),
    "mxq_timer_enable": (c_i32, [c_i32]),
    "mxq_timer_read": (c_i32, [ctypes.c_char_p, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(c_i64)]),
    "mxq_valu_probe": (c_i32, [c_i32, c_i32, c_i64, c_ptr, c_ptr]),
    "mxq_block_quantize": (c_i32, [c_ptr, c_i32, c_ptr, c_ptr, c_i64, c_i64, c_i64, c_i64,
                                   ctypes.POINTER(BlockSpec), c_ptr]),
    "mxq_block_quantize_t": (c_i32, [c_ptr, c_i32, c_ptr, c_ptr, c_i64, c_i64, c_i64, ctypes.POINTER(BlockSpec),
                                     c_ptr]),
    "mxq_block_dequantize": (c_i32, [c_ptr, c_ptr, c_ptr, c_i64, c_i64, c_i64, c_i64, c_ptr]),
    "mxq_block_quantize_packed": (c_i32, [c_ptr, c_i32, c_ptr, c_ptr, c_ptr, c_i64, c_i64, c_i64, c_i64,
                                          ctypes.POINTER(BlockSpec), c_ptr]),
    "mxq_pack": (c_i32, [c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, c_i64, c_i64, c_i64, c_i64, c_i32, c_i32, c_ptr]),
    "mxq_unpack": (c_i32, [c_ptr, c_ptr, c_ptr, c_ptr, c_i64, c_i64, c_i64, c_i64, c_i32, c_i32, c_ptr]),
    "mxq_dequantize_packed": (c_i32, [c_ptr, c_ptr, c_ptr, c_i64, c_i64, c_i64, c_i64, c_i32, c_i32, c_ptr]),
    "mxq_lut_pick_packed": (c_i32, [c_ptr, c_i64, c_i64, c_i32, c_ptr, c_i32, c_ptr, c_ptr]),
    "mxq_lut_lookup_packed": (c_i32, [c_ptr, c_i64, c_i64, c_i32, c_ptr, c_i32, c_ptr, c_ptr]),
    "mxq_systolic": (c_i32, [c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, c_i64, c_i64, c_i64, c_ptr, c_ptr, c_i32, c_i32,
                             ctypes.POINTER(ArithSpec), c_ptr, c_i32, c_ptr]),
    "mxq_systolic_batched": (c_i32, [c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, ctypes.POINTER(SystolicLayout), c_i64,
                                     c_i64, c_i64, c_i64, c_ptr, c_ptr, c_i32, c_i32, ctypes.POINTER(ArithSpec),
                                     c_ptr, c_ptr, c_ptr, c_i32, c_ptr]),
    "mxq_systolic_noalloc": (c_i32, [c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, c_i64, c_i64, c_i64, c_ptr, c_ptr, c_i32,
                                     c_i32, ctypes.POINTER(ArithSpec), c_i32, c_ptr]),
    "mxq_systolic_workspace": (c_i64, [c_i64, c_i64, c_i64, c_i64]),
    "mxq_scores_scale_mask": (c_i32, [c_ptr, c_i64, c_i64, c_i64, c_i64, c_f32, c_ptr, c_i64, c_i64, c_i64, c_i64,
                                      c_i32, c_ptr]),
    "mxq_group_amax": (c_i32, [c_ptr, c_ptr, c_i64, c_i64, c_i64, c_i64, c_ptr, c_ptr]),
    "mxq_mask_minabs": (c_i32, [c_ptr, c_i64, c_i64, c_i64, c_i64, c_i64, c_i64, c_ptr, c_ptr, c_ptr]),
    "mxq_attend_hints": (c_i32, [c_ptr, c_i64, c_ptr, c_i64, c_i64, c_i64, c_f64, c_ptr, c_i64, c_i64, c_i32, c_i64,
                                 c_i64, c_ptr, c_ptr, c_ptr, c_ptr, c_ptr]),
    "mxq_attend_windows": (c_i32, [c_ptr, c_i64, c_ptr, c_i64, c_i64, c_i64, c_f64, c_ptr, c_i64, c_i64, c_i64,
                                   c_i64, c_i64, c_i64, c_i64, c_ptr, c_ptr]),
    "mxq_adder_tree": (c_i32, [c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, c_i64, c_i64, c_i64, c_ptr, c_ptr, c_i32, c_i32,
                               ctypes.POINTER(ArithSpec), c_ptr, c_i32, c_ptr]),
    "mxq_anchor_tree": (c_i32, [c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, c_i64, c_i64, c_i64, c_ptr, c_ptr, c_ptr, c_i32,
                                c_i32, ctypes.POINTER(AnchorSpec), ctypes.POINTER(ArithSpec), c_ptr, c_i32, c_ptr]),
    "mxq_mx_pack": (c_i32, [c_ptr, c_ptr, c_i64, c_i64, c_i32, c_ptr, c_ptr, c_ptr, c_ptr]),
    "mxq_mx_pack_bytes": (c_i32, [c_ptr, c_ptr, c_i64, c_i64, c_i32, c_ptr, c_ptr, c_ptr, c_ptr]),
    "mxq_mx_mfma": (c_i32, [c_ptr, c_ptr, c_i32, c_ptr, c_ptr, c_i32, c_ptr, c_i64, c_i64, c_i64, c_ptr]),
    "mxq_lut_tables": (c_i32, [c_ptr, c_i64, c_i64, c_i32, c_i32, c_ptr, c_i32, c_ptr, c_i32, c_ptr, c_i32, c_i32,
                               c_ptr, c_ptr, c_ptr]),
    "mxq_lut_pick": (c_i32, [c_ptr, c_i64, c_i64, c_i32, c_ptr, c_i32, c_ptr, c_ptr, c_ptr]),
    "mxq_block_lut": (c_i32, [c_ptr, c_i32, c_i64, c_i64, ctypes.POINTER(BlockSpec), c_i32, c_i32, c_ptr, c_i32,
                              c_ptr, c_i32, c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, c_i64, c_ptr, c_ptr]),
    "mxq_softmax_quantize_t": (c_i32, [c_ptr, c_i64, c_i64, c_ptr, c_ptr, ctypes.POINTER(BlockSpec), c_ptr, c_i64,
                                       ctypes.POINTER(SoftmaxTail), c_ptr]),
    "mxq_systolic_fast_lanes": (c_i32, [c_ptr, c_ptr, c_i32, ctypes.POINTER(ArithSpec)]),
    "mxq_block_lut_workspace": (c_i32, [c_i64, c_i64, c_i32, c_i32, c_i32, c_i32, ctypes.POINTER(c_i64)]),
    "mxq_lut_lookup": (c_i32, [c_ptr, c_i64, c_i64, c_i32, c_ptr, c_i32, c_ptr, c_ptr]),
    "mxq_lut_finder": (c_i32, [c_ptr, c_i64, c_i64, c_i32, c_ptr, c_i32, c_ptr, c_i64, c_ptr, c_ptr]),
    "mxq_round_bits": (c_i32, [c_ptr, c_ptr, c_i32, c_ptr, c_i64, c_i32, c_ptr]),
    "mxq_round_int": (c_i32, [c_ptr, c_i32, c_ptr, c_i64, c_i32, c_ptr]),
    "mxq_bf16": (c_i32, [c_ptr, c_ptr, c_i64, c_ptr]),
    "mxq_float_em": (c_i32, [c_ptr, c_i32, c_ptr, c_i64, c_i32, c_i32, c_i32, c_i32, c_f32, c_ptr]),
    "mxq_microsoft": (c_i32, [c_ptr, c_ptr, c_i64, c_i32, c_i32, c_f32, c_i32, c_i32, c_ptr]),
    "mxq_scale_factor": (c_i32, [c_ptr, c_ptr, c_i64, ctypes.POINTER(BlockSpec), c_ptr]),
    "mxq_microsoft_dither": (c_i32, [c_ptr, c_ptr, c_ptr, c_i64, c_i32, c_i32, c_f32, c_i32, c_ptr]),
    "mxq_scale_factor_dither": (c_i32, [c_ptr, c_ptr, c_ptr, c_i64, ctypes.POINTER(BlockSpec), c_ptr]),
    "mxq_block_quantize_dither": (c_i32, [c_ptr, c_i32, c_ptr, c_ptr, c_ptr, c_ptr, c_i64, c_i64, c_i64, c_i64,
                                          ctypes.POINTER(BlockSpec), c_ptr]),
    "mxq_exact_add": (c_i32, [c_ptr, c_ptr, c_ptr, c_i64, c_i32, c_i32, c_i32, c_i32, c_f32, c_ptr]),
    "mxq_truncate_significand": (c_i32, [c_ptr, c_ptr, c_i64, c_i32, c_ptr]),
    "mxq_flush_product": (c_i32, [c_ptr, c_ptr, c_i64, c_f32, c_ptr]),
    "mxq_saturate": (c_i32, [c_ptr, c_ptr, c_i64, c_f32, c_f32, c_ptr]),
}

# mxq_block_spec codes
SCALE_NONE, SCALE_MXQUANT, SCALE_OCP, SCALE_OCP_NO_CLIP = 0, 1, 2, 3
ELEM_NONE, ELEM_QTORCH, ELEM_IEEE, ELEM_OCP, ELEM_MICROSOFT = 0, 1, 2, 3, 4
MODE_CODE = {"ties_away": 0, "rne": 1, "truncate": 2}
MS_MODE_CODE = {"nearest": 0, "even": 1, "floor": 2, "dither": 3}
GRID_CODE = {"qtorch": 0, "ieee": 1, "ocp": 2}
ARITH_MXGEMMINI, ARITH_MXQUANT = 0, 1


def load(path: str = LIB_PATH) -> ctypes.CDLL:
    """Open the library (once) and declare every entry point's C signature."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(path):
                raise RuntimeError(f"mxq: the HIP library {path} is not built; run __graft_entry__.build() "
                                   "or microscaling-quant_amd/csrc/build.py")
            lib = ctypes.CDLL(path)
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype, fn.argtypes = res, args
                _FN[name] = fn
            if lib.mxq_version() != ABI_VERSION:
                _FN.clear()
                raise RuntimeError(f"mxq: {path} has C ABI revision {lib.mxq_version()}, this package binds "
                                   f"revision {ABI_VERSION}; rebuild the library")
            _lib = lib
    return _lib


def memo_spec(make):
    """make, remembered per positional arguments (their types included): a spec struct is only read once built,
    and building one, with the reference's argument checks, costs about a microsecond of every call.  Arguments
    that cannot be hashed are built afresh; errors are raised as make raises them."""
    cached = functools.lru_cache(maxsize=512, typed=True)(make)

    @functools.wraps(make)
    def spec(*args):
        try:
            return cached(*args)
        except TypeError:
            return make(*args)
    return spec


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = load().mxq_last_error()
        raise RuntimeError(f"mxq: {what} failed ({rc}): {msg.decode() if msg else 'unknown error'}")


def compute_device(*tensors: torch.Tensor) -> torch.device:
    """The GPU the kernels run on: the tensors' CUDA device, or the current one for CPU tensors."""
    for t in tensors:
        if isinstance(t, torch.Tensor) and t.device.type == "cuda":
            return t.device
    if not torch.cuda.is_available():
        raise RuntimeError("mxq: no GPU is visible; this implementation runs its kernels on gfx950 only "
                           "(CPU tensors are computed on the current GPU and copied back)")
    return torch.device("cuda", torch.cuda.current_device())


def to_device(t: torch.Tensor, dev: torch.device) -> torch.Tensor:
    return t if t.device == dev else t.to(dev)


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream(dev: torch.device) -> int:
    """torch's current stream of `dev` as a hipStream_t handle (an int)."""
    if _raw_stream is not None:
        return _raw_stream(dev.index if dev.index is not None else torch.cuda.current_device())
    return torch.cuda.current_stream(dev).cuda_stream


_SAME_DEVICE = contextlib.nullcontext()


def on(dev: torch.device):
    """A context in which `dev` is the current device: torch.cuda.device(dev), or nothing to do when it already
    is (the common case, and a microsecond less per call)."""
    if dev.index is None or dev.index == torch.cuda.current_device():
        return _SAME_DEVICE
    return torch.cuda.device(dev)


def ptr(t: Optional[torch.Tensor]) -> int:
    return 0 if t is None else t.data_ptr()


def aligned(t: torch.Tensor, nbytes: int = 16) -> torch.Tensor:
    """t itself when its first element sits on an nbytes boundary, else a fresh contiguous copy (torch's
    allocator hands out 256-byte aligned blocks).  Views at an odd offset into a larger storage are valid
    inputs; kernels that load 16 bytes a lane need the copy."""
    return t if t.data_ptr() % nbytes == 0 else torch.empty_like(t, memory_format=torch.contiguous_format).copy_(t)


def back(t: torch.Tensor, like: torch.Tensor) -> torch.Tensor:
    """Return a result on the device of the caller's tensor `like`."""
    return t if t.device == like.device else t.to(like.device)


def numel(shape: Sequence[int]) -> int:
    n = 1
    for s in shape:
        n *= int(s)
    return n


def run(name: str, *args) -> None:
    """Call entry point `name` with args; raise RuntimeError on a nonzero status."""
    fn = _FN.get(name)
    if fn is None:
        load()
        fn = _FN[name] if name in _FN else getattr(load(), name)
    rc = fn(*args)
    if rc != 0:
        check(rc, name)


def ew_prepare(x: torch.Tensor, dtype: torch.dtype):
    """(compute device, contiguous copy of x converted to dtype on that device)."""
    dev = compute_device(x)
    xd = to_device(x.detach(), dev).to(dtype).contiguous()
    return dev, xd


def timer_enable(on: bool) -> None:
    """Start (True) or stop timing the library's kernel launches with HIP events (see mxq_timer_enable)."""
    run("mxq_timer_enable", 1 if on else 0)


def timer_read(kernel: str):
    """(summed milliseconds, launches) of the timed launches of `kernel` since the last read; waits for them."""
    ms, n = ctypes.c_double(0.0), c_i64(0)
    run("mxq_timer_read", kernel.encode(), ctypes.byref(ms), ctypes.byref(n))
    return ms.value, n.value
