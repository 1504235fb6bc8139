"""mxq_systolic_noalloc (the systolic entry point that allocates nothing) through the C ABI, bit for bit against
mxq_systolic with a caller's workspace: two calls in a row, the second smaller, each with tiles that the fast
kernel hands to the general kernel (so the flags kept in the library's device array decide results), then the
general kernel alone; and the size limit, refused before any launch."""
import ctypes

import numpy as np
import pytest
import torch

from _util import assert_bits_equal
from oracle import block as ob
from oracle import numerics as nx
from oracle import systolic as osys

pytestmark = pytest.mark.gpu


def _operands(rng, K, M, N, wild_cols):
    A = rng.standard_normal((K, M)).astype(np.float32)
    B = (rng.standard_normal((K, N)) * 0.02).astype(np.float32)
    pa, xa = ob.mxgemmini_quantize(A, "MXFP8_E4M3", 0)
    pb, xb = ob.mxgemmini_quantize(B, "MXFP8_E4M3", 0)
    for c in wild_cols:                                 # a code far past the fast kernel's bound: general kernel
        pb[3, c] = 2.0 ** 60
    return [torch.from_numpy(np.ascontiguousarray(t)).cuda() for t in (pa, xa, pb, xb)]


def _args(ops, K, M, N):
    from mxq import _lib, matmul
    sched = matmul.HW_FINAL
    le = (ctypes.c_int32 * 16)(*[e for e, _ in sched])
    lm = (ctypes.c_int32 * 16)(*[m for _, m in sched])
    return [_lib.ptr(t) for t in ops], le, lm, matmul.MXGEMMINI().kernel.ctype()


def _with_workspace(ops, K, M, N, force):
    from mxq import _lib
    from mxq.matmul._systolic import workspace_elements
    p, le, lm, ar = _args(ops, K, M, N)
    C = torch.empty(M, N, device="cuda")
    work = torch.empty(workspace_elements(K, M, N, 1), dtype=torch.int32, device="cuda")
    _lib.run("mxq_systolic", *p, _lib.ptr(C), K, M, N, le, lm, 16, 32, ar, _lib.ptr(work), force,
             _lib.stream(C.device))
    return C


def _no_alloc(ops, K, M, N, force):
    from mxq import _lib
    p, le, lm, ar = _args(ops, K, M, N)
    C = torch.full((M, N), float("nan"), device="cuda")
    _lib.run("mxq_systolic_noalloc", *p, _lib.ptr(C), K, M, N, le, lm, 16, 32, ar, force, _lib.stream(C.device))
    return C


def test_no_alloc_matches_workspace_entry(cuda):
    rng = np.random.default_rng(31)
    cases = [(4096, 512, 1024, [5, 700]), (1000, 100, 200, [150])]      # the second call smaller, a K tail
    for K, M, N, wild in cases:
        ops = _operands(rng, K, M, N, wild)
        for force in (1, 0):                            # the fast kernel and its flags last
            want = _with_workspace(ops, K, M, N, force)
            got = _no_alloc(ops, K, M, N, force)
            torch.cuda.synchronize()
            assert_bits_equal(got.cpu().numpy(), want.cpu().numpy(), f"noalloc K={K} M={M} N={N} force={force}")
        # the columns the general kernel computed, against the oracle
        pa, xa, pb, xb = (t.cpu().numpy() for t in ops)
        oracle = osys.systolic(pa, xa, pb[:, wild], xb[:, wild], nx.MXGEMMINI(), osys.HW_FINAL)
        assert_bits_equal(got.cpu().numpy()[:, wild], oracle, "general-kernel columns vs the oracle")


def test_no_alloc_size_limit(cuda):
    """ceil(M/32) * ceil(N/32) above 262144 is refused before any launch, with the reason."""
    from mxq import _lib
    lib = _lib.load()
    t = torch.zeros(64, device="cuda")
    p, le, lm, ar = _args([t, t, t, t], 32, 16416, 16416)
    rc = lib.mxq_systolic_noalloc(*p, _lib.ptr(t), 32, 16416, 16416, le, lm, 16, 32, ar, 0, _lib.stream(t.device))
    assert rc == 1 and b"262144" in lib.mxq_last_error()


def test_no_alloc_refuses_overlapping_streams(cuda):
    """A call on a second stream while the first stream's call (4096^3, milliseconds of kernels) may still run
    is refused with MXQ_EBUSY and launches nothing; once that call is done, the second stream's call runs and
    gives the same bits; calls on one stream back to back are never refused."""
    from mxq import _lib
    lib = _lib.load()
    rng = np.random.default_rng(32)
    K = M = N = 4096
    ops = _operands(rng, K, M, N, [])
    p, le, lm, ar = _args(ops, K, M, N)
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    C1 = torch.empty(M, N, device="cuda")
    C2 = torch.full((M, N), float("nan"), device="cuda")
    torch.cuda.synchronize()
    call = lambda C, s: lib.mxq_systolic_noalloc(*p, _lib.ptr(C), K, M, N, le, lm, 16, 32, ar, 0,   # noqa: E731
                                                 s.cuda_stream)
    assert call(C1, s1) == 0
    assert call(C1, s1) == 0                            # the same stream: ordered by it
    rc = call(C2, s2)
    busy = rc == 3
    assert rc in (0, 3)
    if busy:
        assert b"another stream" in lib.mxq_last_error()
        s2.synchronize()
        assert torch.isnan(C2).all(), "a refused call launches nothing"
    s1.synchronize()
    assert busy, "the first stream's 4096^3 call was still queued when the second call came"
    assert call(C2, s2) == 0
    s2.synchronize()
    assert torch.equal(C1, C2)
