"""matmul.adder_tree and matmul.anchor_tree on the GPU, bit for bit against the oracle (oracle/trees.py)."""
from functools import partial

import numpy as np
import pytest
import torch

from _util import assert_bits_equal, special_f32
from oracle import block as ob
from oracle import numerics as nx
from oracle import trees as ot

pytestmark = pytest.mark.gpu


def _codes(rng, K, n, fmt="MXFP8_E4M3", mode="ties_away", floor=1e-38, scale=1.0):
    V = (rng.standard_normal((K, n)) * scale).astype(np.float32)
    return ob.mxgemmini_quantize(V, fmt, 0, 32, mode, floor)


def _t(*arrs):
    return [torch.from_numpy(np.ascontiguousarray(a)).cuda() for a in arrs]


def _arith(name, *a):
    from mxq import matmul
    return getattr(matmul, name)(*a), getattr(nx, name)(*a)


ADDER_CASES = [
    (2, [(4, 4)], ("MXGEMMINI",)),
    (4, [(4, 3), (8, 7)], ("MXGEMMINI",)),
    (8, [(4, 4), (4, 6), (8, 7)], ("MXGEMMINI",)),
    (16, [(8, 7)] * 4, ("MXGEMMINI",)),
    (16, [(4, 4), (4, 5), (4, 6), (8, 7)], ("MXGEMMINI", 4, 3, None)),
    (32, [(4, 5), (4, 5), (4, 6), (4, 6), (8, 7)], ("MXGEMMINI",)),
    (16, [(5, 4), (5, 6), (6, 8), (8, 10)], ("MXQUANT", 4, 3)),
    (8, [(8, 23)] * 3, ("MXQUANT", 8, 23)),
]


@pytest.mark.parametrize("case", ADDER_CASES, ids=[f"s{c[0]}_{i}" for i, c in enumerate(ADDER_CASES)])
@pytest.mark.parametrize("shape", [(256, 64, 96), (77, 33, 70), (5, 3, 9)])
def test_adder_tree_against_oracle(cuda, case, shape):
    from mxq import matmul
    size, sched, ar_args = case
    K, M, N = shape
    rng = np.random.default_rng(size * 31 + K)
    PA, XA = _codes(rng, K, M)
    PB, XB = _codes(rng, K, N, scale=0.02)
    ar, orc = _arith(*ar_args)
    got = matmul.adder_tree(*_t(PA, XA, PB, XB), ar, sched, size).cpu().numpy()
    want = ot.adder_tree(PA, XA, PB, XB, orc, sched, size)
    assert_bits_equal(got, want, f"adder {size} {ar_args} {shape}")


ANCHOR_CASES = [
    # size, width, schedule, bits, drop, headroom, emin, arithmetic
    (16, None, None, None, "truncate", None, None, ("MXGEMMINI",)),
    (16, 4, [(4, 4), (4, 5), (4, 6), (8, 7)], None, "rne", None, None, ("MXGEMMINI",)),
    (8, 2, [(4, 4)] * 4, [9, 7, 7], "truncate", 3, -6, ("MXGEMMINI",)),
    (16, 8, [(8, 7), (4, 6)], [12, 10, 10, 8, 8], "rne", 5, None, ("MXGEMMINI",)),
    (8, 1, [(4, 3)] * 8, [10, 6], "truncate", 2, None, ("MXGEMMINI",)),
    (32, 16, [(8, 7), (8, 7)], [16, 14, 12, 11, 11, 9], "truncate", 6, -3, ("MXGEMMINI",)),
    (32, None, None, None, "rne", None, None, ("MXGEMMINI", 4, 3, None)),
    (16, 16, [(6, 9)], [20] * 6, "truncate", 7, None, ("MXQUANT", 4, 3)),
    (4, 4, [(8, 23)], [24] * 4, "rne", 4, None, ("MXQUANT", 8, 23)),
]


@pytest.mark.parametrize("case", ANCHOR_CASES, ids=[f"a{i}" for i in range(len(ANCHOR_CASES))])
@pytest.mark.parametrize("shape", [(256, 40, 72), (45, 17, 33)])
def test_anchor_tree_against_oracle(cuda, case, shape):
    from mxq import matmul
    size, width, sched, bits, drop, head, emin, ar_args = case
    K, M, N = shape
    rng = np.random.default_rng(size * 7 + K)
    PA, XA = _codes(rng, K, M)
    PB, XB = _codes(rng, K, N, scale=0.3)
    PA[3:9, 1] = 0.0
    PB[20, :] *= np.float32(64.0)
    ar, orc = _arith(*ar_args)
    got = matmul.anchor_tree(*_t(PA, XA, PB, XB), ar, sched, size, width=width, bits=bits, drop=drop,
                             headroom=head, emin=emin).cpu().numpy()
    want = ot.anchor_tree(PA, XA, PB, XB, orc, sched, size, 32, width, bits, drop, head, emin)
    assert_bits_equal(got, want, f"anchor {case} {shape}")


def _wild(rng, K, n):
    """Codes off every grid: large (saturating), subnormal, specials; scales incl. non-powers of two."""
    P = (rng.standard_normal((K, n)) * np.exp2(rng.integers(-20, 12, (K, n)))).astype(np.float32)
    sp = special_f32()
    idx = rng.choice(P.size, size=min(P.size // 6, sp.size), replace=False)
    P.flat[idx] = sp[: idx.size]
    X = np.exp2(rng.integers(-8, 8, (-(-K // 32), n))).astype(np.float32)
    X[0, :2] = np.float32(0.3)
    return P, X


@pytest.mark.parametrize("which", ["adder", "anchor"])
@pytest.mark.parametrize("ar_args", [("MXGEMMINI",), ("MXQUANT", 4, 3)])
def test_trees_wild_codes(cuda, which, ar_args):
    """NaN, Inf, signed zeros, subnormals, saturating products: the trees' special-value paths."""
    from mxq import matmul
    rng = np.random.default_rng(17)
    K, M, N = 96, 24, 20
    PA, XA = _wild(rng, K, M)
    PB, XB = _wild(rng, K, N)
    ar, orc = _arith(*ar_args)
    if which == "adder":
        sched = [(4, 4), (4, 6), (5, 7), (8, 7)]
        got = matmul.adder_tree(*_t(PA, XA, PB, XB), ar, sched, 16).cpu().numpy()
        want = ot.adder_tree(PA, XA, PB, XB, orc, sched, 16)
    else:
        got = matmul.anchor_tree(*_t(PA, XA, PB, XB), ar, [(8, 7), (4, 6)], 16, width=8, drop="rne").cpu().numpy()
        want = ot.anchor_tree(PA, XA, PB, XB, orc, [(8, 7), (4, 6)], 16, 32, 8, None, "rne")
    assert_bits_equal(got, want, f"{which} wild {ar_args}")


def test_trees_callable_arithmetic_and_scheme(cuda):
    """An Arithmetic without a kernel description runs the reference's loop with its callables: same bits as
    the kernel; a Scheme swaps the reducers in reduce=."""
    from mxq import Scheme, block, matmul
    from mxq.matmul import Arithmetic
    rng = np.random.default_rng(3)
    PA, XA = _codes(rng, 64, 12)
    PB, XB = _codes(rng, 64, 10)
    ops = _t(PA, XA, PB, XB)
    hw = matmul.MXGEMMINI()
    hand = Arithmetic(name="hand", product=hw.product, acc_add=hw.acc_add, tile_add=hw.tile_add)
    sched = [(4, 4), (4, 5), (4, 6), (8, 7)]
    assert torch.equal(matmul.adder_tree(*ops, hand, sched), matmul.adder_tree(*ops, hw, sched))
    kw = dict(width=8, bits=[14, 12, 12, 10, 10], drop="rne", headroom=5, emin=-5)
    assert torch.equal(matmul.anchor_tree(*ops, hand, None, 16, **kw), matmul.anchor_tree(*ops, hw, None, 16, **kw))
    q = partial(block.mxgemmini.quantize, fmt="MXFP8_E4M3", axis=0)
    s = Scheme("anchor", a=q, b=q, reduce=partial(matmul.anchor_tree, arith=hw, width=4))
    A = torch.randn(64, 12, generator=torch.Generator().manual_seed(0)).cuda()
    B = torch.randn(64, 10, generator=torch.Generator().manual_seed(1)).cuda()
    Y = s.matmul(A, B).cpu().numpy()
    PA2, XA2 = ob.mxgemmini_quantize(A.cpu().numpy(), "MXFP8_E4M3", 0)
    PB2, XB2 = ob.mxgemmini_quantize(B.cpu().numpy(), "MXFP8_E4M3", 0)
    assert_bits_equal(Y, ot.anchor_tree(PA2, XA2, PB2, XB2, nx.MXGEMMINI(), None, 16, 32, 4), "scheme anchor")


def test_trees_empty_and_zero_k(cuda):
    from mxq import matmul
    hw = matmul.MXGEMMINI()
    z = lambda *s: torch.zeros(*s, device="cuda")                                      # noqa: E731
    for fn in (lambda *o: matmul.adder_tree(*o, hw, [(8, 7)] * 4), lambda *o: matmul.anchor_tree(*o, hw)):
        Y = fn(z(0, 5), z(0, 5), z(0, 7), z(0, 7))
        assert Y.shape == (5, 7) and torch.equal(Y, z(5, 7))
        assert fn(z(64, 0), z(2, 0), z(64, 7), z(2, 7)).shape == (0, 7)


# ------------------------------------------------------------------------------------ fast kernels
def _launches(kernel, fn):
    """Runs fn with the library's kernel timer on; returns (fn's result, launches of `kernel`)."""
    from mxq import _lib
    torch.cuda.synchronize()
    _lib.timer_read(kernel)
    _lib.timer_enable(True)
    try:
        out = fn()
    finally:
        _lib.timer_enable(False)
    return out, _lib.timer_read(kernel)[1]


def _edge_columns(n, w=48):
    """Column slices checked against the oracle: the first and last w columns (every tile position kind)."""
    return [slice(0, min(w, n)), slice(max(0, n - w), n)]


ADDER_FAST = [
    (16, [(4, 4), (4, 5), (4, 6), (8, 7)], ("MXGEMMINI",)),
    (16, [(8, 7)] * 4, ("MXGEMMINI",)),
    (4, [(4, 3), (8, 7)], ("MXGEMMINI",)),
    (8, [(4, 4), (4, 4), (4, 7)], ("MXGEMMINI",)),
    (32, [(4, 4), (4, 5), (4, 6), (8, 7), (8, 7)], ("MXGEMMINI",)),
    (16, [(4, 4), (4, 5), (4, 6), (8, 7)], ("MXGEMMINI", 4, 3, None)),
    (16, [(4, 6), (4, 6), (4, 9), (4, 9)], ("MXGEMMINI",)),
]


@pytest.mark.parametrize("case", ADDER_FAST, ids=[f"af{i}" for i in range(len(ADDER_FAST))])
@pytest.mark.parametrize("shape", [(256, 136, 200), (77, 40, 70), (64, 2944, 2944)])
def test_adder_fast_kernel(cuda, case, shape):
    """The fast adder kernel on its own configurations: every output equal to the general kernel's, and the
    oracle's on edge column slices (columns are independent chains); 2944 x 2944 takes the 64 x 64 tiles."""
    from mxq import matmul
    size, sched, ar_args = case
    K, M, N = shape
    rng = np.random.default_rng(size * 13 + K + M)
    PA, XA = _codes(rng, K, M)
    PB, XB = _codes(rng, K, N, scale=0.02)
    ar, orc = _arith(*ar_args)
    ops = _t(PA, XA, PB, XB)
    got, n = _launches("adder_fast", lambda: matmul.adder_tree(*ops, ar, sched, size))
    assert n == 1, "the fast adder kernel did not run"
    gen = matmul.adder_tree(*ops, ar, sched, size, force_general=True)
    assert_bits_equal(got.cpu().numpy(), gen.cpu().numpy(), f"adder fast vs general {case} {shape}")
    got = got.cpu().numpy()
    for cs in _edge_columns(N):
        want = ot.adder_tree(PA, XA, PB[:, cs], XB[:, cs], orc, sched, size)
        assert_bits_equal(got[:, cs], want, f"adder fast vs oracle {case} {shape} {cs}")


ANCHOR_FAST = [
    # size, width, drop, headroom, bits, arithmetic
    (16, None, "truncate", None, None, ("MXGEMMINI",)),
    (16, 8, "truncate", None, None, ("MXGEMMINI",)),
    (16, 4, "rne", None, None, ("MXGEMMINI",)),
    (32, None, "rne", None, None, ("MXGEMMINI", 4, 3, None)),
    (32, 16, "truncate", 7, [18] * 6, ("MXGEMMINI",)),
    (8, 8, "rne", 5, [12] * 5, ("MXGEMMINI", 4, 3, -20)),
]


@pytest.mark.parametrize("case", ANCHOR_FAST, ids=[f"nf{i}" for i in range(len(ANCHOR_FAST))])
@pytest.mark.parametrize("shape", [(256, 136, 200), (45, 40, 70), (64, 2944, 2944)])
def test_anchor_fast_kernel(cuda, case, shape):
    """The fast anchor kernel on its own configurations, against the general kernel everywhere and the oracle
    on edge column slices.  Zero codes (a zero column, zero K rows) and a row of small codes, whose trees have
    anchors too low for the fast path, send some tiles to the general kernel."""
    from mxq import matmul
    size, width, drop, head, bits, ar_args = case
    K, M, N = shape
    rng = np.random.default_rng(size * 5 + K + M)
    PA, XA = _codes(rng, K, M)
    PB, XB = _codes(rng, K, N, scale=0.3)
    PA[:, 3] = 0.0
    PA[min(5, K - 1), :] = 0.0
    PA[:, 7] *= np.float32(2.0 ** -14)
    ar, orc = _arith(*ar_args)
    ops = _t(PA, XA, PB, XB)
    kw = dict(width=width, bits=bits, drop=drop, headroom=head)
    got, n = _launches("anchor_fast", lambda: matmul.anchor_tree(*ops, ar, None, size, **kw))
    assert n == 1, "the fast anchor kernel did not run"
    gen = matmul.anchor_tree(*ops, ar, None, size, force_general=True, **kw)
    assert_bits_equal(got.cpu().numpy(), gen.cpu().numpy(), f"anchor fast vs general {case} {shape}")
    got = got.cpu().numpy()
    for cs in _edge_columns(N):
        want = ot.anchor_tree(PA, XA, PB[:, cs], XB[:, cs], orc, None, size, 32, width, bits, drop, head)
        assert_bits_equal(got[:, cs], want, f"anchor fast vs oracle {case} {shape} {cs}")


@pytest.mark.parametrize("which", ["adder", "anchor"])
def test_trees_fast_kernel_falls_back(cuda, which):
    """Tiles whose codes the fast kernels cannot take (overflowing e4 levels, saturating products, Inf, NaN,
    tiny anchors) are computed by the general kernel: the result equals the general kernel's alone."""
    from mxq import matmul
    rng = np.random.default_rng(23)
    K, M, N = 96, 130, 140
    PA, XA = _codes(rng, K, M)
    PB, XB = _codes(rng, K, N)
    PA[:, 70:] *= np.float32(64.0)            # products up to 256: beyond the e4 levels' bound
    PB[10, 100] = np.inf
    PB[40, 30] = np.nan
    PA[:, 1] *= np.float32(2.0 ** -40)
    XB[1, 5] = np.float32(0.3)
    hw = matmul.MXGEMMINI()
    ops = _t(PA, XA, PB, XB)
    if which == "adder":
        sched = [(4, 4), (4, 5), (4, 6), (8, 7)]
        fn = lambda fg: matmul.adder_tree(*ops, hw, sched, force_general=fg)        # noqa: E731
        want = ot.adder_tree(PA, XA, PB, XB, nx.MXGEMMINI(), sched)
    else:
        fn = lambda fg: matmul.anchor_tree(*ops, hw, force_general=fg)              # noqa: E731
        want = ot.anchor_tree(PA, XA, PB, XB, nx.MXGEMMINI())
    got, n = _launches(f"{which}_fast", lambda: fn(False))
    assert n == 1
    assert_bits_equal(got.cpu().numpy(), fn(True).cpu().numpy(), f"{which} fallback vs general")
    assert_bits_equal(got.cpu().numpy(), want, f"{which} fallback vs oracle")


def _golden_tree_cases():
    import json
    import os
    z = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "trees.npz"), allow_pickle=False)
    return z, [tuple(c) for c in json.loads(str(z["cases"]))]


@pytest.mark.parametrize("case", _golden_tree_cases()[1], ids=lambda c: c[0])
def test_trees_against_reference_fixtures(cuda, case):
    """Both reducers on the GPU against the reference's own outputs (tests/golden/trees.npz), bit for bit."""
    from mxq import matmul
    z, _ = _golden_tree_cases()
    name, tree, (aname, aargs), fmt, K, M, N, kw = case
    ops = _t(*(z[f"{name}_{k}"] for k in ("PA", "XA", "PB", "XB")))
    ar = getattr(matmul, aname)(*aargs)
    kw = dict(kw)
    if "schedule" in kw:
        kw["schedule"] = [tuple(x) for x in kw["schedule"]]
    if tree == "anchor":
        Y = matmul.anchor_tree(*ops, ar, **kw)
    else:
        Y = matmul.adder_tree(*ops, ar, kw.pop("schedule"), **kw)
    assert_bits_equal(Y.cpu().numpy(), z[f"{name}_Y"], f"{tree} tree {name}")
