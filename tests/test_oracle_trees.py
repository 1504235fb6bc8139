"""Pins of the oracle's adder and anchor trees (oracle/trees.py), CPU only.

  * exact-rational scalar models (oracle/brute.py), one output at a time, on MXGEMMINI with K tails, every
    adder size, anchor widths 1-16, both drops, custom level widths that fall (so the pairing order and the
    odd term's pass-up change bits), headroom, emin, and running sums that set the anchor;
  * textbook reductions: an MXQUANT(8, 23) adder tree is a pairwise float32 sum of the exact products; an
    anchor tree whose terms all sit on its grid returns the exact sum rounded once;
  * invariants: columns are independent; an all-zero K block leaves C unchanged.
"""
import numpy as np
import pytest

from oracle import block as ob
from oracle import brute
from oracle import numerics as nx
from oracle import trees


def _codes(rng, K, n, scale=1.0, fmt="MXFP8_E4M3"):
    V = (rng.standard_normal((K, n)) * scale).astype(np.float32)
    return ob.mxgemmini_quantize(V, fmt, 0, 32, "rne", 2.0 ** -23)


def _bits_eq(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32), np.asarray(b, np.float32).view(np.uint32))


@pytest.mark.parametrize("size,sched", [(2, [(4, 4)]), (4, [(4, 3), (8, 7)]), (8, [(4, 4), (4, 6), (8, 7)]),
                                        (16, [(8, 7)] * 4), (32, [(4, 5), (4, 5), (4, 6), (4, 6), (8, 7)])])
def test_adder_tree_against_scalar_model(size, sched):
    rng = np.random.default_rng(size)
    K = 77 if size <= 16 else 70                     # K tails that end mid-reduction
    PA, XA = _codes(rng, K, 3)
    PB, XB = _codes(rng, K, 4, 0.3)
    got = trees.adder_tree(PA, XA, PB, XB, nx.MXGEMMINI(), sched, size)
    assert _bits_eq(got, brute.adder_tree_mxgemmini(PA, XA, PB, XB, sched, size))


ANCHOR_CASES = [
    # size, width, schedule, bits, drop, headroom, emin
    (16, 16, None, None, "truncate", None, None),
    (16, 4, [(4, 4), (4, 5), (4, 6), (8, 7)], None, "rne", None, None),
    (8, 2, [(4, 4)] * 4, [9, 7, 7], "truncate", 3, -6),
    (16, 8, [(8, 7), (4, 6)], [12, 10, 10, 8, 8], "rne", 5, None),
    (8, 1, [(4, 3)] * 8, [10, 6], "truncate", 2, None),
    (32, 16, [(8, 7), (8, 7)], [16, 14, 12, 11, 11, 9], "truncate", 6, -3),
]


@pytest.mark.parametrize("case", ANCHOR_CASES, ids=[f"a{i}" for i in range(len(ANCHOR_CASES))])
def test_anchor_tree_against_scalar_model(case):
    size, width, sched, bits, drop, head, emin = case
    rng = np.random.default_rng(size * 3 + width)
    K = 45
    PA, XA = _codes(rng, K, 3)
    PB, XB = _codes(rng, K, 4, 0.3)
    PA[3:9, 1] = 0.0                                   # zero products never set the anchor
    PB[20, :] *= np.float32(64.0)                      # one large product per output: c sets later anchors
    sch = [(8, 7)] * (size // width) if sched is None else sched
    hd = trees.default_headroom(width) if head is None else head
    bits_of = (lambda m: trees.default_bits(m, width, hd)) if bits is None else (lambda m: bits)
    got = trees.anchor_tree(PA, XA, PB, XB, nx.MXGEMMINI(), sched, size, 32, width, bits, drop, head, emin)
    want = brute.anchor_tree_mxgemmini(PA, XA, PB, XB, sch, size, width, bits_of, drop, hd, emin)
    assert _bits_eq(got, want)


def test_anchor_tree_truncation_is_active():
    """With narrow levels the tree's result differs from the exactly rounded sum, so the models above see
    the dropping, not a sum that happens to be exact."""
    rng = np.random.default_rng(9)
    PA, XA = _codes(rng, 64, 8)
    PB, XB = _codes(rng, 64, 8)
    narrow = trees.anchor_tree(PA, XA, PB, XB, nx.MXQUANT(8, 23), [(8, 23)], 16, 32, 16, [10] * 6, "truncate", 4)
    wide = trees.anchor_tree(PA, XA, PB, XB, nx.MXQUANT(8, 23), [(8, 23)], 16, 32, 16, [24] * 6, "truncate", 4)
    assert not np.array_equal(narrow, wide)


def test_adder_tree_mxquant_fp32_is_pairwise_sum():
    rng = np.random.default_rng(2)
    K, M, N = 96, 5, 6
    PA, XA = _codes(rng, K, M)
    PB, XB = _codes(rng, K, N)
    got = trees.adder_tree(PA, XA, PB, XB, nx.MXQUANT(8, 23), [(8, 23)] * 4, 16)
    C = np.zeros((M, N), np.float32)
    for g in range(0, K, 32):
        sc = (XA[g // 32][:, None] * XB[g // 32][None, :]).astype(np.float32)
        for k0 in range(g, g + 32, 16):
            v = [(PA[k][:, None] * PB[k][None, :]).astype(np.float32) for k in range(k0, k0 + 16)]
            while len(v) > 1:
                v = [(v[i] + v[i + 1]).astype(np.float32) for i in range(0, len(v), 2)]
            C = (C + (v[0] * sc).astype(np.float32)).astype(np.float32)
    assert _bits_eq(got, C)


def test_anchor_tree_on_grid_is_exact_sum():
    """Small integer codes: every term is a multiple of the grid step, the levels lose nothing, and each tree
    returns the exact sum of its products and c (float32-exact here)."""
    rng = np.random.default_rng(4)
    K, M, N = 64, 4, 5
    PA = rng.integers(-8, 9, (K, M)).astype(np.float32)
    PB = rng.integers(-8, 9, (K, N)).astype(np.float32)
    X = np.ones((K // 32, M), np.float32), np.ones((K // 32, N), np.float32)
    got = trees.anchor_tree(PA, X[0], PB, X[1], nx.MXQUANT(8, 23), [(8, 23)] * 4, 16, 32, 4, [24] * 4,
                            "truncate", 4)
    assert _bits_eq(got, (PA.astype(np.float64).T @ PB.astype(np.float64)).astype(np.float32))


@pytest.mark.parametrize("which", ["adder", "anchor"])
def test_tree_invariants(which):
    rng = np.random.default_rng(6)
    K, M, N = 64, 4, 9
    PA, XA = _codes(rng, K, M)
    PB, XB = _codes(rng, K, N)
    ar = nx.MXGEMMINI()

    def run(pa, xa, pb, xb):
        if which == "adder":
            return trees.adder_tree(pa, xa, pb, xb, ar, [(4, 4), (4, 5), (4, 6), (8, 7)], 16)
        return trees.anchor_tree(pa, xa, pb, xb, ar, [(8, 7)] * 2, 16, 32, 8)

    full = run(PA, XA, PB, XB)
    assert _bits_eq(full[:, 3:7], run(PA, XA, PB[:, 3:7], XB[:, 3:7]))
    PA0 = np.vstack([PA, np.zeros((32, M), np.float32)])
    PB0 = np.vstack([PB, np.zeros((32, N), np.float32)])
    XA0 = np.vstack([XA, np.ones((1, M), np.float32)])
    XB0 = np.vstack([XB, np.ones((1, N), np.float32)])
    assert _bits_eq(full, run(PA0, XA0, PB0, XB0))
