"""mxq.lut and block.lut on the GPU: bit for bit against the reference's own fixtures and the oracle."""
import os

import numpy as np
import pytest
import torch

from _util import assert_bits_equal
from oracle import block as ob
from oracle import lut as ol

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.mark.parametrize("fmt", ol.FORMATS)
def test_lut_against_reference_fixtures(cuda, fmt):
    from mxq import lut
    z = np.load(os.path.join(GOLDEN, f"lut_{fmt}.npz"), allow_pickle=False)
    assert_bits_equal(lut.values(fmt).numpy(), z["values"], "values")
    assert_bits_equal(lut.decode(torch.from_numpy(z["decode_codes"]).cuda(), fmt).cpu().numpy(), z["decode"], "decode")
    for key in sorted(k[:-2] for k in z.files if k.endswith("_T")):
        G = int(key.split("_g")[1].split("_")[0])
        iters = int(key.split("_i")[1])
        P = torch.from_numpy(z[f"{key}_P"]).cuda()
        T = lut.tables(P, fmt, group=G, max_iters=iters)
        assert_bits_equal(T.cpu().numpy(), z[f"{key}_T"], f"tables {key}")
        I = lut.pick(P, T, group=G)
        assert np.array_equal(I.cpu().numpy(), z[f"{key}_I"]), f"pick {key}"
        assert_bits_equal(lut.lookup(I, T, group=G).cpu().numpy(), z[f"{key}_L"], f"lookup {key}")
        if f"{key}_codes" in z.files:
            F = lut.finder(torch.from_numpy(z[f"{key}_codes"]).cuda(), T, fmt, group=G)
            assert np.array_equal(F.cpu().numpy(), z[f"{key}_F"]), f"finder {key}"


def test_block_lut_against_reference_fixtures(cuda):
    from mxq import block
    z = np.load(os.path.join(GOLDEN, "blocklut.npz"), allow_pickle=False)
    for i, (fmt, G, axis) in enumerate([("MXFP6_E3M2", 1, 0), ("MXFP6_E2M3", 0, 1), ("MXFP8_E5M2", 2, 0),
                                        ("MXFP8_E4M3", 1, 1)]):
        P, X = block.lut.quantize(torch.from_numpy(z[f"c{i}_V"]).cuda(), fmt, axis, 32, rounding_mode="rne",
                                  scale_floor=2.0 ** -23, group=G, max_iters=50)
        assert_bits_equal(P.cpu().numpy(), z[f"c{i}_P"], f"block.lut P {fmt}")
        assert_bits_equal(X.cpu().numpy(), z[f"c{i}_X"], f"block.lut X {fmt}")


@pytest.mark.parametrize("fmt", ol.FORMATS)
def test_tables_pick_against_oracle(cuda, fmt):
    from mxq import lut
    rng = np.random.default_rng(ol.FORMATS.index(fmt))
    for shape, G, iters in [((512, 256), 1, 50), ((300, 97), 0, 50), ((64, 130), 2, 7), ((1, 5), 1, 50)]:
        V = (rng.standard_t(4, shape) * np.exp2(rng.integers(-3, 3, (1, shape[1])))).astype(np.float32)
        P, _ = ob.mxgemmini_quantize(V, fmt, 0, 32, "rne", 2.0 ** -23)
        T = lut.tables(torch.from_numpy(P).cuda(), fmt, group=G, max_iters=iters)
        wT = ol.tables(P, fmt, G, iters)
        assert_bits_equal(T.cpu().numpy(), wT, f"tables {shape} G{G}")
        I = lut.pick(torch.from_numpy(P).cuda(), T, group=G).cpu().numpy()
        assert np.array_equal(I, ol.pick(P, wT, G)), f"pick {shape}"


def test_tables_past_exact_sums(cuda):
    """lut.tables on E5M2 codes with 4 M codes in one group (4096 x 1024, group 10): past about 2.4 M codes of a
    format reaching 57344 in steps of 2^-16, float64 sums of count x value can round, so the k-means adds each
    cluster's bins in bin order (the reference's scatter_add order) instead of by prefix differences.  Tables and
    picks against the oracle (numpy's add.at, also in bin order); the input is checked to be past the bound."""
    from mxq import lut
    rng = np.random.default_rng(41)
    vals, _, _ = ol.tables_of("MXFP8_E5M2")
    grid = np.unique(vals[np.isfinite(vals)])
    K, n, G = 4096, 1024, 10
    P = grid[rng.integers(0, grid.size, (K, n))].astype(np.float32)
    P[rng.random((K, n)) < 0.6] = -57344.0
    assert K * n * 57344.0 / 2.0 ** -16 >= 2.0 ** 53
    T = lut.tables(torch.from_numpy(P).cuda(), "MXFP8_E5M2", group=G, max_iters=50)
    wT = ol.tables(P, "MXFP8_E5M2", G, 50)
    assert_bits_equal(T.cpu().numpy(), wT, "tables of one 4 M-code E5M2 group")


def test_c4_shape(cuda):
    """The LUT benchmark shape: block.lut MXFP6_E3M2 on 4096 x 4096, group 1, 50 iterations (2048 tables)."""
    from mxq import block
    g = torch.Generator().manual_seed(0)
    V = torch.randn(4096, 4096, generator=g)
    P, X = block.lut.quantize(V.cuda(), "MXFP6_E3M2", 0, 32, rounding_mode="rne", scale_floor=2.0 ** -23, group=1,
                              max_iters=50)
    wP, wX = ol.lut_quantize(V.numpy(), "MXFP6_E3M2", 0, 32, "rne", 2.0 ** -23, 1, 50)
    assert_bits_equal(X.cpu().numpy(), wX, "X")
    assert_bits_equal(P.cpu().numpy(), wP, "P_lut")


def test_c4_systolic_on_lut_operands(cuda):
    """The LUT benchmark's product: matmul.systolic MXGEMMINI HW_FINAL on two block.lut MXFP6_E3M2 operands of
    4096 x 4096 (seeds 0 and 1; K = M = N = 4096).  The second operand's codes and scales bit for bit against the
    oracle's quantizer (the first one's are test_c4_shape's), then the full GPU product against the oracle's
    reducer on the last 32 columns and on two rows over all 4096 columns (every output is its own chain)."""
    import _pool
    from mxq import block, matmul
    q = lambda V: block.lut.quantize(V, "MXFP6_E3M2", 0, 32, rounding_mode="rne", scale_floor=2.0 ** -23,  # noqa
                                     group=1, max_iters=50)
    A = torch.randn(4096, 4096, generator=torch.Generator().manual_seed(0))
    B = torch.randn(4096, 4096, generator=torch.Generator().manual_seed(1))
    PA, XA = q(A.cuda())
    PB, XB = q(B.cuda())
    Y = matmul.systolic(PA, XA, PB, XB, matmul.MXGEMMINI(), matmul.HW_FINAL).cpu().numpy()
    pa, xa, pb, xb = (t.cpu().numpy() for t in (PA, XA, PB, XB))
    wP, wX = ol.lut_quantize(B.numpy(), "MXFP6_E3M2", 0, 32, "rne", 2.0 ** -23, 1, 50)
    assert_bits_equal(xb, wX, "X_B")
    assert_bits_equal(pb, wP, "P_B")
    cols = slice(4064, 4096)
    assert_bits_equal(Y[:, cols], _pool.systolic(pa, xa, pb[:, cols], xb[:, cols]), "C4 last 32 columns")
    rows = [0, 2731]
    assert_bits_equal(Y[rows], _pool.systolic(pa[:, rows], xa[:, rows], pb, xb), "C4 two rows")


def test_lut_errors(cuda):
    from mxq import lut
    P = torch.tensor([[0.5, 0.3]], device="cuda")
    with pytest.raises(ValueError, match="not a MXFP6_E3M2 code"):
        lut.tables(P, "MXFP6_E3M2", group=0, max_iters=5)
    with pytest.raises(ValueError, match="not a LUT format"):
        lut.tables(P, "MXFP4", group=0, max_iters=5)
    with pytest.raises(ValueError, match="group"):
        lut.tables(P, "MXFP6_E3M2", group=-1, max_iters=5)
    with pytest.raises(ValueError, match="max_iters"):
        lut.tables(P, "MXFP6_E3M2", group=0, max_iters=-2)
    T = torch.zeros(3, 16, device="cuda")
    with pytest.raises(ValueError, match="tables"):
        lut.pick(torch.zeros(4, 4, device="cuda"), T, group=0)
    with pytest.raises(ValueError, match="need"):
        lut.finder(torch.zeros(4, 3, dtype=torch.int64, device="cuda"), torch.zeros(1, 16, device="cuda"), "MXFP6_E3M2",
                   group=1)


@pytest.mark.parametrize("fmt", ol.FORMATS)
def test_grid_index_matches_search(cuda, fmt):
    """The tables' histogram placing each code by its bits (grid index) against the same kernel searching the
    grid (the format passed as unknown): identical tables, and both the oracle's, on every code of the format
    (both zeros, subnormals, the largest, E4M3's 480) at group 0, 1 and 2.  The pick on values that are no code
    (and on every code) against the oracle, as entries and as int64 indices."""
    from mxq import _lib, lut
    from mxq.lut import formats as lf
    from mxq.lut import kmeans
    rng = np.random.default_rng(ol.FORMATS.index(fmt) + 40)
    vals = lf._tables(fmt)[0].numpy()
    codes = vals[np.isfinite(vals)]
    for G in (0, 1, 2):
        P = rng.choice(codes, size=(257, 64)).astype(np.float32)
        P[:, 5] = -0.0
        Pd = torch.from_numpy(P).cuda()
        T, err = kmeans.fit(Pd, fmt, G, 50)
        assert int(err.item()) == 0
        f = lf._format(fmt)
        g_d, s_d, o_d = kmeans._device_grid(f.name, Pd.device)
        ng, nv = T.shape[0], g_d.numel()
        T2 = torch.empty_like(T)
        work = torch.empty(ng * nv + 1, dtype=torch.int32, device="cuda")
        _lib.run("mxq_lut_tables", _lib.ptr(Pd), 257, 64, G, 50, _lib.ptr(g_d), nv, _lib.ptr(s_d), s_d.numel(),
                 _lib.ptr(o_d), 0, 0, _lib.ptr(T2), _lib.ptr(work), _lib.stream(Pd.device))
        assert_bits_equal(T2.cpu().numpy(), T.cpu().numpy(), f"tables by grid search {fmt} G{G}")
        assert_bits_equal(T.cpu().numpy(), ol.tables(P, fmt, G, 50), f"tables vs oracle {fmt} G{G}")
        Q = P.copy()
        Q[3, :7] = [0.3, -1e-30, 1e30, 0.0, -0.0, 2.0 ** -140, -7.7]
        Qd = torch.from_numpy(Q).cuda()
        Tn = T.cpu().numpy()
        want_i = ol.pick(Q, Tn, G)
        assert_bits_equal(kmeans.pick_values(Qd, T, group=G).cpu().numpy(), ol.lookup(want_i, Tn, G), "values")
        assert np.array_equal(lut.pick(Qd, T, group=G).cpu().numpy(), want_i), f"pick indices {fmt} G{G}"


def _steps(V, fmt, G, iters, mode, floor):
    """block.lut along axis 0 step by step: the float32 quantize kernel, the histogram and k-means kernels,
    the pick kernel (the path for shapes the one-call path does not take)."""
    from mxq import block
    from mxq.lut import kmeans
    P, X = block.mxgemmini.quantize(V, fmt, axis=0, rounding_mode=mode, scale_floor=floor)
    T, err = kmeans.fit(P, fmt, G, iters)
    assert int(err.item()) == 0
    return kmeans.pick_values(P, T, group=G), X


_FUSED_CASES = [  # (shape, group, input dtype, rounding, scale floor)
    ((100, 48), 0, torch.float32, "rne", 2.0 ** -23),
    ((4100, 144), 1, torch.float32, "rne", 2.0 ** -23),      # a tail block, a tile of 16 live columns
    ((1285, 16), 3, torch.bfloat16, "ties_away", 2.0 ** -23),  # two splits, the second shorter
    ((2048, 256), 1, torch.float16, "truncate", None),      # four splits of 16 blocks, two tiles
    ((1, 16), 1, torch.float32, "rne", None),
    ((96, 2048), 8, torch.float32, "ties_away", 2.0 ** -23),  # groups of two tiles
    ((33, 160), 5, torch.bfloat16, "rne", 2.0 ** -23),
    ((70, 4096), 12, torch.float32, "rne", 2.0 ** -23),      # one group over 32 tiles
]


@pytest.mark.parametrize("fmt", ol.FORMATS)
@pytest.mark.parametrize("case", range(len(_FUSED_CASES)))
def test_block_lut_one_call_against_steps(cuda, fmt, case):
    """block.lut's one-call path (mxq_block_lut: byte codes, fused counts, code-map pick) bit for bit against the
    step-by-step kernels on the same input: P (table entries) and X.  Shapes with tails, one and several splits,
    groups inside a tile and wider than one, all three input types and rounding modes; the FP8 formats at
    groups 0 and 1 take 32-column tiles."""
    from mxq import block
    from mxq.scale_factor import MXQUANT_FLOOR
    shape, G, dt, mode, floor = _FUSED_CASES[case]
    floor = MXQUANT_FLOOR if floor is None else floor
    g = torch.Generator().manual_seed(case * 10 + ol.FORMATS.index(fmt))
    V = (torch.randn(shape, generator=g) * torch.exp2(torch.randint(-6, 6, (1, shape[1]), generator=g).float()))
    V = V.to(dt).cuda()
    V[0, 0] = 0.0
    if shape[0] > 40:
        V[32:64, 1] = 0.0                                    # an all-zero block
        V[5, 2] = -0.0
    P, X = block.lut.quantize(V, fmt, 0, 32, rounding_mode=mode, scale_floor=floor, group=G, max_iters=50)
    wP, wX = _steps(V, fmt, G, 50, mode, floor)
    assert_bits_equal(X.cpu().numpy(), wX.cpu().numpy(), f"X {fmt} {shape} G{G}")
    assert_bits_equal(P.cpu().numpy(), wP.cpu().numpy(), f"P {fmt} {shape} G{G}")


@pytest.mark.parametrize("fmt", ol.FORMATS)
def test_block_lut_one_call_against_oracle(cuda, fmt):
    """The one-call path against the oracle's block.lut on a Student-t input with per-column scale spread
    (600 x 96, group 1, and 64 x 32, group 0, 7 iterations)."""
    from mxq import block
    rng = np.random.default_rng(70 + ol.FORMATS.index(fmt))
    for shape, G, iters in [((600, 96), 1, 50), ((64, 32), 0, 7)]:
        V = (rng.standard_t(4, shape) * np.exp2(rng.integers(-8, 8, (1, shape[1])))).astype(np.float32)
        P, X = block.lut.quantize(torch.from_numpy(V).cuda(), fmt, 0, 32, rounding_mode="rne",
                                  scale_floor=2.0 ** -23, group=G, max_iters=iters)
        wP, wX = ol.lut_quantize(V, fmt, 0, 32, "rne", 2.0 ** -23, G, iters)
        assert_bits_equal(X.cpu().numpy(), wX, f"X {fmt} {shape}")
        assert_bits_equal(P.cpu().numpy(), wP, f"P {fmt} {shape}")


@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16])
def test_block_lut_one_call_misaligned_view(cuda, dt):
    """A contiguous view at an element offset that is not a 16-byte boundary (a slice of a flat buffer, as flat
    parameter storage hands out) quantizes as a fresh copy of it does, on the one-call path."""
    from mxq import block
    K, n = 96, 64
    flat = torch.randn(K * n + 3, generator=torch.Generator().manual_seed(5)).to(dt).cuda()
    V = flat[1:1 + K * n].view(K, n)
    assert V.is_contiguous() and V.data_ptr() % 16
    kw = dict(rounding_mode="rne", scale_floor=2.0 ** -23, group=1, max_iters=50)
    P, X = block.lut.quantize(V, "MXFP6_E3M2", 0, 32, **kw)
    wP, wX = block.lut.quantize(V.clone(), "MXFP6_E3M2", 0, 32, **kw)
    assert_bits_equal(X.cpu().numpy(), wX.cpu().numpy(), f"X of a misaligned {dt} view")
    assert_bits_equal(P.cpu().numpy(), wP.cpu().numpy(), f"P of a misaligned {dt} view")


def test_block_lut_one_call_errors(cuda):
    """A non-finite V gives codes that are not values of the format: the one-call path raises what the tables
    raise (E3M2 has no NaN or Inf code: the encoder flags it; E5M2 has them: the count flags it), and the
    argument checks come in the step-by-step path's order."""
    from mxq import block
    V = torch.randn(64, 32, device="cuda")
    V[7, 3] = float("nan")
    for fmt in ("MXFP6_E3M2", "MXFP8_E5M2"):
        with pytest.raises(ValueError, match=f"not a {fmt} code"):
            block.lut.quantize(V, fmt, 0, 32, rounding_mode="rne", scale_floor=2.0 ** -23, group=1, max_iters=5)
    W = torch.randn(64, 32, device="cuda")
    W[9, 30] = float("inf")
    with pytest.raises(ValueError, match="not a MXFP8_E5M2 code"):
        block.lut.quantize(W, "MXFP8_E5M2", 0, 32, rounding_mode="rne", scale_floor=2.0 ** -23, group=1, max_iters=5)
    ok = torch.randn(64, 32, device="cuda")
    with pytest.raises(ValueError, match="group"):
        block.lut.quantize(ok, "MXFP6_E3M2", 0, 32, rounding_mode="rne", scale_floor=2.0 ** -23, group=-1,
                           max_iters=5)
    with pytest.raises(ValueError, match="max_iters"):
        block.lut.quantize(ok, "MXFP6_E3M2", 0, 32, rounding_mode="rne", scale_floor=2.0 ** -23, group=0,
                           max_iters=-1)
    with pytest.raises(ValueError):
        block.lut.quantize(ok, "MXFP6_E3M2", 0, 32, rounding_mode="nearest", scale_floor=2.0 ** -23, group=0,
                           max_iters=5)
