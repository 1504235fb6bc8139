"""Block quantization and the elementwise primitives on the GPU, bit for bit against the oracle."""
import numpy as np
import pytest
import torch

from _util import assert_bits_equal, random_f32, special_f32
from oracle import block as ob
from oracle import numerics as nx

pytestmark = pytest.mark.gpu

FMTS = list(nx.FORMATS)


def _edge_matrix(rng, rows, cols, scale=1.0):
    V = (rng.standard_normal((rows, cols)) * scale).astype(np.float32)
    sp = special_f32()
    idx = rng.choice(V.size, size=min(sp.size, V.size // 4), replace=False)
    V.flat[idx] = sp[: idx.size]
    if rows >= 40 and cols >= 3:
        V[0:32, 1] = 0.0                                   # an all-zero block
        V[0:32, 2] = np.float32(2.0 ** -130)               # a subnormal block
    return V


def _run(fn, V, *args, **kw):
    import mxq
    P, X = fn(torch.from_numpy(V).cuda(), *args, **kw)
    return P.cpu().numpy(), X.cpu().numpy()


@pytest.mark.parametrize("fmt", FMTS + ["FP32"])
def test_mxquant(cuda, fmt):
    from mxq import block
    rng = np.random.default_rng(1)
    for shape, axis, bs in [((4096, 512), 0, 32), ((4100, 64), 0, 32), ((64, 4100), 1, 32), ((96, 8, 5), 1, 32),
                            ((100, 33), 0, 7), ((128, 128), -1, 16)]:
        V = _edge_matrix(rng, shape[0], int(np.prod(shape[1:]))).reshape(shape)
        P, X = _run(block.mxquant.quantize, V, fmt, axis=axis, block_size=bs)
        wP, wX = ob.mxquant_quantize(V, fmt, axis, bs)
        assert_bits_equal(P, wP, f"P {fmt} {shape} {axis} {bs}")
        assert_bits_equal(X, wX, f"X {fmt} {shape} {axis} {bs}")


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("mode", ["ties_away", "rne", "truncate"])
def test_mxgemmini(cuda, fmt, mode):
    from mxq import block
    rng = np.random.default_rng(2)
    for shape, axis, bs, floor, via in [((4096, 512), 0, 32, 1e-38, None), ((4100, 96), 0, 32, 2.0 ** -23, None),
                                        ((64, 4096), 1, 32, 1e-38, (3, 1)), ((50, 30), 0, 3, 2.0 ** -23, (5, 4))]:
        V = _edge_matrix(rng, shape[0], shape[1], scale=float(np.exp2(rng.integers(-20, 20))))
        P, X = _run(block.mxgemmini.quantize, V, fmt, axis=axis, block_size=bs, rounding_mode=mode,
                    scale_floor=floor, via=via)
        wP, wX = ob.mxgemmini_quantize(V, fmt, axis, bs, mode, floor, via)
        assert_bits_equal(P, wP, f"P {fmt} {mode} {shape}")
        assert_bits_equal(X, wX, f"X {fmt} {mode} {shape}")


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("placement", ["top", "below_top", "no_clip"])
def test_ocp(cuda, fmt, placement):
    from mxq import block
    rng = np.random.default_rng(3)
    for mode in ("even", "nearest", "floor"):
        for shape, axis in [((4096, 512), 0), ((4100, 40), 0), ((40, 4100), 1)]:
            V = _edge_matrix(rng, shape[0], shape[1], scale=float(np.exp2(rng.integers(-30, 30))))
            P, X = _run(block.ocp.quantize, V, fmt, axis=axis, rounding_mode=mode, placement=placement)
            wP, wX = ob.ocp_quantize(V, fmt, axis, 32, mode, 8, placement)
            assert_bits_equal(P, wP, f"P {fmt} {mode} {placement} {shape}")
            assert_bits_equal(X, wX, f"X {fmt} {mode} {placement} {shape}")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float64])
def test_low_precision_inputs(cuda, dtype):
    from mxq import block
    rng = np.random.default_rng(4)
    for shape in ((512, 256), (100, 260), (70, 24)):            # 8, 4 and 8 columns per lane; short last block
        V = torch.from_numpy(_edge_matrix(rng, *shape) * 3).to(dtype)
        V32 = V.to(torch.float32).numpy()
        for fmt in FMTS:
            P, X = block.mxgemmini.quantize(V.cuda(), fmt, axis=0, rounding_mode="rne")
            wP, wX = ob.mxgemmini_quantize(V32, fmt, 0, 32, "rne")
            assert_bits_equal(P.cpu().numpy(), wP, f"P {dtype} {fmt} {shape}")
            assert_bits_equal(X.cpu().numpy(), wX, f"X {dtype} {fmt} {shape}")
        P, X = block.ocp.quantize(V.cuda(), "MXFP8_E4M3", axis=0)
        wP, wX = ob.ocp_quantize(V32, "MXFP8_E4M3", 0)
        assert_bits_equal(P.cpu().numpy(), wP, f"ocp P {dtype} {shape}")
        P, X = block.mxquant.quantize(V.cuda(), "MXFP6_E3M2", axis=0, block_size=16)
        wP, wX = ob.mxquant_quantize(V32, "MXFP6_E3M2", 0, 16)
        assert_bits_equal(P.cpu().numpy(), wP, f"mxquant bs16 P {dtype} {shape}")


def test_contiguous_block_layout(cuda):
    """axis = last with 32 | n runs the eight-lanes-per-block kernel; odd n runs the strided one."""
    from mxq import block
    rng = np.random.default_rng(5)
    for shape in [(300, 256), (7, 3, 64), (33, 100)]:
        V = _edge_matrix(rng, shape[0], int(np.prod(shape[1:]))).reshape(shape)
        for fn, ref in [(block.mxgemmini.quantize, ob.mxgemmini_quantize), (block.ocp.quantize, ob.ocp_quantize),
                        (block.mxquant.quantize, ob.mxquant_quantize)]:
            P, X = _run(fn, V, "MXFP8_E4M3", axis=-1)
            wP, wX = ref(V, "MXFP8_E4M3", -1)
            assert_bits_equal(P, wP, f"P {shape} {fn.__module__}")
            assert_bits_equal(X, wX, f"X {shape} {fn.__module__}")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_transposed_view_layout(cuda, dtype):
    """Axis 0 of a transposed view (V = M.t(), M row-major) runs the transposing kernel on M as it lies: the same
    codes and scales as the oracle on V, for every rule; tiles cut by both edges, n and inner off multiples of 4
    and of 32 (scalar loads and stores), and the aligned whole-tile path."""
    from mxq import block
    rng = np.random.default_rng(9)
    quantizers = [(block.mxgemmini.quantize, lambda V, f: ob.mxgemmini_quantize(V, f, 0, 32, "rne"),
                   dict(rounding_mode="rne")),
                  (block.mxgemmini.quantize, lambda V, f: ob.mxgemmini_quantize(V, f, 0, 32, "truncate", 2.0 ** -23),
                   dict(rounding_mode="truncate", scale_floor=2.0 ** -23)),
                  (block.mxquant.quantize, lambda V, f: ob.mxquant_quantize(V, f, 0, 32), {}),
                  (block.ocp.quantize, lambda V, f: ob.ocp_quantize(V, f, 0, 32, "nearest", 8, "top"),
                   dict(rounding_mode="nearest"))]
    for n, inner in [(2048, 256), (192, 128), (100, 70), (33, 130), (64, 3), (7, 65)]:
        M = torch.from_numpy(_edge_matrix(rng, inner, n, scale=float(np.exp2(rng.integers(-10, 10))))).to(dtype)
        V32 = M.to(torch.float32).numpy().T.copy()
        Md = M.cuda()
        for fn, ref, kw in quantizers:
            for fmt in ("MXFP8_E4M3", "MXFP4", "MXFP6_E2M3"):
                P, X = fn(Md.t(), fmt, axis=0, **kw)
                wP, wX = ref(V32, fmt)
                assert_bits_equal(P.cpu().numpy(), wP, f"P {dtype} {n}x{inner} {fmt} {kw}")
                assert_bits_equal(X.cpu().numpy(), wX, f"X {dtype} {n}x{inner} {fmt} {kw}")
                assert P.is_contiguous() and P.shape == (n, inner) and X.shape == (-(-n // 32), inner)


def test_contiguous_views_with_length_one_axes(cuda):
    """Contiguous views whose length-one axes carry strides other than a fresh tensor's (torch ignores those
    strides when it calls a view contiguous): every axis of each, the same codes and scales as the oracle."""
    from mxq import block
    rng = np.random.default_rng(12)
    base = torch.from_numpy(_edge_matrix(rng, 40, 70)).cuda()
    views = [base[:, :33][:1], base[:1, :64].unsqueeze(1), base.t()[:, :1], base.t()[:, 3:4].unsqueeze(0)]
    for V in views:
        assert V.is_contiguous()
        V32 = V.cpu().numpy().copy()
        for axis in range(V.ndim):
            P, X = block.mxgemmini.quantize(V, "MXFP8_E4M3", axis=axis)
            wP, wX = ob.mxgemmini_quantize(V32, "MXFP8_E4M3", axis)
            assert_bits_equal(P.cpu().numpy(), wP, f"P {tuple(V.shape)} {V.stride()} axis {axis}")
            assert_bits_equal(X.cpu().numpy(), wX, f"X {tuple(V.shape)} {V.stride()} axis {axis}")


def test_cpu_tensors_round_trip_through_gpu(cuda):
    from mxq import block
    V = torch.randn(64, 8)
    P, X = block.mxgemmini.quantize(V, "MXFP4", axis=0)
    assert P.device.type == "cpu" and X.device.type == "cpu"
    wP, wX = ob.mxgemmini_quantize(V.numpy(), "MXFP4", 0)
    assert_bits_equal(P.numpy(), wP, "P")
    assert_bits_equal(X.numpy(), wX, "X")


def test_dequantize(cuda):
    from mxq import block
    rng = np.random.default_rng(6)
    V = _edge_matrix(rng, 4100, 64)
    P, X = block.ocp.quantize(torch.from_numpy(V).cuda(), "MXFP6_E3M2", axis=0)
    got = block.dequantize(P, X, axis=0).cpu().numpy()
    assert_bits_equal(got, ob.dequantize(P.cpu().numpy(), X.cpu().numpy(), 0), "dequantize axis 0")
    P2, X2 = block.mxgemmini.quantize(torch.from_numpy(V).cuda(), "MXFP8_E5M2", axis=1, block_size=5)
    got2 = block.mxgemmini.dequantize(P2, X2, axis=1, block_size=5).cpu().numpy()
    assert_bits_equal(got2, ob.dequantize(P2.cpu().numpy(), X2.cpu().numpy(), 1, 5), "dequantize axis 1")
    # every vector width of the flat kernel (inner a multiple of 4, of 2 only, odd), 3-D views, tails
    for shape, axis, bs in [((4096, 512), 0, 32), ((3, 70, 6), 1, 32), ((5, 33, 7), 1, 16), ((2, 9, 40), -1, 32)]:
        W = _edge_matrix(rng, shape[0], int(np.prod(shape[1:]))).reshape(shape)
        P3, X3 = block.mxquant.quantize(torch.from_numpy(W).cuda(), "MXFP8_E4M3", axis=axis, block_size=bs)
        got3 = block.dequantize(P3, X3, axis=axis, block_size=bs).cpu().numpy()
        assert_bits_equal(got3, ob.dequantize(P3.cpu().numpy(), X3.cpu().numpy(), axis, bs), f"dequantize {shape}")


# ------------------------------------------------------------------------------------------ elementwise
@pytest.fixture(scope="module")
def corpus():
    rng = np.random.default_rng(11)
    return np.concatenate([special_f32(), random_f32(rng, 200000, -40, 40), random_f32(rng, 50000, -149, 128)])


def test_elementwise_rounding(cuda, corpus):
    from mxq import rounding
    x = torch.from_numpy(corpus).cuda()
    assert_bits_equal(rounding.bf16(x).cpu().numpy(), nx.bf16(corpus), "bf16")
    b = torch.from_numpy(nx.bits_of(corpus)).cuda()
    for keep in (0, 3, 7, 22):
        for mode in ("ties_away", "rne", "truncate"):
            got = rounding.round_bits(b, keep, mode).cpu().numpy()
            assert_bits_equal(got, nx.round_bits(nx.bits_of(corpus), keep, mode), f"round_bits {keep} {mode}")
    k = (corpus * np.float32(3.5)).astype(np.float32)
    for mode in ("ties_away", "rne", "truncate"):
        assert_bits_equal(rounding.round_int(torch.from_numpy(k).cuda(), mode).cpu().numpy(),
                          nx.round_int(k, mode), f"round_int {mode}")


def test_elementwise_float_em(cuda, corpus):
    from mxq.element_quant import float_em, microsoft
    x = torch.from_numpy(corpus).cuda()
    for grid, pairs in [("qtorch", [(4, 3), (8, 7), (6, 9)]), ("ieee", [(4, 4), (8, 7), (8, 22), (5, 10)]),
                        ("ocp", [(4, 3), (2, 1), (3, 2)])]:
        for e, m in pairs:
            for mode in ("ties_away", "rne", "truncate"):
                got = float_em.quantize(x, e, m, mode, grid).cpu().numpy()
                assert_bits_equal(got, nx.float_em(corpus, e, m, mode, grid), f"{grid} e{e}m{m} {mode}")
    x64 = torch.from_numpy(corpus.astype(np.float64) * 1.000001).cuda()
    got = float_em.quantize(x64, 8, 7, "rne", "ieee").cpu().numpy()
    assert_bits_equal(got, nx.float_em(corpus.astype(np.float64) * 1.000001, 8, 7, "rne", "ieee"), "f64 ieee")
    for fmt in FMTS:
        for mode in ("even", "nearest", "floor"):
            got = microsoft.quantize(x, fmt, mode).cpu().numpy()
            assert_bits_equal(got, nx.microsoft_fmt(corpus, fmt, mode), f"microsoft {fmt} {mode}")


def test_elementwise_scale_and_arith(cuda, corpus):
    from mxq import arith, scale_factor
    a = np.abs(corpus)
    at = torch.from_numpy(a).cuda()
    assert_bits_equal(scale_factor.mxquant(at).cpu().numpy(), nx.scale_mxquant(a), "mxquant")
    assert_bits_equal(scale_factor.mxquant(at, 2.0 ** -23).cpu().numpy(), nx.scale_mxquant(a, 2.0 ** -23), "mxquant hw")
    assert_bits_equal(scale_factor.ocp(at, 8).cpu().numpy(), nx.scale_ocp(a, 8), "ocp")
    assert_bits_equal(scale_factor.ocp_below_top(at, 4).cpu().numpy(), nx.scale_ocp_below_top(a, 4), "ocp_below_top")
    for fmt in FMTS:
        assert_bits_equal(scale_factor.ocp_no_clip(at, fmt).cpu().numpy(), nx.scale_ocp_no_clip(a, fmt), f"no_clip {fmt}")
    rng = np.random.default_rng(12)
    b = rng.permutation(corpus)
    bt = torch.from_numpy(b).cuda()
    x = torch.from_numpy(corpus).cuda()
    for e, m in [(4, 4), (4, 6), (7, 10), (8, 7), (8, 23)]:
        got = arith.exact_add(x, bt, e, m).cpu().numpy()
        assert_bits_equal(got, nx.exact_add(corpus, b, e, m), f"exact_add e{e}m{m}")
    assert_bits_equal(arith.truncate_significand(x, 3).cpu().numpy(), nx.truncate_significand(corpus, 3), "trunc")
    assert_bits_equal(arith.flush_product(x, -16).cpu().numpy(), nx.flush_product(corpus, -16), "flush")
    assert_bits_equal(arith.saturate(x, 448.0, 448.0).cpu().numpy(), nx.saturate(corpus, 448.0, 448.0), "sat")


def test_c3_full_size_column_slices(cuda):
    """The bf16 sweep at its full size, 8192 x 8192 (Student-t(3) x 0.5 with 0.1% of entries x 100): each
    format's whole GPU result, checked bit for bit against the oracle on the first and the last 64 columns at
    full height (axis-0 blocks keep columns independent), and the dequantized slice against P * X."""
    from mxq import block
    torch.manual_seed(2)
    t = torch.distributions.StudentT(torch.tensor(3.0)).sample((8192, 8192)) * 0.5
    idx = torch.randperm(8192 * 8192, generator=torch.Generator().manual_seed(2))[:67109]
    t.view(-1)[idx] *= 100
    V = t.to(torch.bfloat16)
    del t
    Vd = V.cuda()
    cols = [slice(0, 64), slice(8128, 8192)]
    V32 = [V[:, c].to(torch.float32).numpy() for c in cols]
    for fmt in FMTS:
        P, X = block.mxgemmini.quantize(Vd, fmt, axis=0, rounding_mode="rne")
        assert P.shape == (8192, 8192) and X.shape == (256, 8192)
        for c, v32 in zip(cols, V32):
            wP, wX = ob.mxgemmini_quantize(v32, fmt, 0, 32, "rne")
            assert_bits_equal(P[:, c].cpu().numpy(), wP, f"C3 P {fmt} {c}")
            assert_bits_equal(X[:, c].cpu().numpy(), wX, f"C3 X {fmt} {c}")
            D = block.mxgemmini.dequantize(P[:, c].contiguous(), X[:, c].contiguous(), axis=0).cpu().numpy()
            assert_bits_equal(D, ob.dequantize(wP, wX, 0), f"C3 dequantize {fmt} {c}")
        del P, X


def test_compose_with_callables(cuda):
    """block.compose with callables the fused kernel does not take (the reference's generic composition on the
    device): the library's own scale and element functions passed as callables, a user's torch pair, and each
    step left out, on 2-D and 3-D inputs with padded last blocks and negative axes, against the oracle's compose
    with the numpy twins."""
    from functools import partial

    from mxq import block, element_quant, scale_factor
    rng = np.random.default_rng(12)
    pairs = [
        (lambda a: scale_factor.mxquant(a), partial(element_quant.float_em.quantize, e=4, m=3, rounding_mode="rne",
                                                    grid="ocp"),
         lambda a: nx.scale_mxquant(a), lambda z: nx.float_em(z, 4, 3, "rne", "ocp")),
        (lambda a: torch.where(a > 0, a, torch.ones_like(a)), lambda z: torch.round(z * 16) / 16,
         lambda a: np.where(a > 0, a, np.float32(1)).astype(np.float32),
         lambda z: (np.round(z * np.float32(16)) / np.float32(16)).astype(np.float32)),
        (None, lambda z: torch.round(z * 4) / 4, None, lambda z: (np.round(z * np.float32(4)) / 4).astype(np.float32)),
        (lambda a: scale_factor.mxquant(a), None, lambda a: nx.scale_mxquant(a), None),
    ]
    for shape, axis, bs in [((100, 40), 0, 32), ((3, 70, 5), -2, 32), ((48, 33), -1, 16)]:
        V = (rng.standard_normal(shape) * 3).astype(np.float32)
        for ts, te, ns, ne in pairs:
            P, X = block.compose(torch.from_numpy(V).cuda(), scale=ts, elem=te, axis=axis, block_size=bs)
            assert P.device.type == "cuda" and P.is_contiguous() and X.is_contiguous()
            wP, wX = ob.compose(V, ns, ne, axis, bs)
            assert_bits_equal(P.cpu().numpy(), wP, f"compose P {shape} axis {axis}")
            assert_bits_equal(X.cpu().numpy(), wX, f"compose X {shape} axis {axis}")


def _grid_edge_input(fmt, seed):
    """K = 96 rows (three blocks) by 256 columns: every block's first row is 1.999 (the scale is 1, so the
    element grid sees the values as they are), the rest cycle through the format's grid values below 2, their
    midpoints (the ties), the float32 neighbours of those, both zeros and values that round to zero, with random
    signs.  Column 5 holds a NaN and column 9 an Inf in the first block, beside finite columns of the same waves."""
    from oracle import packed as op
    e, m = op.FORMATS[fmt]
    bias = (1 << (e - 1)) - 1
    grid = sorted({(mf / (1 << m)) * 2.0 ** (1 - bias) if ef == 0 else (1 + mf / (1 << m)) * 2.0 ** (ef - bias)
                   for ef in range(1 << e) for mf in range(1 << m)})
    grid = np.array([g for g in grid if g < 2.0], dtype=np.float64)
    mids = ((grid[:-1] + grid[1:]) / 2).astype(np.float32)
    pts = np.concatenate([grid.astype(np.float32), mids, np.nextafter(mids, np.float32(0)),
                          np.nextafter(mids, np.float32(4)), np.float32([0.0, -0.0, 1e-30, -1e-30, 2.0 ** -126])])
    rng = np.random.default_rng(seed)
    V = rng.choice(pts, size=(96, 256)).astype(np.float32)
    V *= np.where(rng.random(V.shape) < 0.5, np.float32(-1), np.float32(1))
    V[::32, :] = np.float32(1.999)
    V[7, 5] = np.nan
    V[3, 9] = np.inf
    return V


@pytest.mark.parametrize("fmt", ["MXFP8_E4M3", "MXFP8_E5M2", "MXFP6_E3M2", "MXFP6_E2M3", "MXFP4"])
def test_mxgemmini_rne_grid_edges(cuda, fmt):
    """mxgemmini at nearest even, which runs on the hardware conversions when a wave's values are finite and
    in range, on every tie, signed zero and subnormal step of the format: float32 codes against the oracle,
    and the one-pass code bytes against the oracle's encoding of them; the NaN and Inf blocks take the general
    path in the same launches."""
    import mxq
    from mxq import block
    from oracle import packed as op
    V = _grid_edge_input(fmt, 5)
    for dt in (torch.float32, torch.bfloat16):
        Vt = torch.from_numpy(V).to(dt)
        V32 = Vt.float().numpy()
        P, X = block.mxgemmini.quantize(Vt.cuda(), fmt, axis=0, rounding_mode="rne", scale_floor=2.0 ** -23)
        wP, wX = ob.mxgemmini_quantize(V32, fmt, 0, 32, "rne", 2.0 ** -23)
        assert_bits_equal(X.cpu().numpy(), wX, f"X {fmt} {dt}")
        assert_bits_equal(P.cpu().numpy(), wP, f"P {fmt} {dt}")
        finite = np.isfinite(V32).all(axis=0)
        Vf = torch.from_numpy(V32[:, finite]).to(dt).contiguous()
        codes, scales = mxq.packed.quantize(Vf.cuda(), fmt, "mxgemmini", 0, 32, rounding_mode="rne",
                                            scale_floor=2.0 ** -23)
        fP, fX = ob.mxgemmini_quantize(Vf.float().numpy(), fmt, 0, 32, "rne", 2.0 ** -23)
        want_c, want_s, err = op.pack(fP, fX, fmt, 0, 32)
        assert not err
        assert np.array_equal(codes.cpu().numpy(), want_c), f"codes {fmt} {dt}"
        assert np.array_equal(scales.cpu().numpy(), want_s), f"scales {fmt} {dt}"


def _ocp_edge_input(fmt, cols, seed):
    """K = 96 rows (three blocks) by `cols` columns for block.ocp: every block's first row is 1.999 * 2^emax
    (the OCP scale is then 1), the rest cycle through the format's grid, its ties and their float32 neighbours,
    values between max_norm and 2^(emax + 1) (which saturate), the float32 just below half the smallest
    subnormal step (which microxcaling's float32 rounding sends up a step), signed zeros and values that
    round to zero, with random signs.  Column 5 holds a NaN and column 9 an Inf in the first block; two
    elements hold the exceptional value, so that their waves, and only theirs, leave the conversions."""
    from oracle import packed as op
    e, m = op.FORMATS[fmt]
    bias = (1 << (e - 1)) - 1
    grid = sorted({(mf / (1 << m)) * 2.0 ** (1 - bias) if ef == 0 else (1 + mf / (1 << m)) * 2.0 ** (ef - bias)
                   for ef in range(1 << e) for mf in range(1 << m)})
    top = {"MXFP8_E4M3": 448.0, "MXFP8_E5M2": 57344.0, "MXFP6_E3M2": 28.0, "MXFP6_E2M3": 7.5, "MXFP4": 6.0}[fmt]
    emax = int(np.floor(np.log2(top)))
    grid = np.array([g for g in grid if g <= top], dtype=np.float64)
    mids = ((grid[:-1] + grid[1:]) / 2).astype(np.float32)
    over = np.linspace(top, 2.0 ** (emax + 1), 9)[1:-1].astype(np.float32)
    odd = np.nextafter(np.float32(grid[1] / 2), np.float32(0))
    pts = np.concatenate([grid.astype(np.float32), mids, np.nextafter(mids, np.float32(0)),
                          np.nextafter(mids, np.float32(1e9)), over, np.float32([0.0, -0.0, 1e-30])])
    rng = np.random.default_rng(seed)
    V = rng.choice(pts, size=(96, cols)).astype(np.float32)
    V *= np.where(rng.random(V.shape) < 0.5, np.float32(-1), np.float32(1))
    V[::32, :] = np.float32(1.999 * 2.0 ** emax)
    V[7, 5] = np.nan
    V[3, 9] = np.inf
    V[40, 20], V[70, cols - 3] = odd, -odd
    return V


@pytest.mark.parametrize("fmt", ["MXFP8_E4M3", "MXFP8_E5M2", "MXFP6_E3M2", "MXFP6_E2M3", "MXFP4"])
@pytest.mark.parametrize("cols", [256, 90112], ids=["row_a_lane", "four_rows_a_lane"])
def test_ocp_even_grid_edges(cuda, fmt, cols):
    """block.ocp at "even" (microxcaling's rule), which runs on the hardware conversions, clamped to max_norm,
    when a wave's values and scaled values are finite and none is the one value microxcaling rounds apart:
    every tie, saturating value, signed zero and subnormal step of the format against the oracle.  256 columns
    take one row a lane (4 values a lane: FP6 stays on the grid); 90112 take four rows a lane (16 values: FP6
    converts too).  The NaN, Inf and exceptional-value waves take the general path in the same launches."""
    from mxq import block
    V = _ocp_edge_input(fmt, cols, 11)
    P, X = block.ocp.quantize(torch.from_numpy(V).cuda(), fmt, axis=0, rounding_mode="even")
    wP, wX = ob.ocp_quantize(V, fmt, 0)
    assert_bits_equal(X.cpu().numpy(), wX, f"X {fmt}")
    assert_bits_equal(P.cpu().numpy(), wP, f"P {fmt}")


@pytest.mark.parametrize("elem", ["ocp", "microsoft"])
def test_c_abi_own_max_norm(cuda, elem):
    """A C caller's spec with a max_norm other than the format's own (the Python quantizers always pass the
    format's): E4M3 at nearest even, unscaled, saturating at 240, where the hardware conversions would saturate at
    448.  The kernel keeps such waves on the software grid: the grid clamped at 240 (OCP), and microxcaling's
    element step with max_norm 240, bit for bit; then the same values at the format's own 448 against the
    oracle's grids (the conversions' path)."""
    import ctypes

    from mxq import _lib
    rng = np.random.default_rng(17)
    V = (rng.standard_normal((64, 256)) * 150).astype(np.float32)
    V[3, :8] = [239.9, 240.0, 241.0, 300.0, -300.0, 447.0, 0.0, -0.0]
    Vd = torch.from_numpy(V).cuda()
    for max_norm in (240.0, 448.0):
        if elem == "ocp":
            spec = _lib.BlockSpec(scale_rule=_lib.SCALE_NONE, elem=_lib.ELEM_OCP, e=4, m=3, rounding=1,
                                  max_norm=max_norm)
            g = nx._ocp(V, 4, 3, "rne")
            want = np.where(np.abs(g) > max_norm, np.copysign(np.float32(max_norm), g), g).astype(np.float32)
        else:
            spec = _lib.BlockSpec(scale_rule=_lib.SCALE_NONE, elem=_lib.ELEM_MICROSOFT, e=4, m=5, rounding=1,
                                  max_norm=max_norm)
            want = nx.microsoft(V, 4, 5, max_norm, "even")
        P = torch.empty_like(Vd)
        X = torch.empty(2, 256, device="cuda")
        _lib.run("mxq_block_quantize", _lib.ptr(Vd), 0, _lib.ptr(P), _lib.ptr(X), 1, 64, 256, 32,
                 ctypes.byref(spec), _lib.stream(Vd.device))
        assert_bits_equal(P.cpu().numpy(), want, f"{elem} E4M3 codes saturating at {max_norm}")


@pytest.mark.parametrize("placement", ["top", "below_top", "no_clip"])
@pytest.mark.parametrize("on", ["cuda", "cpu"])
def test_ocp_dither(cuda, placement, on):
    """block.ocp with rounding_mode="dither" (mxq/microxcaling/elemwise.py:41-43): the uniforms are drawn as the
    reference draws them, on V's device (the GPU's or the CPU's default generator): for no_clip one per block
    maximum first, then one per element of the blocked, zero-padded tensor.  Reseeding and drawing the same
    tensors in that order gives the oracle the same draws: codes and scales bit for bit, every format, both
    layouts, tails."""
    from mxq import block
    rng = np.random.default_rng(23)
    for fmt in FMTS:
        for shape, axis, bs in [((100, 33), 0, 32), ((5, 70, 3), 1, 16)]:
            V = (rng.standard_normal(shape) * np.exp2(rng.integers(-8, 8, shape))).astype(np.float32)
            V.flat[:3] = [0.0, -0.0, 1e-40]
            torch.manual_seed(1234)
            P, X = block.ocp.quantize(torch.from_numpy(V).to(on), fmt, axis=axis, block_size=bs,
                                      rounding_mode="dither", placement=placement)
            assert P.device.type == on
            torch.manual_seed(1234)
            outer, n, inner = int(np.prod(shape[:axis])), shape[axis], int(np.prod(shape[axis + 1:]))
            nb = -(-n // bs)
            ua = torch.rand(outer * inner * nb, device=on) if placement == "no_clip" else None
            u = torch.rand(outer * inner * nb * bs, device=on)
            wP, wX = ob.ocp_quantize(V, fmt, axis, bs, "dither", 8, placement,
                                     draws=(None if ua is None else ua.cpu().numpy(), u.cpu().numpy()))
            assert_bits_equal(X.cpu().numpy(), wX, f"X {fmt} {shape} {placement} dither on {on}")
            assert_bits_equal(P.cpu().numpy(), wP, f"P {fmt} {shape} {placement} dither on {on}")


def test_microsoft_and_no_clip_dither(cuda):
    """element_quant.microsoft.quantize and scale_factor.ocp_no_clip with "dither": one draw per element (per
    maximum), torch.rand_like of the rounded tensor on its device; against the oracle given the same draws."""
    from mxq import scale_factor
    from mxq.element_quant import microsoft
    rng = np.random.default_rng(29)
    for fmt in FMTS:
        eb, mb, _, mn = nx.FORMATS[fmt][4]
        z = (rng.standard_normal((64, 48)) * np.exp2(rng.integers(-6, 4, (64, 48)))).astype(np.float32)
        zt = torch.from_numpy(z).cuda()
        torch.manual_seed(77)
        got = microsoft.quantize(zt, fmt, rounding_mode="dither").cpu().numpy()
        torch.manual_seed(77)
        u = torch.rand_like(zt).cpu().numpy()
        assert_bits_equal(got, nx.microsoft(z, eb, mb, mn, "dither", True, u), f"microsoft dither {fmt}")
        amax = np.abs(z).max(axis=1, keepdims=True)
        at = torch.from_numpy(amax).cuda()
        torch.manual_seed(78)
        X = scale_factor.ocp_no_clip(at, fmt, rounding_mode="dither").cpu().numpy()
        torch.manual_seed(78)
        ua = torch.rand_like(at).cpu().numpy()
        assert_bits_equal(X, nx.scale_ocp_no_clip(amax, fmt, "dither", 8, ua), f"ocp_no_clip dither {fmt}")
