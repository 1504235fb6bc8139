"""mxq.packed on the GPU: one-pass quantize to code and E8M0 bytes, pack / unpack / dequantize, and 4-bit LUT
indices, bit for bit against the oracle (oracle/packed.py over oracle/block.py's quantizers)."""
import numpy as np
import pytest
import torch

from _util import assert_bits_equal
from oracle import block as ob
from oracle import lut as ol
from oracle import packed as op

pytestmark = pytest.mark.gpu

FMTS = sorted(op.FORMATS)


def _oracle(method, V, fmt, axis, bs, **kw):
    if method == "mxgemmini":
        return ob.mxgemmini_quantize(V, fmt, axis, bs, kw.get("rounding_mode", "ties_away"),
                                     kw.get("scale_floor", 1e-38))
    if method == "ocp":
        return ob.ocp_quantize(V, fmt, axis, bs, kw.get("rounding_mode", "even"), 8, kw.get("placement", "top"))
    return ob.mxquant_quantize(V, fmt, axis, bs)


# (shape, axis, block size, input dtype): the split kernel with 4-wide and 1-wide columns and a tail block,
# the contiguous-block kernel, the strided kernel
LAYOUTS = [((4100, 72), 0, 32, torch.float32), ((3, 70, 33), 1, 32, torch.bfloat16),
           ((64, 96), 1, 32, torch.float16), ((100, 40), 0, 16, torch.float32)]


def _input(rng, shape, dtype):
    V = rng.standard_normal(shape).astype(np.float32) * np.float32(3.0)
    flat = V.reshape(-1)
    flat[: flat.size // 50] = 0.0                       # some all-zero blocks (the 1e-38 floor's scale)
    return torch.from_numpy(V).to(dtype)


@pytest.mark.parametrize("method,opts", [("mxgemmini", {}), ("mxgemmini", {"rounding_mode": "rne",
                                                                           "scale_floor": 2.0 ** -23}),
                                         ("ocp", {}), ("ocp", {"placement": "below_top"}), ("mxquant", {})],
                         ids=["mxg", "mxg_hw", "ocp", "ocp_bt", "mxquant"])
@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("layout", range(len(LAYOUTS)))
def test_quantize_packed_against_oracle(cuda, method, opts, fmt, layout):
    import mxq
    shape, axis, bs, dt = LAYOUTS[layout]
    rng = np.random.default_rng(layout * 31 + len(fmt))
    V = _input(rng, shape, dt)
    P, X = _oracle(method, V.float().numpy(), fmt, axis, bs, **opts)
    want_c, want_s, err = op.pack(P, X, fmt, axis, bs)
    codes, scales = mxq.packed.quantize(V.cuda(), fmt, method, axis, bs, check=False, **opts)
    _, c_ok = op.encode(P, *op.FORMATS[fmt])
    assert np.array_equal(codes.cpu().numpy()[c_ok], want_c[c_ok]), f"codes {method} {fmt} {LAYOUTS[layout]}"
    assert np.array_equal(scales.cpu().numpy(), want_s), f"scales {method} {fmt} {LAYOUTS[layout]}"
    if err:
        assert method == "mxquant", "only the qtorch grid has codes some byte formats lack"
        with pytest.raises(ValueError, match="not a"):
            mxq.packed.quantize(V.cuda(), fmt, method, axis, bs, **opts)
    else:
        assert np.array_equal(codes.cpu().numpy(), want_c)


@pytest.mark.parametrize("fmt", FMTS)
def test_pack_unpack_dequantize(cuda, fmt):
    """The GPU's own block.mxgemmini output packs to the oracle's bytes and to the one-pass quantize's bytes;
    unpack gives P back and X back outside all-zero blocks (2^-127 there); dequantize of the bytes equals
    block.dequantize of (P, X) bit for bit."""
    import mxq
    rng = np.random.default_rng(7)
    V = _input(rng, (200, 130), torch.float32).cuda()
    P, X = mxq.block.mxgemmini.quantize(V, fmt, axis=0)
    codes, scales = mxq.packed.pack(P, X, fmt)
    want_c, want_s, err = op.pack(P.cpu().numpy(), X.cpu().numpy(), fmt)
    assert err == 0
    assert np.array_equal(codes.cpu().numpy(), want_c) and np.array_equal(scales.cpu().numpy(), want_s)
    qc, qs = mxq.packed.quantize(V, fmt)
    assert torch.equal(qc, codes) and torch.equal(qs, scales)
    P2, X2 = mxq.packed.unpack(codes, scales, fmt)
    assert_bits_equal(P2.cpu().numpy(), P.cpu().numpy(), "unpack P")
    zero = X2 != X
    assert (X[zero] == np.float32(1e-38)).all() and (X2[zero] == 2.0 ** -127).all()
    d = mxq.packed.dequantize(codes, scales, fmt)
    assert_bits_equal(d.cpu().numpy(), mxq.block.mxgemmini.dequantize(P, X).cpu().numpy(), "dequantize")


def test_packed_specials_and_errors(cuda):
    """NaN codes: E4M3 and E5M2 have them, FP6 and FP4 raise; a non-power-of-two scale of a nonzero block
    raises; mxquant's smallest E4M3 qtorch values are no OCP E4M3 codes; check=False returns the bytes."""
    import mxq
    V = torch.randn(64, 8).cuda()
    V[3, 2] = float("nan")
    for fmt in ("MXFP8_E4M3", "MXFP8_E5M2"):
        codes, scales = mxq.packed.quantize(V, fmt)
        assert int(scales[0, 2]) == 0xFF and int(codes[3, 2]) & 0x7F == 0x7F
    for fmt in ("MXFP6_E3M2", "MXFP6_E2M3", "MXFP4"):
        with pytest.raises(ValueError, match="not a"):
            mxq.packed.quantize(V, fmt)
    W = torch.full((32, 4), 1e-4, device="cuda")
    with pytest.raises(ValueError, match="E8M0"):
        mxq.packed.quantize(W, "MXFP8_E4M3", scale_floor=3e-3)
    T = torch.tensor([[2.0 ** -7 * 1.125] + [1.0] * 31], device="cuda").t().contiguous()
    with pytest.raises(ValueError, match="not a MXFP8_E4M3 value"):
        mxq.packed.quantize(T, "MXFP8_E4M3", "mxquant")
    codes, _ = mxq.packed.quantize(T, "MXFP8_E4M3", "mxquant", check=False)
    assert codes.shape == T.shape
    with pytest.raises(ValueError, match="FP32"):
        mxq.packed.quantize(V, "FP32")
    with pytest.raises(ValueError, match="method"):
        mxq.packed.quantize(V, "MXFP4", "lut")
    with pytest.raises(TypeError, match="option"):
        mxq.packed.quantize(V, "MXFP4", "mxquant", rounding_mode="rne")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("fmt", FMTS)
def test_quantize_packed_rne_kernel(cuda, dtype, fmt):
    """block.mxgemmini rne bytes with inner % 8 == 0 (the one-pass kernel for the OCP grid at nearest even):
    eight lanes per block column with partial waves and tail blocks against the oracle everywhere; four lanes
    (4128 x 2048) against pack() of the float32 quantizer everywhere and the oracle on the columns around the
    planted values; both floors (1e-38 divides, 2^-23 is a power of two), waves with NaN, Inf, huge, subnormal
    and all-zero blocks (the software path)."""
    import mxq
    rng = np.random.default_rng(len(fmt) * 7 + {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2}[dtype])
    for shape, axis in [((4100, 136), 0), ((3, 70, 40), 1), ((4128, 2048), 0)]:
        V = rng.standard_normal(shape).astype(np.float32) * np.float32(2.0)
        flat = V.reshape(-1)
        sp = [np.nan, np.inf, -np.inf, 6.0e4, 2.0 ** -140, -0.0]
        at = rng.choice(flat.size, len(sp), replace=False)
        flat[at] = sp
        if axis == 0:
            V[64:96, 16:24] = 0.0                                    # all-zero blocks in one lane's columns
        Vt = torch.from_numpy(V).to(dtype)
        Vd = Vt.cuda()
        for floor in (1e-38, 2.0 ** -23):
            codes, scales = mxq.packed.quantize(Vd, fmt, "mxgemmini", axis, 32, check=False,
                                                rounding_mode="rne", scale_floor=floor)
            got_c, got_s = codes.cpu().numpy(), scales.cpu().numpy()
            if V.size <= 600_000:
                P, X = ob.mxgemmini_quantize(Vt.float().numpy(), fmt, axis, 32, "rne", floor)
                want_c, want_s, _ = op.pack(P, X, fmt, axis, 32)
                _, c_ok = op.encode(P, *op.FORMATS[fmt])
                assert np.array_equal(got_c[c_ok], want_c[c_ok]), f"codes {dtype} {fmt} {shape} floor {floor}"
                assert np.array_equal(got_s, want_s), f"scales {dtype} {fmt} {shape} floor {floor}"
                continue
            P, X = mxq.block.mxgemmini.quantize(Vd, fmt, axis=axis, rounding_mode="rne", scale_floor=floor)
            _, c_ok = op.encode(P.cpu().numpy(), *op.FORMATS[fmt])
            pc, ps = mxq.packed.pack(P, X, fmt, axis, 32, check=False)
            assert np.array_equal(got_c[c_ok], pc.cpu().numpy()[c_ok]), f"codes {dtype} {fmt} {shape} floor {floor}"
            assert np.array_equal(got_s, ps.cpu().numpy()), f"scales {dtype} {fmt} {shape} floor {floor}"
            for col in sorted({int(a) % shape[1] for a in at} | {20}):
                cols = slice(col - col % 8, col - col % 8 + 8)
                Po, Xo = ob.mxgemmini_quantize(Vt[:, cols].float().numpy(), fmt, 0, 32, "rne", floor)
                wc, ws, _ = op.pack(Po, Xo, fmt)
                _, ok = op.encode(Po, *op.FORMATS[fmt])
                assert np.array_equal(got_c[:, cols][ok], wc[ok]), f"codes {dtype} {fmt} cols {cols} floor {floor}"
                assert np.array_equal(got_s[:, cols], ws), f"scales {dtype} {fmt} cols {cols} floor {floor}"


@pytest.mark.parametrize("n,group,width", [(40, 0, 16), (41, 1, 16), (7, 0, 5)])
def test_pick_lookup_packed(cuda, n, group, width):
    """Nibbles equal lut.pick's int64 indices packed two to a byte; lookup of them equals lut.lookup."""
    import mxq
    rng = np.random.default_rng(n)
    P, _ = ob.mxgemmini_quantize(rng.standard_normal((96, n)).astype(np.float32), "MXFP6_E3M2", 0)
    ng = -(-n // (1 << group))
    if width == 16:
        T = ol.tables(P, "MXFP6_E3M2", group, 10)
    else:
        safe = ol.tables_of("MXFP6_E3M2")[2]
        T = np.sort(rng.choice(safe, (ng, width), replace=True), axis=1).astype(np.float32)
    I = ol.pick(P, T, group)
    Pc, Tc = torch.from_numpy(P).cuda(), torch.from_numpy(np.ascontiguousarray(T)).cuda()
    I4 = mxq.packed.pick(Pc, Tc, group=group)
    assert np.array_equal(I4.cpu().numpy(), op.pack_indices(I))
    got = mxq.packed.lookup(I4, Tc, group=group, n=n)
    assert_bits_equal(got.cpu().numpy(), ol.lookup(I, T, group), "lookup")


@pytest.fixture(scope="module")
def c3_input(cuda):
    """bf16 8192 x 8192: Student-t (3 degrees of freedom) times 0.5, 0.1% of entries times 100, seeded."""
    g = torch.Generator().manual_seed(11)
    torch.manual_seed(11)
    t = torch.distributions.StudentT(torch.tensor(3.0)).sample((8192, 8192)) * 0.5
    idx = torch.randperm(8192 * 8192, generator=g)[:67109]
    t.view(-1)[idx] *= 100
    return t.to(torch.bfloat16).cuda()


@pytest.mark.parametrize("fmt", FMTS)
def test_quantize_packed_full_size_c3(c3_input, fmt):
    """rne on the bf16 8192 x 8192 input: the one-pass bytes equal pack() of block.mxgemmini's own float32 output
    over every element, and the oracle's bytes on the first and last 64 columns."""
    import mxq
    V = c3_input
    codes, scales = mxq.packed.quantize(V, fmt, rounding_mode="rne")
    P, X = mxq.block.mxgemmini.quantize(V, fmt, axis=0, rounding_mode="rne")
    pc, ps = mxq.packed.pack(P, X, fmt)
    assert torch.equal(codes, pc) and torch.equal(scales, ps)
    del P, X, pc, ps
    for cols in (slice(0, 64), slice(8192 - 64, 8192)):
        Vs = V[:, cols].float().cpu().numpy()
        Po, Xo = ob.mxgemmini_quantize(Vs, fmt, 0, 32, "rne")
        wc, ws, err = op.pack(Po, Xo, fmt)
        assert err == 0
        assert np.array_equal(codes[:, cols].cpu().numpy(), wc), f"{fmt} codes {cols}"
        assert np.array_equal(scales[:, cols].cpu().numpy(), ws), f"{fmt} scales {cols}"
