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
