"""Pins of the packed-format oracle (oracle/packed.py) against the reference's own code tables, torch's float8
casts, the OCP spec's FP4 values and the format table's max_norm."""
import math
import os

import numpy as np
import pytest
import torch

from oracle import block as ob
from oracle import packed as op

GOLDEN_DIR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
GOLDEN = {"MXFP8_E4M3": "lut_MXFP8_E4M3", "MXFP8_E5M2": "lut_MXFP8_E5M2", "MXFP6_E3M2": "lut_MXFP6_E3M2",
          "MXFP6_E2M3": "lut_MXFP6_E2M3"}
MAX_NORM = {"MXFP8_E4M3": 448.0, "MXFP8_E5M2": 57344.0, "MXFP6_E3M2": 28.0, "MXFP6_E2M3": 7.5, "MXFP4": 6.0}


@pytest.mark.parametrize("fmt", sorted(GOLDEN))
def test_code_table_is_the_references(fmt):
    """Every code's value equals the reference's decode of it (tests/golden, written by the reference), except
    E4M3's 0x7F and 0xFF: MX-Gemmini's decoders read them as +-480, OCP as NaN."""
    d = np.load(os.path.join(GOLDEN_DIR, GOLDEN[fmt] + ".npz"), allow_pickle=False)
    e, m = op.FORMATS[fmt]
    codes, want = d["decode_codes"], d["decode"]
    got = op.decode(codes, e, m)
    keep = np.ones(codes.shape, dtype=bool)
    if fmt == "MXFP8_E4M3":
        keep &= (codes & 0x7F) != 0x7F
        assert np.array_equal(np.abs(want[~keep]), [480.0, 480.0]) and np.isnan(got[~keep]).all()
    same = (got.view(np.uint32) == want.view(np.uint32)) | (np.isnan(got) & np.isnan(want))
    assert same[keep].all()


@pytest.mark.parametrize("fmt,dt", [("MXFP8_E4M3", torch.float8_e4m3fn), ("MXFP8_E5M2", torch.float8_e5m2)])
def test_encode_matches_torch_float8(fmt, dt):
    """torch's float8 casts (OCP encodings, round to nearest even) of every finite value give its code."""
    e, m = op.FORMATS[fmt]
    vals = op.code_table(e, m)
    fin = np.isfinite(vals)
    codes, ok = op.encode(vals[fin], e, m)
    assert ok.all()
    want = torch.from_numpy(vals[fin]).to(dt).view(torch.uint8).numpy()
    assert np.array_equal(codes, want)


def test_fp4_values_and_max_norms():
    """OCP MX v1.0's FP4 (E2M1) values, and the largest finite value of each format is its max_norm."""
    e, m = op.FORMATS["MXFP4"]
    assert op.code_table(e, m)[:8].tolist() == [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0]
    for fmt, (e, m) in op.FORMATS.items():
        vals = op.code_table(e, m)
        assert float(np.nanmax(vals[np.isfinite(vals)])) == MAX_NORM[fmt], fmt


@pytest.mark.parametrize("fmt", sorted(op.FORMATS))
def test_encode_round_trips_and_rejects(fmt):
    """Every value encodes to a code that decodes to it; midpoints between neighbours, values past the range and
    specials the format lacks are rejected; -0 keeps its sign bit."""
    e, m = op.FORMATS[fmt]
    vals = op.code_table(e, m)
    fin = vals[np.isfinite(vals)]
    codes, ok = op.encode(fin, e, m)
    assert ok.all()
    assert np.array_equal(op.decode(codes, e, m).view(np.uint32), fin.view(np.uint32))
    pos = np.unique(fin[fin > 0])
    mids = ((pos[:-1].astype(np.float64) + pos[1:]) / 2).astype(np.float32)
    mids = mids[~np.isin(mids, pos)]
    assert not op.encode(mids, e, m)[1].any()
    beyond = np.array([MAX_NORM[fmt] * 2, -MAX_NORM[fmt] * 2, pos[0] / 2], dtype=np.float32)
    assert not op.encode(beyond, e, m)[1].any()
    c, ok = op.encode(np.array([-0.0, np.inf, np.nan], dtype=np.float32), e, m)
    assert c[0] == 1 << (e + m) and ok[0]
    assert ok[1] == (fmt == "MXFP8_E5M2") and ok[2] == (fmt in ("MXFP8_E4M3", "MXFP8_E5M2"))


def test_e8m0():
    k = np.arange(-127, 128)
    x = np.ldexp(np.ones(k.shape, dtype=np.float32), k).astype(np.float32)
    b, ok = op.e8m0_encode(x, False)
    assert ok.all() and np.array_equal(b, k + 127)
    assert np.array_equal(op.e8m0_decode(b).view(np.uint32), x.view(np.uint32))
    b, ok = op.e8m0_encode(np.array([np.nan, 1e-38, 3.0, 2.0 ** -128], dtype=np.float32), False)
    assert b[0] == 0xFF and ok.tolist() == [True, False, False, False]
    b, ok = op.e8m0_encode(np.array([1e-38], dtype=np.float32), True)
    assert ok.all() and b[0] == 0
    assert math.isnan(float(op.e8m0_decode(np.array([0xFF]))[0]))


@pytest.mark.parametrize("fmt", sorted(op.FORMATS))
def test_pack_of_quantized_blocks(fmt):
    """mxgemmini and ocp codes and scales all pack; an all-zero block's 1e-38 scale packs to 2^-127 and
    dequantizes to the same zeros; unpack gives the codes back."""
    rng = np.random.default_rng(4)
    V = rng.standard_normal((70, 12)).astype(np.float32)
    V[32:64, 3] = 0.0
    for P, X in (ob.mxgemmini_quantize(V, fmt, 0), ob.ocp_quantize(V, fmt, 0)):
        codes, scales, err = op.pack(P, X, fmt)
        assert err == 0
        P2, X2 = op.unpack(codes, scales, fmt)
        assert np.array_equal(P2.view(np.uint32), P.view(np.uint32))
        nb = X.shape[0]
        Pp = np.concatenate([P, np.zeros((nb * 32 - P.shape[0], P.shape[1]), np.float32)]).reshape(nb, 32, -1)
        zero = (np.abs(Pp) == 0).all(axis=1)
        assert np.array_equal(X2[~zero], X[~zero]) and (X2[zero] == np.float32(2.0 ** -127)).all()
        assert np.array_equal(ob.dequantize(P2, X2, 0).view(np.uint32), ob.dequantize(P, X, 0).view(np.uint32))
    P, X = ob.mxgemmini_quantize(V, fmt, 0)
    assert X[1, 3] == np.float32(1e-38) and op.pack(P, X, fmt)[1][1, 3] == 0


def test_pack_indices():
    rng = np.random.default_rng(2)
    for n in (1, 6, 7):
        I = rng.integers(0, 16, (5, n))
        B = op.pack_indices(I)
        assert B.shape == (5, (n + 1) // 2) and np.array_equal(op.unpack_indices(B, n), I)
        assert np.array_equal(B[:, 0] & 0xF, I[:, 0])
