"""The oracle against the fixtures the reference itself wrote (tests/golden/make_golden.py): the functions only
an import of the reference pins -- LUT tables, safe sets and finder, ocp_no_clip, microxcaling "even", the
composed systolic datapaths."""
import json
import os

import numpy as np
import pytest

from _util import assert_bits_equal
from oracle import block as ob
from oracle import lut as ol
from oracle import numerics as nx
from oracle import systolic as osys

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _load(name):
    return np.load(os.path.join(GOLDEN, name), allow_pickle=False)


@pytest.mark.parametrize("fmt", ol.FORMATS)
def test_lut_formats(fmt):
    z = _load(f"lut_{fmt}.npz")
    vals, _, safe = ol.tables_of(fmt)
    assert_bits_equal(safe, z["values"], f"values {fmt}")
    assert_bits_equal(vals[z["decode_codes"]], z["decode"], f"decode {fmt}")


@pytest.mark.parametrize("fmt", ol.FORMATS)
def test_lut_tables_pick_lookup_finder(fmt):
    z = _load(f"lut_{fmt}.npz")
    keys = sorted(k[:-2] for k in z.files if k.endswith("_T"))
    assert keys
    for key in keys:
        G = int(key.split("_g")[1].split("_")[0])
        iters = int(key.split("_i")[1])
        P = z[f"{key}_P"]
        T = ol.tables(P, fmt, G, iters)
        assert_bits_equal(T, z[f"{key}_T"], f"tables {fmt} {key}")
        I = ol.pick(P, T, G)
        assert np.array_equal(I, z[f"{key}_I"]), f"pick {fmt} {key}"
        assert_bits_equal(ol.lookup(I, T, G), z[f"{key}_L"], f"lookup {fmt} {key}")
        if f"{key}_codes" in z.files:
            F = ol.finder(z[f"{key}_codes"], T, fmt, G)
            assert np.array_equal(F, z[f"{key}_F"]), f"finder {fmt} {key}"


def test_block_lut():
    z = _load("blocklut.npz")
    for i, (fmt, G, axis) in enumerate([("MXFP6_E3M2", 1, 0), ("MXFP6_E2M3", 0, 1), ("MXFP8_E5M2", 2, 0),
                                        ("MXFP8_E4M3", 1, 1)]):
        P, X = ol.lut_quantize(z[f"c{i}_V"], fmt, axis, 32, "rne", 2.0 ** -23, G, 50)
        assert_bits_equal(P, z[f"c{i}_P"], f"block.lut P {fmt}")
        assert_bits_equal(X, z[f"c{i}_X"], f"block.lut X {fmt}")


def test_ocp_no_clip():
    z = _load("noclip.npz")
    for fmt in nx.FORMATS:
        for mode in ("even", "nearest", "floor"):
            assert_bits_equal(nx.scale_ocp_no_clip(z["amax"], fmt, mode), z[f"{fmt}_{mode}"], f"no_clip {fmt} {mode}")
        P, X = ob.ocp_quantize(z[f"{fmt}_V"], fmt, 0, 32, "even", 8, "no_clip")
        assert_bits_equal(P, z[f"{fmt}_P"], f"ocp no_clip P {fmt}")
        assert_bits_equal(X, z[f"{fmt}_X"], f"ocp no_clip X {fmt}")


def test_microsoft_even():
    z = _load("ms_even.npz")
    for fmt in nx.FORMATS:
        assert_bits_equal(nx.microsoft_fmt(z[f"{fmt}_z"], fmt, "even"), z[f"{fmt}_even"], f"microsoft even {fmt}")


def test_systolic_end_to_end():
    z = _load("systolic.npz")
    cases = [("hw", nx.MXGEMMINI(), osys.HW_FINAL, 16, 32), ("hw_tail", nx.MXGEMMINI(), osys.HW_FINAL, 16, 32),
             ("hw_e5m2", nx.MXGEMMINI(5, 2), osys.HW_FINAL, 16, 32),
             ("hw_noflush", nx.MXGEMMINI(4, 3, None), [(4, 3)] * 8 + [(8, 7)] * 8, 16, 32),
             ("mxquant", nx.MXQUANT(4, 3), osys.HW_FINAL, 16, 32),
             ("mxquant_e5m10", nx.MXQUANT(5, 10), [(6, 9)] * 16, 16, 32),
             ("fp32_lanes", nx.MXGEMMINI(), [(8, 23)] * 16, 16, 32),
             ("size8", nx.MXGEMMINI(), [(4, 4)] * 7 + [(8, 7)], 8, 32)]
    for name, ar, sched, size, bs in cases:
        Y = osys.systolic(z[f"{name}_PA"], z[f"{name}_XA"], z[f"{name}_PB"], z[f"{name}_XB"], ar, sched, size, bs)
        assert_bits_equal(Y, z[f"{name}_Y"], f"systolic {name}")


def _hw_side():
    from oracle import attend as oatt
    q = lambda V: ob.mxgemmini_quantize(V, "MXFP8_E4M3", 0)                       # noqa: E731
    return oatt.Side(q, q, lambda *ops: osys.systolic(*ops, nx.MXGEMMINI(), osys.HW_FINAL))


def _torch_cpu_softmax(S):
    import torch
    return torch.softmax(torch.from_numpy(np.ascontiguousarray(S)), dim=-1).numpy()


def attend_cases():
    z = _load("attend.npz")
    for i in range(len([k for k in z.files if k.endswith("_meta")])):
        B, H, Hkv, T, D, masked, chunk = (int(x) for x in z[f"c{i}_meta"])
        yield (i, z[f"c{i}_q"], z[f"c{i}_k"], z[f"c{i}_v"], z[f"c{i}_mask"] if masked else None, D ** -0.5,
               None if chunk < 0 else chunk, z[f"c{i}_o"])


@pytest.mark.parametrize("case", list(attend_cases()), ids=lambda c: f"c{c[0]}")
def test_attend(case):
    """The reference's attend (CPU softmax) on GQA, chunked, masked and unmasked shapes, bit for bit."""
    from oracle import attend as oatt
    i, q, k, v, mask, scale, chunk, o = case
    side = _hw_side()
    got = oatt.attend(q, k, v, mask, scale, side, side, _torch_cpu_softmax, chunk=chunk)
    assert_bits_equal(got, o, f"attend c{i}")


def _tree_cases():
    z = _load("trees.npz")
    return [tuple(c) for c in json.loads(str(z["cases"]))]


@pytest.mark.parametrize("case", _tree_cases(), ids=lambda c: c[0])
def test_trees(case):
    """oracle/trees.py against the reference's anchor_tree and adder_tree on the cases tests/golden/make_golden.py
    lists: widths 1-16, sizes 2-32, falling level widths, both drops, emin, headroom, MXGEMMINI and MXQUANT,
    four code formats, K tails, zero rows, columns and blocks."""
    from oracle import trees as otr
    name, tree, (aname, aargs), fmt, K, M, N, kw = case
    z = _load("trees.npz")
    ops = [z[f"{name}_{k}"] for k in ("PA", "XA", "PB", "XB")]
    ar = getattr(nx, aname)(*aargs)
    kw = dict(kw)
    if "schedule" in kw:
        kw["schedule"] = [tuple(x) for x in kw["schedule"]]
    if tree == "anchor":
        Y = otr.anchor_tree(*ops, ar, **kw)
    else:
        Y = otr.adder_tree(*ops, ar, kw.pop("schedule"), **kw)
    assert_bits_equal(Y, z[f"{name}_Y"], f"{tree} tree {name}")


def _cpu_exp(x):
    import torch
    return torch.exp(torch.from_numpy(np.ascontiguousarray(x))).numpy()


def _cpu_rowsum(x):
    import torch
    return torch.from_numpy(np.ascontiguousarray(x)).sum(-1, keepdim=True).numpy()


def _cpu_mean(x):
    import torch
    return torch.from_numpy(np.ascontiguousarray(x)).mean(-1, keepdim=True).numpy()


def _cpu_rsqrt(x):
    import torch
    return torch.rsqrt(torch.from_numpy(np.ascontiguousarray(x))).numpy()


def test_vector_bf16_softmax_and_rmsnorm():
    """oracle/vector.py against the reference's vector="bf16" softmax (with -inf and finfo.min scores) and its
    RMSNorm, rounded and not, on bf16 and float32 activations and weights, with torch's CPU exp, sum, mean and
    rsqrt as the reference calls them."""
    from oracle import vector as ov
    z = _load("vector.npz")
    assert_bits_equal(ov.softmax_bf16(z["softmax_S"], _cpu_exp, _cpu_rowsum), z["softmax_bf16"], "softmax bf16")
    for i in range(3):
        xd, wd = (str(d) for d in z[f"rms{i}_dtypes"])
        for prec in (None, "bf16"):
            y = ov.rmsnorm(z[f"rms{i}_x"], z[f"rms{i}_w"], 1e-6, prec, _cpu_mean, _cpu_rsqrt,
                           xd == "torch.bfloat16", wd == "torch.bfloat16")
            assert_bits_equal(y, z[f"rms{i}_{prec}"], f"rmsnorm {xd} x {wd} {prec}")


def test_vector_bf16_attend():
    """oracle/attend.py with vector="bf16" against the reference's attend on three shapes (GQA 2:1 causal, chunks
    of 16, batch 2 with no mask)."""
    from functools import partial

    from oracle import attend as oatt
    from oracle import vector as ov
    z = _load("vector.npz")
    q = lambda V: ob.mxgemmini_quantize(V, "MXFP8_E4M3", 0)                           # noqa: E731
    hw = oatt.Side(q, q, lambda *ops: osys.systolic(*ops, nx.MXGEMMINI(), osys.HW_FINAL))
    sm = partial(ov.softmax_bf16, exp=_cpu_exp, rowsum=_cpu_rowsum)
    for i in range(3):
        B, H, Hkv, T, D, masked, chunk = (int(x) for x in z[f"c{i}_meta"])
        o = oatt.attend(z[f"c{i}_q"], z[f"c{i}_k"], z[f"c{i}_v"], z[f"c{i}_mask"] if masked else None, D ** -0.5,
                        hw, hw, sm, chunk=None if chunk < 0 else chunk, vector="bf16")
        assert_bits_equal(o, z[f"c{i}_o"], f"attend vector bf16 c{i}")
