"""The batched attention path's score kernel through the C ABI, bit for bit against the torch steps it replaces
(mxq/nn/_attention.py:128-135): `r(S * scale)`, `r(S + mask row)` with r the identity or rounding.bf16."""
import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu


def _scores(Z, n, m, Tk, seed):
    g = torch.Generator().manual_seed(seed)
    S = torch.randn(Z, n * m, Tk, generator=g) * 40
    S.view(-1)[:: 97] = float("inf")
    S.view(-1)[5:: 131] = float("nan")
    S.view(-1)[7:: 89] = -0.0
    S.view(-1)[11:: 53] = 3e38
    S.view(-1)[13:: 61] = 1e-40
    return S.cuda()


def _run(name, *args):
    from mxq import _lib
    _lib.run(name, *args)


@pytest.mark.parametrize("bf16", [0, 1])
@pytest.mark.parametrize("shape", [(3, 4, 5, 64), (2, 1, 7, 33), (1, 2, 3, 1), (5, 2, 2, 130)])
@pytest.mark.parametrize("mask_kind", ["none", "shared", "batched", "expanded"])
def test_scores_scale_mask(cuda, bf16, shape, mask_kind):
    from mxq import _lib
    Z, n, m, Tk = shape
    Hkv, z0, s0, Tq = 2, 3, 2, m + 4
    Bm = (z0 + Z - 1) // Hkv + 1
    S = _scores(Z, n, m, Tk, sum(shape) + bf16)
    g = torch.Generator().manual_seed(7)
    full = torch.randn(Bm, Tq, Tk, generator=g) * 8
    full[:, :, ::3] = torch.finfo(torch.float32).min
    full[:, :, 1::17] = float("-inf")
    if mask_kind == "shared":
        bias = full[:1].cuda()
    elif mask_kind == "batched":
        bias = full.cuda()
    elif mask_kind == "expanded":
        bias = full[:, :1].cuda().expand(Bm, Tq, Tk)
    else:
        bias = None
    scale = 0.08838834764831845
    from mxq import rounding
    r = rounding.bf16 if bf16 else (lambda x: x)
    want = r(S * scale)
    if bias is not None:
        b_of = [(z0 + z) // Hkv if bias.shape[0] > 1 else 0 for z in range(Z)]
        rows = torch.stack([bias[b, s0:s0 + m] for b in b_of])                      # Z x m x Tk
        want = r(want.view(Z, n, m, Tk) + rows[:, None]).view(Z, n * m, Tk)
    got = S.clone()
    mask = None
    b_stride = r_stride = 0
    if bias is not None:
        b0 = z0 // Hkv if bias.shape[0] > 1 else 0
        mask = bias[b0, s0]
        b_stride = bias.stride(0) if bias.shape[0] > 1 else 0
        r_stride = bias.stride(1)
    _run("mxq_scores_scale_mask", _lib.ptr(got), Z, n, m, Tk, ctypes.c_float(scale), _lib.ptr(mask), b_stride,
         r_stride, z0, Hkv, bf16, _lib.stream(got.device))
    assert torch.equal(got.view(torch.int32), want.view(torch.int32))


def test_glue_rejects(cuda):
    from mxq import _lib
    S = torch.zeros(4, device="cuda")
    with pytest.raises(RuntimeError, match="bad shape"):
        _run("mxq_scores_scale_mask", _lib.ptr(S), 1, 1, 1, 4, ctypes.c_float(1.0), None, 0, 0, 0, 0, 0,
             _lib.stream(S.device))
    _run("mxq_scores_scale_mask", _lib.ptr(S), 0, 1, 1, 4, ctypes.c_float(1.0), None, 0, 0, 0, 1, 0,
         _lib.stream(S.device))                                                       # empty: no launch
