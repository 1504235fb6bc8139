"""mxq.nn on the GPU: attend, MXLinear and patch with Schemes built from the gfx950 kernels.

attend: S and O bit for bit against oracle/attend.py run with the oracle's quantizers and systolic reducer and
with the same torch.softmax on the same GPU; and bit for bit against the reference's own outputs
(tests/golden/attend.npz, written with torch's CPU softmax): on these shapes the GPU's and the CPU's
torch.softmax give the same float32 probabilities, so the emulated outputs agree everywhere (measured: no
output differs), and any difference would come from one of the two softmax implementations.
"""
import math
import os
from functools import partial

import numpy as np
import pytest
import torch
from torch import nn

from _util import assert_bits_equal
from oracle import attend as oatt
from oracle import block as ob
from oracle import lut as ol
from oracle import numerics as nx
from oracle import systolic as osys

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _hw(mxq):
    from mxq import Scheme, block, matmul, schedule
    q = partial(block.mxgemmini.quantize, fmt="MXFP8_E4M3", axis=0)
    return Scheme("hw", a=q, b=q, reduce=partial(matmul.systolic, arith=matmul.MXGEMMINI(), schedule=schedule.HW_FINAL))


def _hw_oracle():
    q = lambda V: ob.mxgemmini_quantize(V, "MXFP8_E4M3", 0)                       # noqa: E731
    return oatt.Side(q, q, lambda *ops: osys.systolic(*ops, nx.MXGEMMINI(), osys.HW_FINAL))


def _lut(mxq):
    from mxq import Scheme, block, matmul, schedule
    a = partial(block.lut.quantize, fmt="MXFP6_E3M2", axis=0, block_size=32, rounding_mode="rne",
                scale_floor=2.0 ** -23, group=1, max_iters=50)
    b = partial(block.mxgemmini.quantize, fmt="MXFP8_E4M3", axis=0)
    return Scheme("lut", a=a, b=b, rows=2,
                  reduce=partial(matmul.systolic, arith=matmul.MXGEMMINI(), schedule=schedule.HW_FINAL))


def _lut_oracle():
    a = lambda V: ol.lut_quantize(V, "MXFP6_E3M2", 0, 32, "rne", 2.0 ** -23, 1, 50)  # noqa: E731
    b = lambda V: ob.mxgemmini_quantize(V, "MXFP8_E4M3", 0)                           # noqa: E731
    return oatt.Side(a, b, lambda *ops: osys.systolic(*ops, nx.MXGEMMINI(), osys.HW_FINAL), rows=2)


def _gpu_softmax(S):
    return torch.softmax(torch.from_numpy(np.ascontiguousarray(S)).cuda(), dim=-1).cpu().numpy()


def _causal(B, Tq, Tk):
    m = torch.triu(torch.full((Tq, Tk), torch.finfo(torch.float32).min), Tk - Tq + 1)
    return m[None, None].repeat(B, 1, 1, 1)


def _fixture_cases():
    z = np.load(os.path.join(GOLDEN, "attend.npz"), allow_pickle=False)
    for i in range(len([k for k in z.files if k.endswith("_meta")])):
        B, H, Hkv, T, D, masked, chunk = (int(x) for x in z[f"c{i}_meta"])
        yield (i, z[f"c{i}_q"], z[f"c{i}_k"], z[f"c{i}_v"], z[f"c{i}_mask"] if masked else None,
               None if chunk < 0 else chunk, z[f"c{i}_o"])


@pytest.mark.parametrize("case", list(_fixture_cases()), ids=lambda c: f"c{c[0]}")
def test_attend_fixture_shapes(cuda, case):
    import mxq
    i, q, k, v, mask, chunk, o_ref = case
    D = q.shape[-1]
    t = lambda a: None if a is None else torch.from_numpy(a).cuda()                   # noqa: E731
    got = mxq.nn.attend(t(q), t(k), t(v), t(mask), D ** -0.5, _hw(mxq), _hw(mxq), chunk=chunk).cpu().numpy()
    want = oatt.attend(q, k, v, mask, D ** -0.5, _hw_oracle(), _hw_oracle(), _gpu_softmax, chunk=chunk)
    assert_bits_equal(got, want, f"attend c{i} vs oracle")
    assert_bits_equal(got, o_ref, f"attend c{i} vs the reference's own outputs")


@pytest.mark.parametrize("case", [(1, 4, 1, 70, 32, 16, "hw"), (1, 2, 2, 66, 64, None, "lut"),
                                  (2, 2, 1, 40, 32, 8, "lut"), (1, 2, 2, 512, 128, None, "hw")],
                         ids=["gqa4_tails", "lut_rows2", "lut_chunks", "llama_head_512"])
def test_attend_against_oracle(cuda, case):
    import mxq
    B, H, Hkv, T, D, chunk, kind = case
    g = torch.Generator().manual_seed(11)
    q, k, v = (torch.randn(B, h, T, D, generator=g) for h in (H, Hkv, Hkv))
    mask = _causal(B, T, T)
    s, so = (_hw(mxq), _hw_oracle()) if kind == "hw" else (_lut(mxq), _lut_oracle())
    hw, hwo = _hw(mxq), _hw_oracle()
    got = mxq.nn.attend(q.cuda(), k.cuda(), v.cuda(), mask.cuda(), D ** -0.5, s, hw, chunk=chunk).cpu().numpy()
    want = oatt.attend(q.numpy(), k.numpy(), v.numpy(), mask.numpy(), D ** -0.5, so, hwo, _gpu_softmax, chunk=chunk)
    assert_bits_equal(got, want, f"attend {case}")


def _gpu_fn(fn):
    """A numpy -> numpy callable running the torch call fn on the GPU (the device under test's library op)."""
    return lambda x: fn(torch.from_numpy(np.ascontiguousarray(x)).cuda()).cpu().numpy()


GPU_EXP = _gpu_fn(torch.exp)
GPU_ROWSUM = _gpu_fn(lambda t: t.sum(-1, keepdim=True))
GPU_MEAN = _gpu_fn(lambda t: t.mean(-1, keepdim=True))
GPU_RSQRT = _gpu_fn(torch.rsqrt)


def _bf16_steps_apart(a, b):
    """How many bf16 steps two bf16-valued float32 arrays are apart, elementwise (as integers)."""
    return np.abs((a.view(np.int32) >> 16).astype(np.int64) - (b.view(np.int32) >> 16).astype(np.int64))


def test_vector_bf16_softmax_and_rmsnorm(cuda):
    """vector="bf16" softmax and RMSNorm on the GPU: bit for bit against oracle/vector.py given the GPU's exp,
    sum, mean and rsqrt (every step around those library calls, and every bf16 rounding, pinned); against the
    reference's own CPU outputs (tests/golden/vector.npz) they differ only where those library calls do: at most
    1 bf16 step, on at most 2 % of the outputs."""
    from mxq.nn import _vector
    from oracle import vector as ov
    z = np.load(os.path.join(GOLDEN, "vector.npz"), allow_pickle=False)
    S = z["softmax_S"]
    got = _vector.softmax(torch.from_numpy(S).cuda(), "bf16").cpu().numpy()
    assert_bits_equal(got, ov.softmax_bf16(S, GPU_EXP, GPU_ROWSUM), "softmax bf16 vs oracle")
    d = _bf16_steps_apart(got, z["softmax_bf16"])
    assert d.max() <= 1 and (d > 0).mean() <= 0.02, (d.max(), (d > 0).mean())
    dt = {"torch.bfloat16": torch.bfloat16, "torch.float32": torch.float32}
    for i in range(3):
        xd, wd = (dt[str(v)] for v in z[f"rms{i}_dtypes"])
        x = torch.from_numpy(z[f"rms{i}_x"]).to(xd).cuda()
        w = torch.from_numpy(z[f"rms{i}_w"]).to(wd).cuda()
        for prec in (None, "bf16"):
            got = _vector.rmsnorm(x, w, 1e-6, prec).float().cpu().numpy()
            want = ov.rmsnorm(z[f"rms{i}_x"], z[f"rms{i}_w"], 1e-6, prec, GPU_MEAN, GPU_RSQRT,
                              xd == torch.bfloat16, wd == torch.bfloat16)
            assert_bits_equal(got, want, f"rmsnorm {xd} x {wd} {prec} vs oracle")
            ref = z[f"rms{i}_{prec}"]
            if prec == "bf16" or (xd == torch.bfloat16 and wd == torch.bfloat16):
                d = _bf16_steps_apart(got, ref)
                assert d.max() <= 1 and (d > 0).mean() <= 0.02, (xd, wd, prec, d.max())
            else:
                np.testing.assert_allclose(got, ref, rtol=2.0 ** -20, atol=0)


def test_attend_vector_bf16(cuda):
    """attend with vector="bf16" (score steps and softmax rounded) on the reference's three fixture shapes and on
    a batched causal shape: bit for bit against oracle/attend.py with oracle/vector.py's softmax over the GPU's
    exp and row sum; and bit for bit against the reference's CPU outputs (measured: the bf16 softmax rows come
    out the same from both devices' library calls on these shapes, so no output differs)."""
    import mxq
    from functools import partial

    from oracle import vector as ov
    z = np.load(os.path.join(GOLDEN, "vector.npz"), allow_pickle=False)
    sm = partial(ov.softmax_bf16, exp=GPU_EXP, rowsum=GPU_ROWSUM)
    hwo = _hw_oracle()
    t = lambda a: None if a is None else torch.from_numpy(a).cuda()                   # noqa: E731
    for i in range(3):
        B, H, Hkv, T, D, masked, chunk = (int(x) for x in z[f"c{i}_meta"])
        q, k, v = z[f"c{i}_q"], z[f"c{i}_k"], z[f"c{i}_v"]
        mask = z[f"c{i}_mask"] if masked else None
        chunk = None if chunk < 0 else chunk
        got = mxq.nn.attend(t(q), t(k), t(v), t(mask), D ** -0.5, _hw(mxq), _hw(mxq), chunk=chunk,
                            vector="bf16").cpu().numpy()
        want = oatt.attend(q, k, v, mask, D ** -0.5, hwo, hwo, sm, chunk=chunk, vector="bf16")
        assert_bits_equal(got, want, f"attend vector bf16 c{i} vs oracle")
        assert_bits_equal(got, z[f"c{i}_o"], f"attend vector bf16 c{i} vs the reference's own outputs")
    g = torch.Generator().manual_seed(8)
    q, k, v = (torch.randn(1, h, 256, 64, generator=g) for h in (4, 2, 2))
    mask = _causal(1, 256, 256)
    got = mxq.nn.attend(q.cuda(), k.cuda(), v.cuda(), mask.cuda(), 0.125, _hw(mxq), _hw(mxq), vector="bf16")
    want = oatt.attend(q.numpy(), k.numpy(), v.numpy(), mask.numpy(), 0.125, hwo, hwo, sm, vector="bf16")
    assert_bits_equal(got.cpu().numpy(), want, "attend vector bf16 batched 1x4x256x64 GQA 2:1")


def test_mxlinear_against_oracle(cuda):
    import mxq
    torch.manual_seed(4)
    lin = nn.Linear(96, 48).cuda()
    m = mxq.nn.MXLinear(lin, _hw(mxq))
    x = torch.randn(3, 7, 96, device="cuda", dtype=torch.bfloat16)
    y = m(x)
    A = x.reshape(-1, 96).float().t().contiguous().cpu().numpy()
    W = lin.weight.detach().float().t().contiguous().cpu().numpy()
    so = _hw_oracle()
    Y = osys.systolic(*so.a(A), *so.b(W), nx.MXGEMMINI(), osys.HW_FINAL)
    Y = (torch.from_numpy(Y) + lin.bias.detach().float().cpu()).to(torch.bfloat16).reshape(3, 7, 48)
    assert y.dtype == torch.bfloat16 and torch.equal(y.cpu(), Y)
    assert torch.equal(mxq.nn.MXLinear(lin, _hw(mxq), chunk=5)(x), y)


def _tiny_llama(seed):
    from transformers import LlamaConfig, LlamaForCausalLM
    cfg = LlamaConfig(vocab_size=64, hidden_size=64, intermediate_size=96, num_hidden_layers=2,
                      num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=128)
    torch.manual_seed(seed)
    return LlamaForCausalLM(cfg).eval().cuda()


def test_patch_on_gpu(cuda):
    import mxq
    from mxq.nn import is_attention, patch
    model = _tiny_llama(0)
    ids = torch.randint(0, 64, (2, 20), generator=torch.Generator().manual_seed(0)).cuda()
    before = model(ids).logits
    hw = _hw(mxq)
    h = patch(model, [("lm_head", None), (is_attention, None), (nn.Linear, hw),
                      ("model.layers.0.self_attn", (hw, hw))], vector="bf16")
    assert isinstance(model.model.layers[0].mlp.up_proj, mxq.nn.MXLinear)
    assert {name: names for name, _, names in h.cores} == {"model.layers.0.self_attn": ("hw", "hw"),
                                                           "model.layers.1.self_attn": ("exact", "exact")}
    assert len(h.norms) == 5
    out = model(ids).logits
    assert torch.isfinite(out).all() and not torch.equal(out, before)
    h.revert()
    assert torch.equal(model(ids).logits, before)


def test_exact_core_matches_eager(cuda):
    """The EXACT core (fp32 operands, float64 sums) against transformers' eager attention."""
    from mxq.nn import patch
    from mxq.nn._vector import EXACT
    model = _tiny_llama(2)
    ids = torch.randint(0, 64, (2, 14), generator=torch.Generator().manual_seed(2)).cuda()
    model.set_attn_implementation("eager")
    eager = model(ids).logits
    h = patch(model, [(lambda name, mod, parent: True, (EXACT, EXACT))])
    torch.testing.assert_close(model(ids).logits, eager, rtol=1e-4, atol=1e-4)
    h.revert()


def test_attend_batched_launch_ranges(cuda, monkeypatch):
    """The batched path split into launches of fewer pairs than a batch row holds, each launched as soon as it
    is prepared (a budget of one byte of prepared codes), two batch rows with their own left-padding masks, GQA
    2:1: bit for bit against the oracle's per-call loop."""
    import mxq
    from mxq.nn import _attention
    monkeypatch.setattr(_attention, "ELEMENTS_PER_LAUNCH", 3 * 2 * 48 * 48)
    monkeypatch.setattr(_attention, "PREPARED_BYTES", 1)
    B, H, Hkv, T, D = 2, 8, 4, 48, 32
    g = torch.Generator().manual_seed(9)
    q, k, v = (torch.randn(B, h, T, D, generator=g) for h in (H, Hkv, Hkv))
    mask = _causal(B, T, T)
    mask[0, :, :, :5] = torch.finfo(torch.float32).min
    mask[1, :, :, :11] = torch.finfo(torch.float32).min
    hw, hwo = _hw(mxq), _hw_oracle()
    got = mxq.nn.attend(q.cuda(), k.cuda(), v.cuda(), mask.cuda(), D ** -0.5, hw, hw).cpu().numpy()
    want = oatt.attend(q.numpy(), k.numpy(), v.numpy(), mask.numpy(), D ** -0.5, hwo, hwo, _gpu_softmax)
    assert_bits_equal(got, want, "batched launch ranges")
    assert _attention._Batched.of(hw, hw, q.cuda()) is not None, "the hw scheme takes the batched path"


def test_attend_batched_pairwise_fallback(cuda):
    """In one batched launch, the pairs of batch row 1 (right padding: its last 40 keys masked for every query)
    would skip keys and are redone through the per-call loop, those of row 0 (causal) are not; every output
    bit for bit against the oracle.  An all-zero V block behind the padding checks that skipped keys add
    nothing."""
    import mxq
    B, H, Hkv, T, D = 2, 4, 2, 96, 32
    g = torch.Generator().manual_seed(21)
    q, k, v = (torch.randn(B, h, T, D, generator=g) for h in (H, Hkv, Hkv))
    mask = _causal(B, T, T)
    mask[1, :, :, T - 40:] = torch.finfo(torch.float32).min
    v[1, :, T - 32:] = 0.0
    hw, hwo = _hw(mxq), _hw_oracle()
    got = mxq.nn.attend(q.cuda(), k.cuda(), v.cuda(), mask.cuda(), D ** -0.5, hw, hw).cpu().numpy()
    want = oatt.attend(q.numpy(), k.numpy(), v.numpy(), mask.numpy(), D ** -0.5, hwo, hwo, _gpu_softmax)
    assert_bits_equal(got, want, "pairwise fallback")


@pytest.mark.parametrize("K,cols,groups,bs,aligned", [(128, 65536, 32, 32, True), (70, 108, 3, 32, True),
                                                       (9, 80, 4, 5, True), (9, 80, 4, 5, False),
                                                       (13, 30, 3, 3, True)])
def test_group_amax_against_torch(cuda, K, cols, groups, bs, aligned):
    """mxq_group_amax against _code_amax of each column group (the reference's |code| * scale maximum per
    contraction row): C5's Q^T shape, row counts that leave a partial group of four rows, block sizes that split
    one, codes at a 4-byte offset and groups of 10 columns (4-byte loads), with NaN, Inf and zero scales."""
    from mxq.nn import _attention
    g = torch.Generator().manual_seed(K * 7 + cols)
    nb = -(-K // bs)
    flat = torch.randn(K * cols + 1, generator=g)
    codes = (flat[:K * cols] if aligned else flat[1:]).view(K, cols)
    scales = torch.ldexp(torch.ones(nb, cols), torch.randint(-6, 6, (nb, cols), generator=g).float())
    codes[1, 5], codes[2, cols - 1], codes[K - 1, 0] = float("nan"), float("inf"), float("inf")
    scales[0, 3], scales[(K - 1) // bs, 0] = 0.0, 0.0                 # 0 * Inf = NaN in the last row
    dflat = flat.cuda()                                               # the offset kept on the device
    dc, ds = (dflat[:K * cols] if aligned else dflat[1:]).view(K, cols), scales.cuda()
    assert (dc.data_ptr() % 16 == 0) == aligned
    got = _attention._group_amax(dc, ds, bs, groups).cpu()
    per = cols // groups
    want = torch.stack([_attention._code_amax(codes[:, j * per:(j + 1) * per], scales[:, j * per:(j + 1) * per], bs)
                        for j in range(groups)], dim=1)
    assert got.shape == want.shape == (K, groups)
    assert torch.equal(got.isnan(), want.isnan()), "NaN positions differ"
    assert torch.equal(torch.nan_to_num(got), torch.nan_to_num(want)), "group maxima differ"


@pytest.mark.parametrize("kind", ["causal_min", "causal_weak", "window"])
def test_attend_skip_hints(cuda, monkeypatch, kind):
    """The batched path's skip hints (32 x 32 score groups whose mask absorbs every score the call can make):
    every output bit for bit against the oracle; the absorbing causal mask (finfo.min) and a sliding window of
    96 keys mark groups, a causal mask of -30 (which scores can outweigh) marks none."""
    import mxq
    from mxq.nn import _attention as at
    B, H, Hkv, T, D = 1, 2, 2, 256, 64
    g = torch.Generator().manual_seed(5)
    q, k, v = (torch.randn(B, h, T, D, generator=g) for h in (H, Hkv, Hkv))
    i, j = torch.arange(T)[:, None], torch.arange(T)[None, :]
    low = torch.finfo(torch.float32).min
    if kind == "causal_min":
        mask = _causal(B, T, T)
    elif kind == "causal_weak":
        mask = torch.where(j > i, -30.0, 0.0)[None, None]
    else:
        mask = torch.where((j > i) | (j < i - 96), low, 0.0)[None, None]
    marked, tails = [], []
    orig = at._hints

    def spy(*a, **kw):
        skip, k_end, tail_max = orig(*a, **kw)
        marked.append(0 if skip is None else int(skip.sum()))
        tails.append(tail_max is not None)
        return skip, k_end, tail_max

    monkeypatch.setattr(at, "_hints", spy)
    hw, hwo = _hw(mxq), _hw_oracle()
    got = mxq.nn.attend(q.cuda(), k.cuda(), v.cuda(), mask.cuda(), D ** -0.5, hw, hw).cpu().numpy()
    want = oatt.attend(q.numpy(), k.numpy(), v.numpy(), mask.numpy(), D ** -0.5, hwo, hwo, _gpu_softmax)
    assert_bits_equal(got, want, f"attend with {kind} mask")
    assert marked, "the batched path ran"
    assert (sum(marked) == 0) if kind == "causal_weak" else (sum(marked) > 0), marked
    assert all(tails), "scores past k_end are left unstored (256 query rows per call, a multiple of 64)"


@pytest.mark.parametrize("kind", ["query_row_masked", "positive_tail", "mixed_group"])
def test_attend_tail_full_rows(cuda, monkeypatch, kind):
    """Rows for which the keys past their 64-row group's k_end matter, so the softmax reads those scores from
    the mask and the group writes P^T there: a query row whose every key is masked (softmax uniform over all
    keys), a mask whose masked value is +max (the masked keys win), and one such row inside a group of ordinary
    causal rows (the group's other rows keep +0 past k_end).  Every output bit for bit against the oracle; the
    tail path taken."""
    import mxq
    from mxq.nn import _attention as at
    B, H, Hkv, T, D = 1, 2, 1, 256, 64
    g = torch.Generator().manual_seed(13)
    q, k, v = (torch.randn(B, h, T, D, generator=g) for h in (H, Hkv, Hkv))
    low, high = torch.finfo(torch.float32).min, torch.finfo(torch.float32).max
    i, j = torch.arange(T)[:, None], torch.arange(T)[None, :]
    if kind == "query_row_masked":
        mask = torch.where(j > i, low, 0.0)[None, None].clone()
        mask[0, 0, 70] = low
    elif kind == "positive_tail":
        mask = torch.where(j > i, high, 0.0)[None, None]
    else:
        mask = torch.where(j > i, low, 0.0)[None, None].clone()
        mask[0, 0, 100, 200:] = high                       # row 100 of group 64..127 prefers its masked keys
    tails = []
    orig = at._hints

    def spy(*a, **kw):
        out = orig(*a, **kw)
        tails.append(out[2] is not None)
        return out

    monkeypatch.setattr(at, "_hints", spy)
    hw, hwo = _hw(mxq), _hw_oracle()
    got = mxq.nn.attend(q.cuda(), k.cuda(), v.cuda(), mask.cuda(), D ** -0.5, hw, hw).cpu().numpy()
    want = oatt.attend(q.numpy(), k.numpy(), v.numpy(), mask.numpy(), D ** -0.5, hwo, hwo, _gpu_softmax)
    assert_bits_equal(got, want, f"attend, {kind}")
    assert tails and all(tails)


def _c5_inputs(Hkv=32):
    """The attention benchmark's inputs: q, k, v of 1 x heads x 2048 x 128 ~ N(0, 1) from seeds 0, 1, 2, and the
    HF eager causal mask (finfo(float32).min above the diagonal)."""
    q = torch.randn(1, 32, 2048, 128, generator=torch.Generator().manual_seed(0))
    k, v = (torch.randn(1, Hkv, 2048, 128, generator=torch.Generator().manual_seed(i)) for i in (1, 2))
    return q, k, v, _causal(1, 2048, 2048)


def test_c5_full_shape_heads_against_oracle(cuda):
    """The attention benchmark's own call (1 x 32 heads x 2048 x 128, causal, one query chunk, the batched path
    with its causal skip), heads 0 and 31 bit for bit against the oracle run on those two heads alone (each head
    is its own KV head, so heads do not interact), with the GPU's softmax.  The oracle's reducer runs over the
    host cores (tests/_pool.py)."""
    import _pool
    import mxq
    from mxq.nn import _attention as at
    q, k, v, mask = _c5_inputs()
    hw = _hw(mxq)
    assert at._Batched.of(hw, hw, q.cuda()) is not None, "the benchmark's Scheme takes the batched path"
    got = mxq.nn.attend(q.cuda(), k.cuda(), v.cuda(), mask.cuda(), 128 ** -0.5, hw, hw).cpu().numpy()
    heads = [0, 31]
    qz = lambda V: ob.mxgemmini_quantize(V, "MXFP8_E4M3", 0)                       # noqa: E731
    side = oatt.Side(qz, qz, _pool.reducer())
    want = oatt.attend(q[:, heads].numpy(), k[:, heads].numpy(), v[:, heads].numpy(), mask.numpy(), 128 ** -0.5,
                       side, side, _gpu_softmax)
    assert_bits_equal(got[:, :, heads], want, "attend 1x32x2048x128 causal, heads 0 and 31")


def test_c5_gqa8_head_group_against_oracle(cuda):
    """The attention benchmark's GQA variant (32 query heads over 8 KV heads) at full shape on the batched path,
    the four query heads 20-23 that share KV head 5 bit for bit against the oracle run on that group alone
    (query head h reads KV head h // 4), with the GPU's softmax."""
    import _pool
    import mxq
    from mxq.nn import _attention as at
    q, k, v, mask = _c5_inputs(8)
    hw = _hw(mxq)
    assert at._Batched.of(hw, hw, q.cuda()) is not None, "the benchmark's Scheme takes the batched path"
    got = mxq.nn.attend(q.cuda(), k.cuda(), v.cuda(), mask.cuda(), 128 ** -0.5, hw, hw).cpu().numpy()
    qz = lambda V: ob.mxgemmini_quantize(V, "MXFP8_E4M3", 0)                       # noqa: E731
    side = oatt.Side(qz, qz, _pool.reducer())
    want = oatt.attend(q[:, 20:24].numpy(), k[:, 5:6].numpy(), v[:, 5:6].numpy(), mask.numpy(), 128 ** -0.5,
                       side, side, _gpu_softmax)
    assert_bits_equal(got[:, :, 20:24], want, "attend 1x32x2048x128 causal over 8 KV heads, heads 20-23")


@pytest.mark.parametrize("Hkv", [32, 8], ids=["mha", "gqa8"])
def test_c5_full_shape_batched_against_per_pair(cuda, Hkv):
    """Every head of the attention benchmark's call (and of its GQA variant with 8 KV heads) from the batched
    path, bit for bit against the reference's per-pair loop on the same library kernels (a Scheme of plain
    callables, which the batched path does not take)."""
    import mxq
    from mxq import Scheme, block, matmul
    from mxq.nn import _attention as at
    q, k, v, mask = (t.cuda() for t in _c5_inputs(Hkv))
    hw = _hw(mxq)
    loose = Scheme("hw", a=lambda V: block.mxgemmini.quantize(V, "MXFP8_E4M3", axis=0),
                   b=lambda V: block.mxgemmini.quantize(V, "MXFP8_E4M3", axis=0),
                   reduce=lambda *ops: matmul.systolic(*ops, matmul.MXGEMMINI(), matmul.HW_FINAL))
    assert at._Batched.of(loose, loose, q) is None
    got = mxq.nn.attend(q, k, v, mask, 128 ** -0.5, hw, hw)
    want = mxq.nn.attend(q, k, v, mask, 128 ** -0.5, loose, loose)
    assert_bits_equal(got.cpu().numpy(), want.cpu().numpy(), f"attend C5 batched vs per pair, {Hkv} KV heads")


@pytest.mark.parametrize("T", [33, 64, 100, 512, 1000, 2048])
def test_softmax_quantize_t_against_torch(cuda, T):
    """The batched path's softmax and P^T quantize in one kernel against torch.softmax followed by
    block.mxgemmini.quantize of the transpose, as the path otherwise calls them: codes and scales bit for bit,
    on scores with a large spread, HF-style masked tails (finfo.min added), a fully masked row (softmax
    uniform), for three formats and both the reference's rounding modes."""
    from functools import partial

    from mxq import block
    from mxq.nn import _attention
    g = torch.Generator(device="cuda").manual_seed(T)
    R = 300
    S = torch.randn(R, T, device="cuda", generator=g) * torch.exp2(torch.randint(-4, 6, (R, 1), device="cuda",
                                                                                 generator=g).float())
    lo = torch.finfo(torch.float32).min
    keep = torch.arange(T, device="cuda")[None, :] <= torch.arange(R, device="cuda")[:, None] % T
    S = torch.where(keep, S, S + lo)
    S[7] = lo
    for fmt, mode in [("MXFP8_E4M3", "ties_away"), ("MXFP8_E4M3", "rne"), ("MXFP6_E2M3", "ties_away"),
                      ("MXFP4", "rne")]:
        q = partial(block.mxgemmini.quantize, fmt=fmt, axis=0, rounding_mode=mode)
        got = _attention._softmax_pt(S, q, 32, None)
        assert got is not None
        want = q(torch.softmax(S, dim=-1).contiguous().t())
        assert_bits_equal(got[1].cpu().numpy(), want[1].cpu().numpy(), f"scales T={T} {fmt} {mode}")
        assert_bits_equal(got[0].cpu().numpy(), want[0].cpu().numpy(), f"codes T={T} {fmt} {mode}")
        assert got[2] is None
    # the stage bytes the P V product reads instead of a pass over P^T: per problem (96 columns each), 32 keys and
    # 32 columns, whether any code is nonzero or any scale not finite
    S2 = S[:288].contiguous()
    q = partial(block.mxgemmini.quantize, fmt="MXFP8_E4M3", axis=0, rounding_mode="ties_away")
    P, X, live = _attention._softmax_pt(S2, q, 32, None, 96)
    want = q(torch.softmax(S2, dim=-1).contiguous().t())
    assert_bits_equal(P.cpu().numpy(), want[0].cpu().numpy(), f"codes T={T} with stage bytes")
    nb = -(-T // 32)
    Pn = np.pad(P.cpu().numpy(), ((0, nb * 32 - T), (0, 0)))
    nz = (Pn.reshape(nb, 32, 3, 3, 32) != 0).any(axis=(1, 4))                   # stage, problem, group
    bad = ~np.isfinite(X.cpu().numpy()).reshape(nb, 3, 3, 32).all(axis=3)
    assert np.array_equal(live.cpu().numpy(), (nz | bad).transpose(1, 0, 2).astype(np.uint8))


def test_exp_underflows_past_minus_128(cuda):
    """The softmax kernel's tail rule rests on exp(x) = +0 on the device for every float32 x <= -128 (e^-103.98 is
    already below half the smallest subnormal): every float32 in [-512, -128] and a strided sample of the rest down
    to -Inf, through torch.exp on the GPU (the same expf the kernel reproduces bit for bit)."""
    lo, hi = 0xC3000000, 0xC4000000                       # -128 .. -512 as bit patterns
    dense = torch.arange(lo, hi + 1, dtype=torch.int64, device="cuda").to(torch.int32).view(torch.float32)
    sparse = torch.arange(hi, 0xFF800001, 4099, dtype=torch.int64, device="cuda").to(torch.int32).view(torch.float32)
    for x in (dense, sparse, torch.tensor([float("-inf")], device="cuda")):
        e = torch.exp(x)
        assert int(e.view(torch.int32).ne(0).sum()) == 0


@pytest.mark.parametrize("fmt", ["MXFP8_E4M3", "MXFP4"])
def test_softmax_tail_against_full_scores(cuda, fmt):
    """mxq_softmax_quantize_t with a tail (S stored below each 64-row group's k_end only, NaN past it, which it must
    not read) against the same kernel on the whole S: three problems of 128 rows x 256 keys with their own mask
    rows, a causal mask (every group takes the short path), one with a query row masked everywhere (its group reads
    the mask and writes every key) and one with a row whose masked keys carry +max (the same).  Codes, scales and
    stage bytes bit for bit wherever the tailed call writes them; where it does not (past k_end of a short-path
    group), the whole-S call has +0 codes and stage bytes 0, so the P V product never reads them."""
    from functools import partial

    from mxq import _lib, block
    from mxq.nn import _attention
    Z, cols, T, scale = 3, 128, 256, 0.125
    g = torch.Generator(device="cuda").manual_seed(31)
    low, high = torch.finfo(torch.float32).min, torch.finfo(torch.float32).max
    i, j = torch.arange(cols, device="cuda")[:, None], torch.arange(T, device="cuda")[None, :]
    mask = torch.where(j > i + 64, low, 0.0).repeat(Z, 1, 1).contiguous()     # Z x cols x T
    mask[1, 70] = low
    mask[2, 10, 200:] = high
    k_end = torch.tensor([[128, 192]] * Z, dtype=torch.int32, device="cuda")  # group t sees keys < 64 (t + 2)
    tail_max = torch.empty(Z, 2, device="cuda")
    for z in range(Z):
        for t in range(2):
            tail_max[z, t] = mask[z, 64 * t:64 * t + 64, int(k_end[z, t]):].max()
    raw = torch.randn(Z, cols, T, device="cuda", generator=g) * 4
    S_full = (raw * scale + mask).contiguous()
    kk = torch.arange(T, device="cuda")[None, None, :]
    ke_row = k_end.repeat_interleave(64, dim=1)[:, :, None]                      # Z x cols x 1
    S_full = torch.where(kk >= ke_row, 0.0 * scale + mask, S_full)             # what the score step stores there
    S_part = torch.where(kk >= ke_row, torch.full_like(S_full, float("nan")), S_full)
    q = partial(block.mxgemmini.quantize, fmt=fmt, axis=0, rounding_mode="rne")
    epi = _lib.SystolicEpilogue(scale=scale, bf16=0, mask=_lib.ptr(mask), mask_b_stride=cols * T, mask_row_stride=T,
                                z0=0, z_per_b=1, m=cols)
    tail = _lib.SoftmaxTail(k_end=_lib.ptr(k_end), tail_max=_lib.ptr(tail_max), score=epi)
    P, X, live = (t.cpu().numpy() for t in _attention._softmax_pt(S_part.view(Z * cols, T), q, 32, None, cols, tail))
    wP, wX, wlive = (t.cpu().numpy() for t in _attention._softmax_pt(S_full.view(Z * cols, T), q, 32, None, cols))
    assert_bits_equal(live, wlive, "stage bytes")
    full_groups = {(1, 1), (2, 0)}
    for z in range(Z):
        for t in range(2):
            c0, ke = z * cols + 64 * t, int(k_end[z, t])
            kw = T if (z, t) in full_groups else ke
            assert_bits_equal(P[:kw, c0:c0 + 64], wP[:kw, c0:c0 + 64], f"codes z{z} t{t}")
            assert_bits_equal(X[:kw // 32, c0:c0 + 64], wX[:kw // 32, c0:c0 + 64], f"scales z{z} t{t}")
            if kw < T:
                assert not wP[kw:, c0:c0 + 64].any() and not wlive[z, kw // 32:, t * 2:t * 2 + 2].any()
