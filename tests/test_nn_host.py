"""mxq.nn host logic on the CPU: attend's calls, grouping, chunking and key skipping, MXLinear, patch.

The Schemes here are small pure-torch stand-ins (no GPU): a quantizer that shares a power-of-two scale over
`rows` adjacent columns per block and keeps 6 fraction bits, and a float64 reducer.  Every product and sum they
make is exact, so any order of summation gives the same bits, and the numpy restatement in oracle/attend.py
with the same stand-ins must agree bit for bit -- including which columns each call groups together.
"""
import math
from functools import partial

import numpy as np
import pytest
import torch
from torch import nn

from _util import assert_bits_equal
from oracle import attend as oatt

import mxq
from mxq import Scheme
from mxq.nn import MXLinear, attend, is_attention, patch
from mxq.nn import _attention as attention_mod


# ---- stand-in Schemes ---------------------------------------------------------------------------------------

def _t_quant(V, rows, bs=32):
    K, n = V.shape
    nb = math.ceil(K / bs)
    pad = torch.zeros(nb * bs, n, dtype=torch.float32)
    pad[:K] = V
    amax = pad.view(nb, bs, n).abs().amax(dim=1)                                   # nb x n
    ng = math.ceil(n / rows)
    g = torch.zeros(nb, ng * rows)
    g[:, :n] = amax
    gmax = g.view(nb, ng, rows).amax(dim=2).repeat_interleave(rows, dim=1)[:, :n]
    X = torch.ldexp(torch.ones_like(gmax), torch.frexp(gmax).exponent)
    P = torch.round(V / X.repeat_interleave(bs, dim=0)[:K] * 64).clamp(-64, 64) / 64
    return P, X


def _n_quant(V, rows, bs=32):
    P, X = _t_quant(torch.from_numpy(np.ascontiguousarray(V, np.float32)), rows, bs)
    return P.numpy(), X.numpy()


def _t_reduce(P_A, X_A, P_B, X_B, bs=32):
    A = (P_A * X_A.repeat_interleave(bs, dim=0)[:P_A.shape[0]]).double()
    B = (P_B * X_B.repeat_interleave(bs, dim=0)[:P_B.shape[0]]).double()
    return (A.t() @ B).float()


def _n_reduce(*ops, bs=32):
    return _t_reduce(*(torch.from_numpy(np.ascontiguousarray(o, np.float32)) for o in ops), bs=bs).numpy()


def _schemes(rows):
    t = Scheme(f"fake{rows}", a=partial(_t_quant, rows=rows), b=partial(_t_quant, rows=1), reduce=_t_reduce,
               rows=rows)
    n = oatt.Side(partial(_n_quant, rows=rows), partial(_n_quant, rows=1), _n_reduce, rows=rows)
    return t, n


def _cpu_softmax(S):
    return torch.softmax(torch.from_numpy(np.ascontiguousarray(S)), dim=-1).numpy()


def _causal(B, Tq, Tk, pad=None):
    m = torch.triu(torch.full((Tq, Tk), torch.finfo(torch.float32).min), Tk - Tq + 1)[None, None].repeat(B, 1, 1, 1)
    if pad is not None:
        for b, p in enumerate(pad):
            m[b, :, :, :p] = torch.finfo(torch.float32).min
    return m


# ---- attend -------------------------------------------------------------------------------------------------

ATTEND_CASES = [
    # B, H, Hkv, Tq, Tk, D, mask, chunk, rows
    (1, 4, 2, 96, 96, 32, "causal", None, 1),
    (1, 4, 2, 96, 96, 32, "causal", 32, 1),
    (2, 2, 2, 64, 64, 64, None, None, 1),
    (1, 2, 1, 70, 70, 32, "causal", 16, 2),            # tails per head (70 = 4*16 + 6; rows 2)
    (1, 4, 1, 45, 45, 32, "causal", 12, 4),            # tails of 1 query, GQA 4:1, rows 4
    (2, 2, 1, 48, 48, 32, "padded", 16, 1),            # left padding: rows that see no key
    (1, 2, 2, 1, 80, 32, "causal", None, 1),           # one query over 80 keys (decode)
    (1, 2, 2, 33, 33, 40, "causal", 8, 1),             # D not a multiple of the block
]


@pytest.mark.parametrize("case", ATTEND_CASES, ids=[f"c{i}" for i in range(len(ATTEND_CASES))])
def test_attend_matches_oracle(case):
    B, H, Hkv, Tq, Tk, D, kind, chunk, rows = case
    g = torch.Generator().manual_seed(7)
    q, k, v = (torch.randn(B, h, T, D, generator=g) for h, T in ((H, Tq), (Hkv, Tk), (Hkv, Tk)))
    mask = None
    if kind == "causal":
        mask = _causal(B, Tq, Tk)
    elif kind == "padded":
        mask = _causal(B, Tq, Tk, pad=[5, 20])
    t, n = _schemes(rows)
    got = attend(q, k, v, mask, D ** -0.5, t, t, chunk=chunk)
    want = oatt.attend(q.numpy(), k.numpy(), v.numpy(), None if mask is None else mask.numpy(), D ** -0.5, n, n,
                       _cpu_softmax, chunk=chunk)
    assert got.shape == (B, Tq, H, D)
    assert_bits_equal(got.numpy(), want, f"attend {case}")


def test_attend_skips_absorbed_keys():
    """With small chunks under a causal mask, calls multiply only up to the last key they see."""
    seen = []
    t, _ = _schemes(1)

    def counting(P_A, X_A, P_B, X_B):
        seen.append(P_B.shape[1])
        return _t_reduce(P_A, X_A, P_B, X_B)

    s = Scheme("count", a=t.a, b=t.b, reduce=counting)
    g = torch.Generator().manual_seed(1)
    q, k, v = (torch.randn(1, 1, 128, 32, generator=g) for _ in range(3))
    attend(q, k, v, _causal(1, 128, 128), 32 ** -0.5, s, t, chunk=32)
    assert seen == [32, 64, 96, 128]


def test_attend_rejects():
    t, _ = _schemes(2)
    q = torch.zeros(1, 3, 8, 32)
    with pytest.raises(ValueError, match="heads"):
        attend(q, torch.zeros(1, 2, 8, 32), torch.zeros(1, 2, 8, 32), None, 1.0, t, t)
    with pytest.raises(ValueError, match="chunk"):
        attend(torch.zeros(1, 2, 8, 32), torch.zeros(1, 1, 8, 32), torch.zeros(1, 1, 8, 32), None, 1.0, t, t, chunk=3)
    bad = Scheme("bad", a=t.a, b=t.b, reduce=t.reduce, block_size=16)
    with pytest.raises(ValueError, match="block_size"):
        attend(torch.zeros(1, 2, 8, 64), torch.zeros(1, 1, 8, 64), torch.zeros(1, 1, 8, 64), None, 1.0, bad, bad)


def test_attend_mask_extents():
    """A mask whose key (or query) dimension is 1 broadcasts: the same result as the mask expanded to Tq x Tk.
    A key dimension that is neither 1 nor Tk (after the :Tk cut), a query dimension that is neither 1 nor Tq,
    and 1 < mask batch < B cannot broadcast and are refused before any call."""
    t, n = _schemes(1)
    g = torch.Generator().manual_seed(3)
    B, H, T, D = 2, 2, 40, 32
    q, k, v = (torch.randn(B, H, T, D, generator=g) for _ in range(3))
    row = torch.where(torch.arange(T) % 3 == 0, torch.finfo(torch.float32).min, 0.0)
    key1 = row[None, None, :, None].repeat(B, 1, 1, 1)                     # B x 1 x Tq x 1
    got = attend(q, k, v, key1, D ** -0.5, t, t)
    want = attend(q, k, v, key1.expand(B, 1, T, T).contiguous(), D ** -0.5, t, t)
    assert_bits_equal(got.numpy(), want.numpy(), "key-broadcast mask")
    wo = oatt.attend(q.numpy(), k.numpy(), v.numpy(), key1.expand(B, 1, T, T).numpy(), D ** -0.5, n, n, _cpu_softmax)
    assert_bits_equal(got.numpy(), wo, "key-broadcast mask vs oracle")
    longer = _causal(B, T, T + 8)                                            # extra keys are cut off, as HF's
    assert_bits_equal(attend(q, k, v, longer, D ** -0.5, t, t).numpy(),
                      attend(q, k, v, longer[..., :T].contiguous(), D ** -0.5, t, t).numpy(), "long mask")
    for bad in (_causal(B, T, T)[..., :T - 5], _causal(B, T, T)[:, :, :T - 1], torch.zeros(T, T)):
        with pytest.raises(ValueError, match="mask"):
            attend(q, k, v, bad, D ** -0.5, t, t)
    q3, k3, v3 = (torch.randn(3, H, T, D, generator=g) for _ in range(3))
    with pytest.raises(ValueError, match="mask"):
        attend(q3, k3, v3, _causal(2, T, T), D ** -0.5, t, t)


def test_default_step():
    assert attention_mod.ELEMENTS_PER_STEP == 1 << 26 and attention_mod.SLACK == 2.0 ** 16


# ---- MXLinear -----------------------------------------------------------------------------------------------

def _linear(K=64, N=40, bias=True):
    torch.manual_seed(3)
    return nn.Linear(K, N, bias=bias)


@pytest.mark.parametrize("bias", [True, False])
def test_mxlinear_forward(bias):
    lin = _linear(bias=bias)
    t, _ = _schemes(1)
    m = MXLinear(lin, t)
    x = torch.randn(2, 5, 64, dtype=torch.bfloat16)
    y = m(x)
    A = x.reshape(-1, 64).float().t().contiguous()
    want = _t_reduce(*t.a(A), *t.b(lin.weight.detach().float().t().contiguous()))
    if bias:
        want = want + lin.bias.float()
    assert y.dtype == torch.bfloat16 and y.shape == (2, 5, 40)
    assert torch.equal(y, want.to(torch.bfloat16).reshape(2, 5, 40))


def test_mxlinear_chunks_keep_bits():
    lin = _linear()
    t, _ = _schemes(4)
    x = torch.randn(50, 64)
    whole = MXLinear(lin, t)(x)
    for chunk in (4, 8, 48):
        assert torch.equal(MXLinear(lin, t, chunk=chunk)(x), whole)
    assert torch.equal(MXLinear(lin, t, cache_weights=False)(x), whole)


def test_mxlinear_parameters_and_refresh():
    lin = _linear()
    t, _ = _schemes(1)
    m = MXLinear(lin, t)
    assert m.weight is lin.weight and m.bias is lin.bias
    assert set(m.state_dict()) == {"weight", "bias"}
    x = torch.randn(3, 64)
    before = m(x)
    with torch.no_grad():
        lin.weight.mul_(2)
    assert torch.equal(m(x), before)                                            # cached codes
    m.refresh()
    assert not torch.equal(m(x), before)
    assert "scheme='fake1'" in repr(m)
    with pytest.raises(ValueError, match="chunk"):
        MXLinear(lin, t, chunk=0)
    with pytest.raises(ValueError, match="multiple"):
        MXLinear(lin, _schemes(4)[0], chunk=6)


def test_mxlinear_no_tokens():
    lin = _linear()
    t, _ = _schemes(1)
    assert MXLinear(lin, t)(torch.zeros(0, 64)).shape == (0, 40)


# ---- patch --------------------------------------------------------------------------------------------------

def _tiny_llama(seed=0):
    from transformers import LlamaConfig, LlamaForCausalLM
    cfg = LlamaConfig(vocab_size=64, hidden_size=64, intermediate_size=96, num_hidden_layers=2,
                      num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=128)
    torch.manual_seed(seed)
    return LlamaForCausalLM(cfg).eval()


def test_patch_routes_and_reverts(capsys):
    model = _tiny_llama()
    t, _ = _schemes(1)
    t2 = Scheme("other", a=t.a, b=t.b, reduce=t.reduce)
    ids = torch.randint(0, 64, (1, 12), generator=torch.Generator().manual_seed(0))
    before = model(ids).logits
    rules = [("lm_head", None), ("*.mlp.down_proj", t2), (is_attention, None), (nn.Linear, t)]
    patch(model, rules, dry_run=True)
    printed = capsys.readouterr().out
    assert "lm_head" in printed and "left as is" in printed and "other" in printed
    assert isinstance(model.model.layers[0].mlp.down_proj, nn.Linear)               # dry run changed nothing
    h = patch(model, rules)
    rows = {name: (rule, scheme) for name, _, _, rule, scheme in h.table}
    assert rows["lm_head"] == (0, None)
    assert rows["model.layers.1.mlp.down_proj"] == (1, "other")
    assert rows["model.layers.0.self_attn.q_proj"] == (2, None)
    assert rows["model.layers.0.mlp.up_proj"] == (3, "fake1")
    assert isinstance(model.model.layers[1].mlp.down_proj, MXLinear)
    assert isinstance(model.model.layers[1].self_attn.q_proj, nn.Linear)
    assert model(ids).logits.shape == before.shape
    h.revert()
    assert isinstance(model.model.layers[1].mlp.down_proj, nn.Linear)
    assert torch.equal(model(ids).logits, before)


def _ident(V):
    return V.clone(), torch.ones(math.ceil(V.shape[0] / 32), V.shape[1])


IDENT = Scheme("ident", a=_ident, b=_ident, reduce=_t_reduce)


def test_patch_core_and_vector():
    model = _tiny_llama(1)
    t, _ = _schemes(1)
    ids = torch.randint(0, 64, (1, 10), generator=torch.Generator().manual_seed(1))
    before = model(ids).logits
    h = patch(model, [("model.layers.0.self_attn", (t, t)), ("*.self_attn", (IDENT, t))])
    assert model.config._attn_implementation == "mxq"
    cores = {name: names for name, _, names in h.cores}
    assert cores == {"model.layers.0.self_attn": ("fake1", "fake1"), "model.layers.1.self_attn": ("ident", "fake1")}
    assert not hasattr(model.model.layers[1].self_attn, "_mxq_vector")
    out = model(ids).logits
    assert torch.isfinite(out).all() and not torch.equal(out, before)
    h.revert()
    assert model.config._attn_implementation == "sdpa"
    assert not hasattr(model.model.layers[0].self_attn, "_mxq_core")
    assert torch.equal(model(ids).logits, before)


def test_patch_unchosen_core_gets_exact_and_needs_gpu():
    """vector softmax gives an attention module no rule chose the EXACT core, whose quantizers are the gfx950
    kernels: without a GPU that fails loudly, before the model changes."""
    model = _tiny_llama(1)
    t, _ = _schemes(1)
    with pytest.raises(RuntimeError, match="no GPU"):
        patch(model, [("model.layers.0.self_attn", (t, t))], vector="bf16", dry_run=True)
    assert model.config._attn_implementation == "sdpa"


def test_patch_ident_core_matches_eager():
    """attend with no quantization and float64 sums against transformers' eager attention (GQA, causal mask)."""
    model = _tiny_llama(2)
    ids = torch.randint(0, 64, (2, 14), generator=torch.Generator().manual_seed(2))
    model.set_attn_implementation("eager")
    eager = model(ids).logits
    h = patch(model, [(lambda name, mod, parent: True, (IDENT, IDENT))])
    got = model(ids).logits
    torch.testing.assert_close(got, eager, rtol=1e-5, atol=1e-5)
    h.revert()
    assert model.config._attn_implementation == "eager"


def test_patch_rmsnorm_bit_check():
    model = _tiny_llama(3)
    ids = torch.randint(0, 64, (1, 8), generator=torch.Generator().manual_seed(3))
    before = model(ids).logits
    h = patch(model, [], vector={"rmsnorm": "bf16"}, dry_run=True)          # the bit check runs unrounded
    assert len(h.norms) == 5                                                     # 2 x 2 per layer + final norm
    assert "rmsnorm bf16 (5 modules)" in str(h)
    assert torch.equal(model(ids).logits, before)
    h = patch(model, [], vector={"rmsnorm": None})
    assert h.norms == [] and torch.equal(model(ids).logits, before)


class _Block(nn.Module):
    def __init__(self):
        super().__init__()
        self.a = nn.Linear(64, 64)
        self.b = nn.Linear(64, 64)


class _Shared(nn.Module):
    def __init__(self):
        super().__init__()
        self.x = _Block()
        self.y = self.x                                                         # the same subtree twice
        self.z = nn.Linear(64, 64)


class _GemmaNorm(nn.Module):
    """Not the LlamaRMSNorm formula: (1 + weight)."""
    def __init__(self):
        super().__init__()
        self.weight = nn.Parameter(torch.zeros(64))
        self.eps = 1e-6

    def forward(self, x):
        h = x.float()
        return (h * torch.rsqrt(h.pow(2).mean(-1, keepdim=True) + self.eps)) * (1.0 + self.weight)


class _WithNorm(nn.Module):
    def __init__(self):
        super().__init__()
        self.lin = nn.Linear(64, 64)
        self.norm = _GemmaNorm()
        type(self.norm).__name__ = "GemmaLikeRMSNorm"


def test_patch_errors():
    t, _ = _schemes(1)
    model = _Shared()
    with pytest.raises(ValueError, match="must be"):
        patch(model, [("z", "FP8")])
    with pytest.raises(ValueError, match=r"rules \[0\] choose no Linear"):
        patch(model, [("nothing*", t)])
    with pytest.raises(ValueError, match=r"rules \[1\] choose no Linear"):
        patch(model, [(nn.Linear, t), ("z", None)])
    with pytest.raises(ValueError, match="same layer"):
        patch(model, [("x.a", t), ("y.a", None), (nn.Linear, None)])
    with pytest.raises(ValueError, match="choose no attention module"):
        patch(model, [("x", (t, t))])
    with pytest.raises(ValueError, match="vector softmax"):
        patch(model, [], vector="bf16")
    with pytest.raises(ValueError, match="vector must be"):
        patch(model, [], vector={"gelu": "bf16"})
    with pytest.raises(ValueError, match="vector rmsnorm"):
        patch(model, [], vector={"rmsnorm": "bf16"})
    with pytest.raises(ValueError, match="LlamaRMSNorm"):
        patch(_WithNorm(), [], vector={"rmsnorm": "bf16"})
    broken = Scheme("broken", a=t.a, b=t.b, reduce=lambda *a: (_ for _ in ()).throw(RuntimeError("smoke")))
    with pytest.raises(RuntimeError, match="smoke"):
        patch(model, [(nn.Linear, broken)])
    assert isinstance(model.z, nn.Linear)                                       # nothing changed on failure


def test_patch_shared_module_names():
    t, _ = _schemes(1)
    model = _Shared()
    h = patch(model, [("*.a", None), (nn.Linear, t)])
    names = [r[0] for r in h.table]
    assert names == ["x.a", "x.b", "y.a", "y.b", "z"]
    assert [r[3] for r in h.table] == [0, 1, 0, 1, 1]
    assert isinstance(model.x.b, MXLinear) and model.y.b is model.x.b and isinstance(model.x.a, nn.Linear)
    h.revert()
    with pytest.raises(ValueError, match="same layer"):
        patch(model, [("y.a", t), (nn.Linear, None)])
    h = patch(model, [(nn.Linear, t)])
    assert isinstance(model.x.a, MXLinear) and model.y.a is model.x.a
    h.revert()
    assert isinstance(model.x.a, nn.Linear)
