"""experiments.llm_ppl on the GPU with the tapeout recipe: the whole command on a tiny random Llama saved to
disk, every window's NLL equal to the patched model's own forward, the layer table, and a dry run; and the
patched model at layer level, every MXLinear bit for bit against the oracle inside the HF forward."""
import math

import numpy as np
import pytest
import torch

from _util import assert_bits_equal

pytestmark = pytest.mark.gpu


def test_tapeout_perplexity(cuda, tmp_path):
    from transformers import LlamaConfig, LlamaForCausalLM

    from experiments import llm_ppl, recipes
    from mxq.nn import MXLinear, patch
    cfg = LlamaConfig(vocab_size=96, hidden_size=64, intermediate_size=96, num_hidden_layers=2,
                      num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=64)
    torch.manual_seed(0)
    path = tmp_path / "tiny"
    LlamaForCausalLM(cfg).save_pretrained(path)
    tok = tmp_path / "ids.npy"
    np.save(tok, np.random.default_rng(3).integers(0, 96, 400).astype(np.int64))
    args = ["--model", str(path), "--tokens", str(tok), "--seqlen", "64", "--nsamples", "2", "--dtype",
            "float32"]
    base = llm_ppl.main(["--rules", "none", "--out", str(tmp_path / "a.json")] + args)
    hw = llm_ppl.main(["--rules", "hw_mxfp8_tapeout", "--out", str(tmp_path / "b.json")] + args)
    assert math.isfinite(hw["perplexity"]) and hw["perplexity"] != base["perplexity"]
    rows = {name: (rule, scheme) for name, _, _, rule, scheme in hw["layers"]}
    assert rows["lm_head"] == (1, "hw_mxfp8_tapeout") and rows["model.layers.0.mlp.up_proj"][1] == "hw_mxfp8_tapeout"
    assert rows["model.layers.0.self_attn.q_proj"] == (0, None)
    assert hw["schemes"]["hw_mxfp8_tapeout"]["reduce"]["arith"] == "compiled(mxgemmini(prod=e4m3))"

    model = llm_ppl.load_model(str(path), 64, torch.float32)
    patch(model, recipes.RULES["hw_mxfp8_tapeout"])
    assert isinstance(model.lm_head, MXLinear)
    ids = llm_ppl.windows(llm_ppl.token_stream(str(tok)), 64, 2, 0)
    for s in hw["per_sample"]:
        assert (s["nll"], s["tokens"]) == llm_ppl.sample_nll(model, ids[s["index"]])

    lines = []
    dry = llm_ppl.evaluate(llm_ppl.load_model(str(path), 64, torch.float32), ids,
                           recipes.RULES["hw_mxfp8_tapeout_all"], dry_run=True, log=lines.append)
    assert dry is None and "lm_head" in lines[0] and "attention core" in lines[0]


def _tapeout_oracle():
    """The tapeout Scheme in the oracle: block.mxgemmini MXFP8_E4M3 (rne, floor 2^-23) for both operands, the
    systolic reducer with MXGEMMINI and HW_FINAL."""
    from oracle import block as ob
    from oracle import numerics as nx
    from oracle import systolic as osys

    def q(V):
        return ob.mxgemmini_quantize(V, "MXFP8_E4M3", 0, rounding_mode="rne", scale_floor=2.0 ** -23)

    def linear(x, W, b):
        """MXLinear.forward on the host: A = x^T (in x tokens), B = W^T (in x out), + bias in float32."""
        Y = osys.systolic(*q(np.ascontiguousarray(x.T)), *q(np.ascontiguousarray(W.T)), nx.MXGEMMINI(),
                          osys.HW_FINAL)
        return Y if b is None else (Y + b).astype(np.float32)
    return linear


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["fp32", "bf16"])
def test_tapeout_model_layers_against_oracle(cuda, tmp_path, dtype):
    """The tapeout rules on a tiny random Llama loaded from disk, at model level: every MXLinear's output inside
    the HF forward (token rows cut into calls of 24 by `chunk`, codes of the weights cached at patch time) bit
    for bit against the oracle's quantizers and systolic reducer on the captured input; one weight edited in
    place (cached codes still used, then refresh()) compared both ways; every window's NLL recomputed on the
    host in float64 from the GPU logits."""
    from transformers import LlamaConfig, LlamaForCausalLM

    from experiments import llm_ppl, recipes
    from mxq.nn import MXLinear, patch
    cfg = LlamaConfig(vocab_size=96, hidden_size=64, intermediate_size=96, num_hidden_layers=2,
                      num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=64)
    torch.manual_seed(1)
    path = tmp_path / "tiny"
    LlamaForCausalLM(cfg).save_pretrained(path)
    model = llm_ppl.load_model(str(path), 64, dtype)
    h = patch(model, recipes.RULES["hw_mxfp8_tapeout"], chunk=24)
    mx = {name: m for name, m in model.named_modules() if isinstance(m, MXLinear)}
    assert sorted(mx) == sorted([f"model.layers.{i}.mlp.{p}" for i in range(2) for p in
                                 ("gate_proj", "up_proj", "down_proj")] + ["lm_head"])
    assert all(m.chunk == 24 for m in mx.values()) and h.table
    seen = []
    hooks = [m.register_forward_hook(lambda mod, inp, out, name=name: seen.append(
        (name, inp[0].detach().clone(), out.detach().clone()))) for name, m in mx.items()]
    oracle = _tapeout_oracle()

    def check(weights):
        for name, x, y in seen:
            m = mx[name]
            assert y.dtype == dtype and y.shape[:-1] == x.shape[:-1]
            W = weights.get(name, m.weight).detach().float().cpu().numpy()
            b = None if m.bias is None else m.bias.detach().float().cpu().numpy()
            xs = x.reshape(-1, m.in_features).float().cpu().numpy()
            assert xs.shape[0] > 24, "the window's token rows span several reducer calls"
            want = torch.from_numpy(oracle(xs, W, b)).to(dtype).float().numpy()
            got = y.reshape(-1, m.out_features).float().cpu().numpy()
            assert_bits_equal(got, want, f"{name} ({dtype}) vs the oracle's quantize + systolic")
        seen.clear()

    ids = llm_ppl.windows(torch.from_numpy(np.random.default_rng(5).integers(0, 96, 300)).long(), 64, 2, 0)
    for i in range(ids.shape[0]):
        nll, n = llm_ppl.sample_nll(model, ids[i])
        logits = seen[-1][2][0, :-1].double().cpu()                               # lm_head's output
        tgt = ids[i, 1:]
        host = -(logits.gather(1, tgt[:, None])[:, 0] - torch.logsumexp(logits, dim=-1)).sum().item()
        assert n == 63 and math.isclose(nll, host, rel_tol=1e-5), (nll, host)
        check({})

    # an in-place weight edit: the cached codes keep serving until refresh()
    down = mx["model.layers.1.mlp.down_proj"]
    old = down.weight.detach().clone()
    with torch.no_grad():
        down.weight.mul_(-1.5)
    llm_ppl.sample_nll(model, ids[0])
    check({"model.layers.1.mlp.down_proj": old})
    down.refresh()
    llm_ppl.sample_nll(model, ids[0])
    check({})
    for hk in hooks:
        hk.remove()
