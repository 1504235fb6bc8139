"""experiments.recipes and experiments.llm_ppl on the CPU: the recipe's Schemes and rule lists, the window
protocol, the loss against torch's cross entropy, and the whole command on a tiny random Llama saved to disk
(rules "none": no GPU kernel runs)."""
import json
import math

import numpy as np
import pytest
import torch
from torch import nn


def test_recipe_schemes_and_rules():
    from experiments import recipes
    from mxq import matmul, scale_factor
    from mxq.nn import is_attention
    hw = recipes.HW_MXFP8_TAPEOUT
    assert hw.name == "hw_mxfp8_tapeout"
    assert recipes.OPERANDS.keywords == {"fmt": "MXFP8_E4M3", "axis": 0, "rounding_mode": "rne",
                                         "scale_floor": scale_factor.HARDWARE_FLOOR}
    assert scale_factor.HARDWARE_FLOOR == 2.0 ** -23
    assert recipes.ARITHMETIC.name == "compiled(mxgemmini(prod=e4m3))"
    assert recipes.LADDER == [(4, 4)] * 8 + [(4, 5)] * 2 + [(4, 6)] * 5 + [(8, 7)]
    assert hw.reduce.func is matmul.systolic and hw.reduce.keywords["schedule"] == recipes.LADDER
    R = recipes.RULES
    assert set(R) == {"none", "hw_mxfp8_tapeout", "hw_mxfp8_tapeout_proj", "hw_mxfp8_tapeout_core",
                      "hw_mxfp8_tapeout_all", "hw_mxfp8_tapeout_exactcore"}
    assert R["none"] is None
    assert R["hw_mxfp8_tapeout"] == [(is_attention, None), (nn.Linear, hw)]
    assert R["hw_mxfp8_tapeout_proj"] == [(nn.Linear, hw)]
    core = R["hw_mxfp8_tapeout_all"]
    assert core[0][1] == (hw, hw) and core[1:] == [(nn.Linear, hw)]
    assert R["hw_mxfp8_tapeout_exactcore"][0][1][0].name == "exact"


def test_windows():
    from experiments.llm_ppl import windows
    ids = torch.arange(1000)
    w = windows(ids, 64, 0, 0)
    assert w.shape == (15, 64) and torch.equal(w.reshape(-1), ids[:960])
    assert torch.equal(windows(ids, 64, 4, None), w[:4])
    s = windows(ids, 64, 5, 3)
    torch.manual_seed(3)
    assert torch.equal(s, w[torch.randperm(15)[:5]])
    assert len({int(r[0]) for r in s}) == 5 and torch.equal(windows(ids, 64, 5, 3), s)
    assert torch.equal(windows(ids, 64, 99, 3), w)
    with pytest.raises(ValueError, match="fewer than one window"):
        windows(ids[:10], 64, 1, 0)


def _tiny(tmp_path):
    from transformers import LlamaConfig, LlamaForCausalLM
    cfg = LlamaConfig(vocab_size=96, hidden_size=64, intermediate_size=96, num_hidden_layers=2,
                      num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=64)
    torch.manual_seed(0)
    model = LlamaForCausalLM(cfg).eval()
    path = tmp_path / "tiny"
    model.save_pretrained(path)
    return model, str(path)


def test_sample_nll_is_cross_entropy(tmp_path):
    from experiments.llm_ppl import perplexity, sample_nll
    model, _ = _tiny(tmp_path)
    ids = torch.randint(0, 96, (40,), generator=torch.Generator().manual_seed(1))
    nll, n = sample_nll(model, ids)
    with torch.no_grad():
        logits = model(ids[None]).logits[0].float()
    want = F_cross_entropy(logits[:-1], ids[1:])
    assert n == 39 and math.isclose(nll, want, rel_tol=1e-6)
    assert math.isclose(perplexity([{"nll": nll, "tokens": n}, {"nll": 2 * nll, "tokens": n}]),
                        math.exp(3 * nll / (2 * n)))


def F_cross_entropy(logits, target):
    return float(torch.nn.functional.cross_entropy(logits, target, reduction="sum"))


def test_command_on_saved_model(tmp_path):
    """The whole command, rules "none", on the CPU: the record's perplexity is exp of the per-window NLLs the
    model gives; an unknown rule list is refused."""
    from experiments import llm_ppl
    model, path = _tiny(tmp_path)
    stream = np.random.default_rng(2).integers(0, 96, 300).astype(np.int64)
    tok = tmp_path / "ids.npy"
    np.save(tok, stream)
    out = tmp_path / "r.json"
    rec = llm_ppl.main(["--rules", "none", "--model", path, "--tokens", str(tok), "--seqlen", "48",
                        "--nsamples", "3", "--seed", "1", "--device", "cpu", "--dtype", "float32",
                        "--out", str(out)])
    assert json.loads(out.read_text())["perplexity"] == rec["perplexity"]
    ids = llm_ppl.windows(torch.from_numpy(stream), 48, 3, 1)
    got = [(s["nll"], s["tokens"]) for s in rec["per_sample"]]
    want = [llm_ppl.sample_nll(model, ids[i]) for i in range(3)]
    assert all(math.isclose(a, b, rel_tol=1e-5) and n == m for (a, n), (b, m) in zip(got, want))
    assert rec["rules"] == "none" and rec["layers"] == [] and rec["seed"] == 1
    with pytest.raises(SystemExit, match="unknown rules"):
        llm_ppl.main(["--rules", "nope", "--model", path, "--tokens", str(tok)])
