"""experiments.llm_ppl on the GPU with the tapeout recipe: the whole command on a tiny random Llama saved to
disk, every window's NLL equal to the patched model's own forward, the layer table, and a dry run."""
import math

import numpy as np
import pytest
import torch

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
