"""Perplexity of a causal LM under a rule list of experiments.recipes, on one GPU
(experiments/llm_ppl.py of the reference: the same windows, loss and record).

    python -m experiments.llm_ppl --rules hw_mxfp8_tapeout --model /models/TinyLlama --text wiki.test.raw
    python -m experiments.llm_ppl --rules hw_mxfp8_tapeout --model /models/TinyLlama --tokens ids.npy --dry-run

Everything is read from local paths (no hub names, no dataset downloads): --model is a directory written by
save_pretrained; the token stream is either --tokens (a 1-D int array, .npy or a tensor saved by torch.save)
or --text (a text file of non-empty lines joined with blank lines, as WikiText-2 is, tokenized with the
model's tokenizer).  The stream is cut into windows of --seqlen tokens; --nsamples of them are drawn with
--seed (torch.manual_seed, then randperm, MXQuant's protocol), or the first ones with --sequential, or all
with --nsamples 0.  A window's loss is the summed token NLL of the next-token log-softmax in float32; the
perplexity is exp(sum of NLL / sum of tokens), summed in window order.

One process, one GPU: the reference's multi-GPU launcher (samples split over worker processes) is left out,
its sums being the same single-process loop's.
"""
import argparse
import json
import math
import subprocess
import sys
import time
from functools import partial
from pathlib import Path
from typing import Optional

import torch
import torch.nn.functional as F

_HERE = Path(__file__).resolve().parent


def load_model(path: str, seqlen: int, dtype=torch.bfloat16, device: str = "cuda"):
    """A causal LM from a local directory; linear RoPE scaling when seqlen exceeds its context."""
    from transformers import AutoConfig, AutoModelForCausalLM
    config = AutoConfig.from_pretrained(path, local_files_only=True)
    ctx = getattr(config, "max_position_embeddings", None)
    if ctx and seqlen > ctx:
        config.rope_scaling = {"type": "linear", "factor": float(math.ceil(seqlen / ctx))}
    model = AutoModelForCausalLM.from_pretrained(path, config=config, torch_dtype=dtype, local_files_only=True)
    return model.eval().to(device=device, dtype=dtype)


def token_stream(tokens: Optional[str] = None, text: Optional[str] = None, model_path: Optional[str] = None):
    """The 1-D int64 token stream: from an array file, or a text file tokenized with the model's tokenizer."""
    if tokens is not None:
        if tokens.endswith(".npy"):
            import numpy as np
            return torch.from_numpy(np.load(tokens, allow_pickle=False)).long().reshape(-1)
        return torch.load(tokens, weights_only=True).long().reshape(-1)
    if text is None or model_path is None:
        raise ValueError("token_stream: give tokens, or text and model_path")
    from transformers import AutoTokenizer
    tok = AutoTokenizer.from_pretrained(model_path, local_files_only=True)
    lines = Path(text).read_text().splitlines()
    joined = "\n\n".join(x for x in lines if x.strip())
    return tok(joined, return_tensors="pt")["input_ids"][0]


def windows(ids: torch.Tensor, seqlen: int, nsamples: int, seed: Optional[int]) -> torch.Tensor:
    """The stream cut into whole windows of seqlen tokens; nsamples of them (0, or at least all: every one),
    drawn by seed, or the first ones when seed is None."""
    nbatch = ids.numel() // seqlen
    if nbatch == 0:
        raise ValueError(f"windows: the stream has {ids.numel()} tokens, fewer than one window of {seqlen}")
    w = ids[: nbatch * seqlen].reshape(nbatch, seqlen)
    if nsamples == 0 or nsamples >= nbatch:
        return w
    if seed is None:
        return w[:nsamples]
    torch.manual_seed(seed)
    return w[torch.randperm(nbatch)[:nsamples]]


@torch.no_grad()
def sample_nll(model, ids: torch.Tensor):
    """(summed NLL, tokens) of one window: each next token under the float32 log-softmax of the logits."""
    device = next(model.parameters()).device
    ids = ids.unsqueeze(0).to(device)
    logits = model(ids, use_cache=False).logits[0, :-1, :]
    nll = -F.log_softmax(logits.float(), dim=-1).gather(1, ids[0, 1:].unsqueeze(1)).squeeze(1)
    return nll.sum().item(), nll.numel()


def perplexity(per_sample) -> float:
    """exp(mean NLL per token), the sums taken in window order."""
    total, tokens = 0.0, 0
    for s in per_sample:
        total += s["nll"]
        tokens += s["tokens"]
    return math.exp(total / tokens)


def describe(obj):
    """A Scheme, rule list or any piece of one as plain JSON, read off the objects themselves."""
    from mxq import Scheme
    from mxq.matmul import Arithmetic
    if isinstance(obj, Scheme):
        return {"name": obj.name, "a": describe(obj.a), "b": describe(obj.b), "reduce": describe(obj.reduce)}
    if isinstance(obj, partial):
        return {"call": describe(obj.func), **{k: describe(v) for k, v in obj.keywords.items()}}
    if isinstance(obj, Arithmetic):
        return obj.name
    if isinstance(obj, type) or callable(obj):
        public = [m for m in obj.__module__.split(".") if not m.startswith("_")]
        return ".".join(public + [obj.__qualname__])
    if isinstance(obj, (list, tuple)):
        return [describe(v) for v in obj]
    return obj


def _commit() -> str:
    r = subprocess.run(["git", "-C", str(_HERE), "rev-parse", "--short", "HEAD"], capture_output=True, text=True)
    return r.stdout.strip()


def evaluate(model, ids: torch.Tensor, rules, *, label: str = "", vector=None, chunk: Optional[int] = None,
             cache_weights: bool = True, dry_run: bool = False, log=print):
    """Patch `model` with `rules` (None: as loaded), then the NLL of every window of `ids`.  Returns the
    record (None on a dry run, after logging the layer table)."""
    from mxq.nn import patch
    from mxq.nn._vector import resolve
    vector = resolve(vector)
    table, cores, norms = [], [], []
    if rules is not None or any(vector.values()):
        handle = patch(model, rules or [], chunk=chunk, dry_run=dry_run, cache_weights=cache_weights, vector=vector)
        table, cores, norms = handle.table, handle.cores, handle.norms
        if dry_run:
            log(str(handle))
            return None
    t0, per_sample = time.time(), []
    for i in range(ids.shape[0]):
        nll, n = sample_nll(model, ids[i])
        per_sample.append({"index": i, "nll": nll, "tokens": n})
        log(f"  [{label}] sample {i + 1}/{ids.shape[0]}  nll/token {nll / n:.6f}  {time.time() - t0:.1f}s")
    each = [x for _, v in (rules or []) for x in (v if isinstance(v, tuple) else (v,)) if x is not None]
    rule_list = [[describe(sel), None if v is None else [x.name for x in v] if isinstance(v, tuple) else v.name]
                 for sel, v in (rules or [])]
    record = {"rule_list": rule_list, "schemes": {x.name: describe(x) for x in each}, "layers": table,
              "cores": cores, "vector": vector, "rmsnorms": norms, "per_sample": per_sample,
              "seconds": time.time() - t0}
    record["perplexity"] = perplexity(per_sample)
    return record


def main(argv=None) -> Optional[dict]:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--rules", required=True, help="a key of experiments.recipes.RULES")
    ap.add_argument("--model", required=True, help="a local model directory (save_pretrained)")
    src = ap.add_mutually_exclusive_group(required=True)
    src.add_argument("--tokens", help="a 1-D token array (.npy, or a tensor saved with torch.save)")
    src.add_argument("--text", help="a text file, tokenized with the model's tokenizer")
    ap.add_argument("--seqlen", type=int, default=2048)
    ap.add_argument("--nsamples", type=int, default=16, help="windows; 0 = every window")
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--sequential", action="store_true", help="the first nsamples windows instead of seeded ones")
    ap.add_argument("--chunk", type=int, default=None, help="token rows per reducer call")
    ap.add_argument("--no-cache-weights", action="store_true", help="recompute weight codes every forward")
    ap.add_argument("--vector", choices=["none", "bf16"], default="none")
    ap.add_argument("--vector-ops", default="softmax,rmsnorm")
    ap.add_argument("--dtype", choices=["bfloat16", "float32"], default="bfloat16")
    ap.add_argument("--device", default="cuda")
    ap.add_argument("--out", default=None, help="result JSON (default: experiments/results/<label>.json)")
    ap.add_argument("--dry-run", action="store_true")
    args = ap.parse_args(argv)

    from experiments import recipes
    if args.rules not in recipes.RULES:
        raise SystemExit(f"unknown rules {args.rules!r}; known: {', '.join(recipes.RULES)}")
    rules = recipes.RULES[args.rules]
    ops = [op for op in args.vector_ops.split(",") if op]
    vector = None if args.vector == "none" else {op: args.vector for op in ops}
    label = args.rules + (f"_vec-{args.vector}-{'+'.join(ops)}" if vector else "") + \
        ("_fp32" if args.dtype == "float32" else "")
    seed = None if args.sequential else args.seed
    ids = windows(token_stream(args.tokens, args.text, args.model), args.seqlen, args.nsamples, seed)
    model = load_model(args.model, args.seqlen, getattr(torch, args.dtype), args.device)
    record = evaluate(model, ids, rules, label=label, vector=vector, chunk=args.chunk,
                      cache_weights=not args.no_cache_weights, dry_run=args.dry_run)
    if record is None:
        return None
    record = {"rules": args.rules, "model": args.model, "seqlen": args.seqlen, "nsamples": args.nsamples,
              "seed": seed, "mxq_commit": _commit(), "dtype": args.dtype, **record}
    out = Path(args.out or _HERE / "results" / f"{label}.json")
    out.parent.mkdir(parents=True, exist_ok=True)
    out.write_text(json.dumps(record, indent=1))
    print(f"PERPLEXITY [{label}] : {record['perplexity']:.6f}   ({len(record['per_sample'])} samples, "
          f"{record['seconds']:.0f}s)  -> {out}", flush=True)
    return record


if __name__ == "__main__":
    if str(_HERE.parent) not in sys.path:
        sys.path.insert(0, str(_HERE.parent))
    main()
