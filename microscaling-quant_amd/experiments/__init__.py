"""Experiments over the mxq path: the MX-Gemmini recipe (recipes) and the perplexity protocol (llm_ppl)."""
