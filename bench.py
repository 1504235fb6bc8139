"""Benchmark: emulated MX GEMM throughput of matmul.systolic (bit-exact MXGEMMINI, HW_FINAL ladder) on one GPU,
plus block-quantize HBM throughput, the LUT pipeline, the attention core, the adder and anchor trees and the
matrix-core comparison product, each next to its roofline, and the oracle's CPU rate.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-extra]
    python bench.py --copy-calibration        # only a 256 MiB device copy, 5 times (counter calibration)
    python bench.py --only LINE               # one extra line alone: quantize, lut, attend, mfma, trees, llm

A step is one systolic call over the benchmark workload (A = x^T with x 512 x 4096 ~ N(0,1), B = W^T with
W 4096 x 4096 ~ N(0, 0.02), both block.mxgemmini MXFP8_E4M3 codes along K: M = 512, N = 4096, K = 4096),
operands and scales resident in HBM.  `value` is emulated GEMM ops per second (2 per MAC) over the timed
steps.  `roofline.achieved` uses the fast systolic kernel's own average duration, timed with HIP events the
library records around each of its launches on the launch's stream.  One JSON line is printed.
"""
import argparse
import json
import os
import platform
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(REPO, "microscaling-quant_amd"))
sys.path.insert(0, REPO)

METRIC = "emulated MX GEMM GOP/s (systolic, bit-exact) + quantize GB/s vs HBM roofline"
HBM_PEAK_GBS = 8000.0
# MI355X's published vector FP32 peak, 157.3 TFLOP/s, is 78.6 T FMA lane-operations per second: the rate at which
# its 1024 SIMDs retire 32-bit VALU lanes (256 CUs x 128 lanes/clk x 2.4 GHz).  The fast systolic kernel is
# measured above the single-issue 64 lanes/clk/CU figure (SQ_INSTS_VALU x 64 / duration = 45.5 T lane-ops/s),
# so the 128-lane rate is the ceiling it is held against.
VALU_LANE_OPS = 157.3e12 / 2
OPS_PER_MAC_MODEL = 10                      # canonical datapath primitives per emulated MAC
VALU_ROOF_TOPS = VALU_LANE_OPS / OPS_PER_MAC_MODEL * 2 / 1e12   # 15.73 TOP/s emulated
FP8_PEAK_TFLOPS = 5000.0                    # MI355X dense FP8 matrix-core peak


def _events_ms(fn, steps, stream):
    import torch
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record(stream)
    for _ in range(steps):
        fn()
    end.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps


def _kernel_ms(fn, steps, kernel):
    """Average duration of the library kernel `kernel` over `steps` calls of fn (library HIP events)."""
    import torch

    from mxq import _lib
    torch.cuda.synchronize()
    _lib.timer_read(kernel)                                  # drop anything recorded before
    _lib.timer_enable(True)
    try:
        for _ in range(steps):
            fn()
    finally:
        _lib.timer_enable(False)
    total, n = _lib.timer_read(kernel)
    return total / n if n else None, n


def _traffic(name):
    """HBM bytes per launch for `name` from profiles/<name>_traffic.txt ("bytes_per_launch: N"), else None."""
    path = os.path.join(REPO, "profiles", f"{name}_traffic.txt")
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("bytes_per_launch:"):
                    return float(line.split(":", 1)[1])
    except OSError:
        pass
    return None


def _oracle_columns(ops):
    """One worker's share of the CPU baseline: the oracle systolic on a column slice; returns its seconds."""
    from oracle import numerics as nx
    from oracle import systolic as osys
    t0 = time.perf_counter()
    osys.systolic(*ops, nx.MXGEMMINI(), osys.HW_FINAL)
    return time.perf_counter() - t0


def cpu_baseline_systolic(x, W, cols_per_core=32):
    """The oracle (numpy port of the reference's reducer) on the benchmark's operands, over a column slice of
    B: one slice of cols_per_core columns per host core, in a process pool.  Output columns are independent
    chains, so the slice is a fair sample of the whole.  It runs before anything touches the GPU (the pool
    forks), on codes the oracle's own quantizer makes from the same x and W (the GPU's codes equal them bit for
    bit: tests/test_quantize_gpu.py).  cores = the CPUs this process may use, at most 16 (the box's share)."""
    import multiprocessing as mp

    from oracle import block as ob
    cores = max(1, min(16, len(os.sched_getaffinity(0))))
    cols = cols_per_core * cores
    pa, xa = ob.mxgemmini_quantize(x.t().contiguous().numpy(), "MXFP8_E4M3", 0)
    pb, xb = ob.mxgemmini_quantize(W[:cols].t().contiguous().numpy(), "MXFP8_E4M3", 0)
    K, M = pa.shape
    parts = [(pa, xa, pb[:, c:c + cols_per_core], xb[:, c:c + cols_per_core]) for c in range(0, cols, cols_per_core)]
    t0 = time.perf_counter()
    with mp.get_context("fork").Pool(cores) as pool:
        each = pool.map(_oracle_columns, parts)
    dt = time.perf_counter() - t0
    macs = K * M * cols
    one = 2 * K * M * cols_per_core / (sum(each) / len(each)) / 1e9
    return {"value": round(2 * macs / dt / 1e9, 4), "unit": "GOP/s", "cores": cores, "kind": "port",
            "single_core_GOPs": round(one, 4),
            "sample": f"oracle systolic MXGEMMINI HW_FINAL on the benchmark's codes, M={M} x N={cols} columns "
                      f"({cols_per_core} per core) x K={K} ({macs / 1e6:.1f} M MAC, {dt:.1f} s wall, "
                      f"{sum(each):.1f} s of CPU work, numpy, {cores} processes, "
                      f"{platform.processor() or platform.machine()})"}


def quantize_lines(torch, steps):
    """block.mxgemmini on bf16 8192 x 8192 (5 formats, rne) and block.ocp quantize + dequantize on 4096 x 512
    fp32 with rotating buffers past the 256 MB last-level cache: GB/s of algorithmic bytes."""
    from mxq import block
    dev = torch.device("cuda", 0)
    g = torch.Generator(device="cpu").manual_seed(2)
    t = torch.distributions.StudentT(torch.tensor(3.0)).sample((8192, 8192)) * 0.5
    idx = torch.randperm(8192 * 8192, generator=g)[:67109]
    t.view(-1)[idx] *= 100
    V = t.to(torch.bfloat16).to(dev)
    s = torch.cuda.current_stream(dev)
    out, kern = {}, {}
    bytes_c3 = 8192 * 8192 * 2 + 8192 * 8192 * 4 + 256 * 8192 * 4
    for fmt in ("MXFP8_E4M3", "MXFP8_E5M2", "MXFP6_E3M2", "MXFP6_E2M3", "MXFP4"):
        fn = lambda: block.mxgemmini.quantize(V, fmt, axis=0, rounding_mode="rne")   # noqa: E731
        fn()
        ms = _events_ms(fn, steps, s)
        out[fmt] = round(bytes_c3 / ms / 1e6, 1)
        kms, _ = _kernel_ms(fn, steps, "block_quantize")
        kern[fmt] = round(bytes_c3 / kms / 1e6, 1) if kms else None
    # the same quantize written as code and E8M0 bytes in one pass (mxq.packed, not in the reference)
    import mxq
    bytes_pk = 8192 * 8192 * 2 + 8192 * 8192 + 256 * 8192
    pk, pk_kern = {}, {}
    for fmt in ("MXFP8_E4M3", "MXFP8_E5M2", "MXFP6_E3M2", "MXFP6_E2M3", "MXFP4"):
        fn = lambda: mxq.packed.quantize(V, fmt, rounding_mode="rne", check=False)            # noqa: E731
        fn()
        ms = _events_ms(fn, steps, s)
        pk[fmt] = round(bytes_pk / ms / 1e6, 1)
        kms, _ = _kernel_ms(fn, steps, "block_quantize")
        pk_kern[fmt] = round(bytes_pk / kms / 1e6, 1) if kms else None
    del V
    # 17 MB per call: rotate over 64 inputs (1.1 GB with outputs) so HBM, not the cache, serves them
    rot = [torch.randn(4096, 512, device=dev) for _ in range(64)]
    bytes_c1 = 4096 * 512 * 4 * 2 + 128 * 512 * 4
    i = [0]

    def q1():
        block.ocp.quantize(rot[i[0] % 64], "MXFP8_E4M3", axis=0)
        i[0] += 1
    q1()
    ms1 = _events_ms(q1, 64, s)
    kms1, _ = _kernel_ms(q1, 64, "block_quantize")
    P, X = block.ocp.quantize(rot[0], "MXFP8_E4M3", axis=0)
    ms1d = _events_ms(lambda: block.ocp.dequantize(P, X, axis=0), 64, s)
    return {"mxgemmini_bf16_8192x8192_rne_GBs": out, "mxgemmini_bf16_8192x8192_rne_kernel_GBs": kern,
            "mxgemmini_bytes_per_call": bytes_c3,
            "packed_bf16_8192x8192_rne_GBs": pk, "packed_bf16_8192x8192_rne_kernel_GBs": pk_kern,
            "packed_bytes_per_call": bytes_pk,
            "ocp_e4m3_4096x512_quantize_GBs": round(bytes_c1 / ms1 / 1e6, 1),
            "ocp_e4m3_4096x512_quantize_kernel_GBs": round(bytes_c1 / kms1 / 1e6, 1) if kms1 else None,
            "ocp_e4m3_4096x512_dequantize_GBs_cache_resident": round(bytes_c1 / ms1d / 1e6, 1),
            "peak_GBs": HBM_PEAK_GBS}


def lut_line(torch, steps):
    """block.lut MXFP6_E3M2 (rne, 2^-23, group 1, 50 iterations) on two fp32 4096 x 4096 operands, then the
    systolic MXGEMMINI HW_FINAL product of the two LUT operands (K = M = N = 4096)."""
    from mxq import block, matmul
    dev = torch.device("cuda", 0)
    s = torch.cuda.current_stream(dev)
    A = torch.randn(4096, 4096, generator=torch.Generator().manual_seed(0)).to(dev)
    B = torch.randn(4096, 4096, generator=torch.Generator().manual_seed(1)).to(dev)
    q = lambda V: block.lut.quantize(V, "MXFP6_E3M2", 0, 32, rounding_mode="rne", scale_floor=2.0 ** -23,  # noqa
                                     group=1, max_iters=50)
    PA, XA = q(A)
    PB, XB = q(B)
    ms_q = _events_ms(lambda: q(A), steps, s)
    mm = lambda: matmul.systolic(PA, XA, PB, XB, matmul.MXGEMMINI(), matmul.HW_FINAL)        # noqa: E731
    mm()
    ms_mm = _events_ms(mm, steps, s)
    kms, _ = _kernel_ms(mm, steps, "systolic_fast")
    macs = 4096 ** 3
    return {"workload": "block.lut MXFP6_E3M2 4096x4096 (tables, pick, lookup) + systolic 4096^3",
            "lut_quantize_ms": round(ms_q, 3), "systolic_ms": round(ms_mm, 3),
            "systolic_TOPs": round(2 * macs / ms_mm / 1e9, 3),
            "systolic_kernel_TOPs": round(2 * macs / kms / 1e9, 3) if kms else None}


def attend_line(torch, steps):
    """mxq.nn.attend, Llama-3-8B-shaped: 1 x 32 heads x 2048 x 128, causal HF eager mask, Q K^T and P V through
    the MXGEMMINI MXFP8_E4M3 Scheme, softmax in fp32."""
    from functools import partial

    import mxq
    from mxq import Scheme, block, matmul
    dev = torch.device("cuda", 0)
    s = torch.cuda.current_stream(dev)
    qz = partial(block.mxgemmini.quantize, fmt="MXFP8_E4M3", axis=0)
    hw = Scheme("hw", a=qz, b=qz, reduce=partial(matmul.systolic, arith=matmul.MXGEMMINI(), schedule=matmul.HW_FINAL))
    q, k, v = (torch.randn(1, 32, 2048, 128, generator=torch.Generator().manual_seed(i)).to(dev) for i in range(3))
    mask = torch.triu(torch.full((2048, 2048), torch.finfo(torch.float32).min), 1)[None, None].to(dev)
    fn = lambda: mxq.nn.attend(q, k, v, mask, 128 ** -0.5, hw, hw)                      # noqa: E731
    fn()
    ms = _events_ms(fn, steps, s)
    macs = 2 * 32 * 2048 * 2048 * 128
    return {"workload": "nn.attend 1x32x2048x128 causal, MXGEMMINI MXFP8_E4M3 Scheme for QK^T and PV",
            "ms": round(ms, 3), "emulated_TOPs": round(2 * macs / ms / 1e9, 3)}


def llm_line(torch, steps):
    """experiments.llm_ppl's loss on a TinyLlama-1.1B-shaped Llama (22 layers, hidden 2048, MLP 5632, 32 heads,
    4 KV heads, vocab 32000), random-init in bf16, patched with the hw_mxfp8_tapeout rules (every MLP Linear
    and lm_head through the systolic Scheme), one window of 2048 synthetic tokens.  Opt-in (--only llm)."""
    from transformers import LlamaConfig, LlamaForCausalLM

    from experiments import llm_ppl, recipes
    from mxq.nn import patch
    dev = torch.device("cuda", 0)
    s = torch.cuda.current_stream(dev)
    cfg = LlamaConfig(vocab_size=32000, hidden_size=2048, intermediate_size=5632, num_hidden_layers=22,
                      num_attention_heads=32, num_key_value_heads=4, max_position_embeddings=2048)
    torch.manual_seed(0)
    with torch.device(dev):
        model = LlamaForCausalLM(cfg).to(torch.bfloat16).eval()
    ids = torch.randint(0, 32000, (2048,), generator=torch.Generator().manual_seed(1))
    llm_ppl.sample_nll(model, ids)                                            # warm-up (library handles)
    base_ms = _events_ms(lambda: llm_ppl.sample_nll(model, ids), steps, s)
    handle = patch(model, recipes.RULES["hw_mxfp8_tapeout"])
    nll, n = llm_ppl.sample_nll(model, ids)                                   # also caches the weight codes
    ms = _events_ms(lambda: llm_ppl.sample_nll(model, ids), steps, s)
    macs = sum(2048 * k * m for _, k, m, _, scheme in handle.table if scheme)
    return {"workload": "experiments.llm_ppl sample_nll, TinyLlama-1.1B-shaped random bf16 Llama, hw_mxfp8_tapeout "
                        "(MLP + lm_head), 2048 tokens",
            "ms": round(ms, 1), "tokens_per_s": round(2048 / ms * 1e3, 1), "bf16_unpatched_ms": round(base_ms, 1),
            "emulated_macs": macs, "emulated_TOPs_incl_rest": round(2 * macs / ms / 1e9, 3),
            "nll_per_token": round(nll / n, 4)}


def trees_line(torch, steps, P_A, X_A, P_B, X_B):
    """The other two reducers on the benchmark's own codes (M = 512, N = 4096, K = 4096), MXGEMMINI, size 16:
    matmul.adder_tree with bf16 at every level and with the README's ladder [(4, 4), (4, 5), (4, 6), (8, 7)],
    and matmul.anchor_tree with its defaults (one 16-product tree per reduction, bf16 out, truncating 20-bit
    levels).  Emulated ops as for systolic, over the fast kernel's own duration (the general kernel that follows
    it computes only flagged tiles: none on these codes)."""
    from mxq import matmul
    dev = P_A.device
    s = torch.cuda.current_stream(dev)
    ar = matmul.MXGEMMINI()
    macs = P_A.shape[0] * P_A.shape[1] * P_B.shape[1]
    out = {"workload": "adder_tree (size 16: bf16 levels; e4m4, e4m5, e4m6, bf16 levels) and anchor_tree "
                       "(defaults), MXGEMMINI, on the systolic benchmark's codes"}
    ladder = [(4, 4), (4, 5), (4, 6), (8, 7)]
    for name, kernel, fn in (
            ("adder_tree_bf16", "adder_fast", lambda: matmul.adder_tree(P_A, X_A, P_B, X_B, ar, [(8, 7)] * 4)),
            ("adder_tree_ladder", "adder_fast", lambda: matmul.adder_tree(P_A, X_A, P_B, X_B, ar, ladder)),
            ("anchor_tree", "anchor_fast", lambda: matmul.anchor_tree(P_A, X_A, P_B, X_B, ar))):
        fn()
        ms = _events_ms(fn, steps, s)
        kms, _ = _kernel_ms(fn, steps, kernel)
        gms, _ = _kernel_ms(fn, steps, kernel.replace("_fast", "_tree"))
        out[name] = {"ms": round(ms, 3), "kernel": kernel, "kernel_ms": round(kms, 3) if kms else None,
                     "general_kernel_ms": round(gms, 4) if gms else None,
                     "emulated_TOPs": round(2 * macs / (kms or ms) / 1e9, 3)}
    return out


def mfma_line(torch, steps, P_A, X_A, P_B, X_B):
    """mfma_accum (the matrix-core comparison product) on the benchmark's own codes: pack both operands to FP8
    and E8M0 bytes, then V_MFMA_SCALE_F32_32X32X64_F8F6F4.  The kernel rate is held against MI355X's dense FP8
    peak, 5.0 PFLOP/s."""
    import mxq
    dev = P_A.device
    s = torch.cuda.current_stream(dev)
    fn = lambda: mxq.mfma_accum(P_A, X_A, P_B, X_B, "MXFP8_E4M3")                # noqa: E731
    fn()
    ms = _events_ms(fn, steps, s)
    kms, _ = _kernel_ms(fn, steps, "mx_mfma")
    flops = 2 * P_A.shape[0] * P_A.shape[1] * P_B.shape[1]
    k_tf = flops / (kms / 1e3) / 1e12 if kms else None
    return {"workload": "mfma_accum on the same MXFP8_E4M3 codes (M = 512, N = 4096, K = 4096)",
            "ms": round(ms, 4), "kernel": "k_mx_mfma<0, 0, 1>", "kernel_ms": round(kms, 4) if kms else None,
            "kernel_TFLOPs": round(k_tf, 2) if k_tf else None, "peak_TFLOPs": FP8_PEAK_TFLOPS,
            "frac": round(k_tf / FP8_PEAK_TFLOPS, 4) if k_tf else None}


def copy_calibration():
    """A plain device copy of 256 MiB, five times: the reference point for the FETCH_SIZE / WRITE_SIZE
    counters (each launch reads and writes 262144 KiB)."""
    import torch
    x = torch.empty(64 * 1024 * 1024, dtype=torch.float32, device="cuda")
    y = torch.empty_like(x)
    x.fill_(1.0)
    for _ in range(5):
        y.copy_(x)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes_per_launch": x.numel() * 4, "launches": 5}), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-extra", action="store_true", help="only the systolic line (no quantize, LUT, attend)")
    ap.add_argument("--copy-calibration", action="store_true", help="run only the counter-calibration copy")
    ap.add_argument("--only", choices=("quantize", "lut", "attend", "mfma", "trees", "llm"),
                    help="run one extra line alone (for profiling) and print it; not the benchmark line")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU; --gpus {args.gpus} is not supported (the systolic path "
              "would shard over output columns with one final all-gather)", file=sys.stderr)
        sys.exit(2)
    if args.copy_calibration:
        copy_calibration()
        return

    import torch

    M, N, K = 512, 4096, 4096
    g = torch.Generator().manual_seed(0)
    x = torch.randn(M, K, generator=g)
    W = torch.randn(N, K, generator=g) * 0.02
    # the CPU baseline forks its worker pool, so it runs before anything touches the GPU
    cpu = cpu_baseline_systolic(x, W) if not args.no_cpu and args.only is None else None

    import mxq  # noqa: F401
    from mxq import block, matmul
    dev = torch.device("cuda", 0)
    if args.only in ("quantize", "lut", "attend", "llm"):
        fn = {"quantize": lambda: quantize_lines(torch, max(5, args.steps // 2)),
              "lut": lambda: lut_line(torch, 3), "attend": lambda: attend_line(torch, 3),
              "llm": lambda: llm_line(torch, 2)}[args.only]
        print(json.dumps({"only": args.only, args.only: fn()}), flush=True)
        return
    P_A, X_A = block.mxgemmini.quantize(x.t().contiguous().to(dev), "MXFP8_E4M3", axis=0)
    P_B, X_B = block.mxgemmini.quantize(W.t().contiguous().to(dev), "MXFP8_E4M3", axis=0)
    ar = matmul.MXGEMMINI()
    if args.only in ("mfma", "trees"):
        fn = {"mfma": lambda: mfma_line(torch, max(5, args.steps // 2), P_A, X_A, P_B, X_B),
              "trees": lambda: trees_line(torch, 3, P_A, X_A, P_B, X_B)}[args.only]
        print(json.dumps({"only": args.only, args.only: fn()}), flush=True)
        return
    step = lambda: matmul.systolic(P_A, X_A, P_B, X_B, ar, matmul.HW_FINAL)   # noqa: E731
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    s = torch.cuda.current_stream(dev)
    t0 = time.perf_counter()
    ms = _events_ms(step, args.steps, s)
    wall = time.perf_counter() - t0
    kms, launches = _kernel_ms(step, args.steps, "systolic_fast")
    macs = M * N * K
    gops = 2 * macs / (ms / 1e3) / 1e9
    k_tops = 2 * macs / (kms / 1e3) / 1e12 if kms else None
    line = {
        "metric": METRIC, "value": round(gops, 2), "unit": "GOP/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32", "data": "synthetic (seeded N(0,1) activations, N(0,0.02) weights)",
        "config": {"workload": "matmul.systolic MXGEMMINI HW_FINAL on block.mxgemmini MXFP8_E4M3 codes, "
                               "A = x^T (x 512x4096), B = W^T (W 4096x4096)", "M": M, "N": N, "K": K,
                   "emulated_macs_per_step": macs, "timed_wall_s": round(wall, 3)},
        "roofline": {"bound": "valu", "achieved": round(k_tops, 4) if k_tops else None,
                     "peak": round(VALU_ROOF_TOPS, 3), "unit": "TOP/s",
                     "frac": round(k_tops / VALU_ROOF_TOPS, 4) if k_tops else None,
                     "traffic": _traffic("systolic_fast_c2"),
                     "kernel": "k_systolic_fast<16, true>", "kernel_ms": round(kms, 4) if kms else None,
                     "kernel_launches_timed": launches,
                     "note": "VALU-bound emulation (neither HBM nor MFMA): achieved = 2 x 8,589,934,592 emulated "
                             "MACs / the fast kernel's average duration; peak = MI355X vector FP32 157.3 TFLOP/s "
                             "= 78.6 T 32-bit lane-ops/s, / 10 lane-ops per emulated MAC (the datapath's primitive "
                             "count) x 2 ops per MAC; the kernel executes 8.1 VALU lane-ops per MAC "
                             "(SQ_INSTS_VALU, profiles/systolic_fast_c2_valu.txt)"},
    }
    if not args.no_extra:
        line["quantize"] = quantize_lines(torch, max(5, args.steps // 2))
        line["lut_c4"] = lut_line(torch, 3)
        line["attend_c5"] = attend_line(torch, 3)
        line["mfma_c2"] = mfma_line(torch, max(5, args.steps // 2), P_A, X_A, P_B, X_B)
        line["trees_c2"] = trees_line(torch, 3, P_A, X_A, P_B, X_B)
    if cpu is not None:
        line["cpu_baseline"] = cpu
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
