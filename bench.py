"""Benchmark: emulated MX GEMM throughput of matmul.systolic (bit-exact MXGEMMINI, HW_FINAL ladder) on one GPU,
plus block-quantize HBM throughput, the LUT pipeline, the attention core, the adder and anchor trees and the
matrix-core comparison product, each next to its roofline, the oracle's CPU rate on the same work, and a
parity check of what was timed against the oracle.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-extra]
    python bench.py --copy-calibration        # only a 256 MiB device copy, 5 times (counter calibration)
    python bench.py --valu-rates              # only the VALU issue-rate probe, one instruction kind at a time
    python bench.py --only LINE               # one extra line alone: quantize, lut, attend, mfma, trees, llm

A step is one systolic call over the benchmark workload (A = x^T with x 512 x 4096 ~ N(0,1), B = W^T with
W 4096 x 4096 ~ N(0, 0.02), both block.mxgemmini MXFP8_E4M3 codes along K: M = 512, N = 4096, K = 4096),
operands and scales resident in HBM.  `value` is emulated GEMM ops per second (2 per MAC) over the timed
steps.  `roofline.achieved` uses the fast systolic kernel's own average duration, timed with HIP events the
library records around each of its launches on the launch's stream.  Kernels of some tens of microseconds (the
quantizers, the matrix-core product) are timed by replay instead, their recorded library calls issued back to
back between one pair of events, since an event pair per launch adds 15-20 us.  One JSON line is printed.

CPU baselines: the oracle (a numpy restatement of the reference's algorithms) on the host cores, in a process
pool forked before anything touches the GPU, on the same seeded inputs: C2 on a column slice, C1 and C3 at full
size, C4's LUT quantize at full size and its product on a column slice, C5 on two of its 32 heads.  The oracle's
results are then compared with the timed GPU outputs (`parity` in each line).
"""
import argparse
import hashlib
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
# MI355X's published vector FP32 peak, 157.3 TFLOP/s, is 78.6 T lane-operations per second: its 1024 SIMDs each
# retiring one full-rate wave64 VALU instruction every 2 clocks at 2.4 GHz.  gfx950 issues v_add_f32, v_mul_f32
# and v_and_b32 at that rate and v_rndne_f32, v_bfe_u32, v_add3_u32, the packed float16 operations, the mixed
# fma and the float16 and bf16 pack conversions at half of it (`--valu-rates`).
VALU_LANE_OPS = 157.3e12 / 2
# The emulated MAC's VALU issue on gfx950 in full-rate slots: an e4 lane step multiplies, masks the product,
# rounds it to the lane grid (adding and subtracting a constant, two full-rate operations, or v_rndne_f32 at half
# rate: 2 slots either way), adds exactly and rounds to nearest even at m bits (three full-rate operations) = 8.
# The roof prices every MAC at that step.
SLOTS_PER_MAC_MODEL = 8
VALU_ROOF_TOPS = VALU_LANE_OPS / SLOTS_PER_MAC_MODEL * 2 / 1e12   # 19.66 TOP/s emulated
# The algorithmic model of the reference's MAC (roofline.frac_survey_model): 10 lane-operations per emulated MAC
# (multiply, truncate, flush, saturate, the two lane roundings, the +0 fix-up, the exact add, its rounding, the
# zero short-circuit), priced at the same 78.6 T lane-operations per second; the fast kernel does the step in
# fewer, so this fraction can pass 1.
OPS_PER_MAC_MODEL10 = 10
MODEL10_ROOF_TOPS = VALU_LANE_OPS / OPS_PER_MAC_MODEL10 * 2 / 1e12    # 15.73 TOP/s emulated
VALU_PROBE_KINDS = ("v_add_f32", "v_mul_f32", "v_and_b32", "v_rndne_f32", "v_bfe_u32", "v_add3_u32", "v_pk_mul_f16",
                    "v_pk_add_f16", "v_fma_mix_f32", "v_cvt_pkrtz_f16_f32", "v_cvt_pk_bf16_f32")
VALU_CHAIN_KINDS = ("v_mul_f32", "v_pk_mul_f16")     # probe kinds 11 and 12: one dependent chain each
FP8_PEAK_TFLOPS = 5000.0                    # MI355X dense FP8 matrix-core peak
FP6_FP4_PEAK_TFLOPS = 10100.0               # MI355X dense FP6 and FP4 matrix-core peak
MAX_POOL = 16                               # host processes for the CPU baselines (one GPU's CPU share)

C3_FORMATS = ("MXFP8_E4M3", "MXFP8_E5M2", "MXFP6_E3M2", "MXFP6_E2M3", "MXFP4")
# C2 with its second seed, and with the tapeout recipe's operand quantizer (experiments/recipes.py:57-58)
C2_VARIANTS = {"seed1": ("x1", "W1", {}),
               "tapeout_operands": ("x", "W", {"rounding_mode": "rne", "scale_floor": 2.0 ** -23})}
C5_HEADS = (0, 31)


# ------------------------------------------------------------------------------------------------ inputs
def make_inputs(torch):
    """Every line's seeded synthetic input, on the CPU (the GPU lines copy them over)."""
    g = torch.Generator().manual_seed(0)
    x = torch.randn(512, 4096, generator=g)
    W = torch.randn(4096, 4096, generator=g) * 0.02
    g1 = torch.Generator().manual_seed(1)                    # C2's second seed, drawn the same way
    x1 = torch.randn(512, 4096, generator=g1)
    W1 = torch.randn(4096, 4096, generator=g1) * 0.02
    c1 = torch.randn(4096, 512, generator=torch.Generator().manual_seed(10))
    # C3: Student-t (df 3) x 0.5, 0.1 % of the entries (seeded positions) x 100, bfloat16
    torch.manual_seed(2)
    t = torch.distributions.StudentT(torch.tensor(3.0)).sample((8192, 8192)) * 0.5
    idx = torch.randperm(8192 * 8192, generator=torch.Generator().manual_seed(2))[:67109]
    t.view(-1)[idx] *= 100
    c3 = t.to(torch.bfloat16)
    del t
    c4a = torch.randn(4096, 4096, generator=torch.Generator().manual_seed(0))
    c4b = torch.randn(4096, 4096, generator=torch.Generator().manual_seed(1))
    q, k, v = (torch.randn(1, 32, 2048, 128, generator=torch.Generator().manual_seed(i)) for i in range(3))
    mask = torch.triu(torch.full((2048, 2048), torch.finfo(torch.float32).min), 1)[None, None]
    return {"x": x, "W": W, "x1": x1, "W1": W1, "c1": c1, "c3": c3, "c4a": c4a, "c4b": c4b, "q": q, "k": k, "v": v, "mask": mask}


def _digest(a):
    import numpy as np
    return hashlib.blake2b(np.ascontiguousarray(a).tobytes(), digest_size=16).hexdigest()


# -------------------------------------------------------------------------------- CPU baselines (oracle)
_DATA = {}                                   # numpy operands the forked workers read (copy on write)


def _task_systolic(ops):
    from oracle import numerics as nx
    from oracle import systolic as osys
    t0 = time.perf_counter()
    Y = osys.systolic(*ops, nx.MXGEMMINI(), osys.HW_FINAL)
    return time.perf_counter() - t0, Y


def _task_quant(job):
    from oracle import block as ob
    key, fmt, c0, c1 = job
    V = _DATA[key][:, c0:c1]
    t0 = time.perf_counter()
    if key == "c1":
        P, X = ob.ocp_quantize(V, fmt, 0)
    else:
        P, X = ob.mxgemmini_quantize(V, fmt, 0, 32, "rne")
    return time.perf_counter() - t0, _digest(P), _digest(X)


def _task_lut(job):
    from oracle import lut as ol
    key, c0, c1 = job
    t0 = time.perf_counter()
    P, X = ol.lut_quantize(_DATA[key][:, c0:c1], "MXFP6_E3M2", 0, 32, "rne", 2.0 ** -23, 1, 50)
    return time.perf_counter() - t0, P, X


def _pool_map(pool, fn, jobs):
    t0 = time.perf_counter()
    out = pool.map(fn, jobs, chunksize=1)
    return time.perf_counter() - t0, out


def _tiles(pa, xa, pb, xb, rows, cols):
    """Oracle systolic jobs over tiles of rows x cols outputs."""
    M, N = pa.shape[1], pb.shape[1]
    return [((r, c), (pa[:, r:r + rows], xa[:, r:r + rows], pb[:, c:c + cols], xb[:, c:c + cols]))
            for r in range(0, M, rows) for c in range(0, N, cols)]


def _assemble(M, N, where, parts):
    import numpy as np
    Y = np.zeros((M, N), np.float32)
    for (r, c), (_, y) in zip(where, parts):
        Y[r:r + y.shape[0], c:c + y.shape[1]] = y
    return Y


def cpu_baselines(inp, cores):
    """The oracle on every line's work, timed on `cores` host processes (forked here, before any GPU use).
    Returns {line: {"cpu_baseline": {...}, "oracle": what the parity check compares}}."""
    import multiprocessing as mp

    import numpy as np
    import torch

    from oracle import attend as oatt
    from oracle import block as ob
    host = f"{platform.processor() or platform.machine()}, numpy {np.__version__}"
    _DATA.update(c1=inp["c1"].numpy(), c3=inp["c3"].float().numpy(), c4a=inp["c4a"].numpy(),
                 c4b=inp["c4b"].numpy())
    out = {}
    with mp.get_context("fork").Pool(cores) as pool:
        # C2: the oracle systolic on the first 32 x cores columns of the benchmark's codes
        pa, xa = ob.mxgemmini_quantize(inp["x"].t().contiguous().numpy(), "MXFP8_E4M3", 0)
        ncol = 32 * cores
        pb, xb = ob.mxgemmini_quantize(inp["W"][:ncol].t().contiguous().numpy(), "MXFP8_E4M3", 0)
        jobs = _tiles(pa, xa, pb, xb, pa.shape[1], 32)
        dt, parts = _pool_map(pool, _task_systolic, [j for _, j in jobs])
        macs = pa.shape[0] * pa.shape[1] * ncol
        per_core = 2 * pa.shape[0] * pa.shape[1] * 32 / (sum(p[0] for p in parts) / len(parts)) / 1e9
        out["c2"] = {"cpu_baseline": {
            "value": round(2 * macs / dt / 1e9, 4), "unit": "GOP/s", "cores": cores, "kind": "port",
            "single_core_GOPs": round(per_core, 4),
            "sample": f"oracle systolic MXGEMMINI HW_FINAL on the benchmark's codes, M=512 x N={ncol} (columns "
                      f"0..{ncol - 1}, 32 per process) x K=4096: {macs / 1e6:.0f} M MAC, {dt:.1f} s wall, "
                      f"{sum(p[0] for p in parts):.1f} s of CPU work ({host})"},
            "oracle": _assemble(512, ncol, [w for w, _ in jobs], parts), "cols": ncol}
        # C2's variants on their first 32 columns: seed 1 (default quantizer), and seed 0 with the tapeout
        # recipe's operands (rne, floor 2^-23: experiments/recipes.py:57-58)
        var = {}
        for name, (xk, wk, kw) in C2_VARIANTS.items():
            va, vxa = ob.mxgemmini_quantize(inp[xk].t().contiguous().numpy(), "MXFP8_E4M3", 0, **kw)
            vb, vxb = ob.mxgemmini_quantize(inp[wk][:32].t().contiguous().numpy(), "MXFP8_E4M3", 0, **kw)
            var[name] = (va, vxa, vb, vxb)
        _, parts = _pool_map(pool, _task_systolic, list(var.values()))
        out["c2_variants"] = {name: p[1] for name, p in zip(var, parts)}
        # C1: block.ocp quantize of 4096 x 512 fp32, full size, 32 columns per job
        jobs = [("c1", "MXFP8_E4M3", c, c + 32) for c in range(0, 512, 32)]
        dt, parts = _pool_map(pool, _task_quant, jobs)
        nbytes = 4096 * 512 * 8 + 128 * 512 * 4
        out["c1"] = {"cpu_baseline": {
            "value": round(nbytes / dt / 1e9, 3), "unit": "GB/s", "cores": cores, "kind": "port",
            "sample": f"oracle block.ocp MXFP8_E4M3 quantize of the whole 4096 x 512 input, 16 column slices "
                      f"({dt:.2f} s wall, {sum(p[0] for p in parts):.2f} s of CPU work)"},
            "oracle": [(j, p[1], p[2]) for j, p in zip(jobs, parts)]}
        # C3: block.mxgemmini quantize of bf16 8192 x 8192, five formats, full size, 512 columns per job
        per_fmt, c3 = {}, {}
        for fmt in C3_FORMATS:
            jobs = [("c3", fmt, c, c + 512) for c in range(0, 8192, 512)]
            dt, parts = _pool_map(pool, _task_quant, jobs)
            per_fmt[fmt] = round((8192 * 8192 * 6 + 256 * 8192 * 4) / dt / 1e9, 3)
            c3[fmt] = [(j, p[1], p[2]) for j, p in zip(jobs, parts)]
        out["c3"] = {"cpu_baseline": {
            "value": per_fmt, "unit": "GB/s", "cores": cores, "kind": "port",
            "sample": "oracle block.mxgemmini (rne) quantize of the whole bf16 8192 x 8192 input per format, 16 "
                      "column slices; bytes as the GPU line counts them (bf16 in, float32 P and X out)"},
            "oracle": c3}
        # C4: block.lut of both 4096 x 4096 operands at full size (256 columns per job, whole column groups),
        # then the LUT x LUT product on its last 32 columns (all 4096 rows, 256 per job)
        lut = {}
        for key in ("c4a", "c4b"):
            jobs = [(key, c, c + 256) for c in range(0, 4096, 256)]
            dt, parts = _pool_map(pool, _task_lut, jobs)
            lut[key] = (dt, np.concatenate([p[1] for p in parts], axis=1), np.concatenate([p[2] for p in parts], axis=1))
        pa, xa = lut["c4a"][1], lut["c4a"][2]
        pb, xb = lut["c4b"][1][:, 4064:], lut["c4b"][2][:, 4064:]
        jobs = _tiles(pa, xa, pb, xb, 256, 32)
        dt_mm, parts = _pool_map(pool, _task_systolic, [j for _, j in jobs])
        mm_macs = 4096 * 4096 * 32
        out["c4"] = {"cpu_baseline": {
            "value": {"lut_quantize_ms": round(lut["c4a"][0] * 1e3, 1),
                      "systolic_GOPs": round(2 * mm_macs / dt_mm / 1e9, 4)},
            "unit": "ms (block.lut of one operand), GOP/s (systolic)", "cores": cores, "kind": "port",
            "sample": f"oracle block.lut MXFP6_E3M2 of a whole 4096 x 4096 operand (16 column slices); the oracle "
                      f"systolic on columns 4064..4095 of the 4096^3 LUT x LUT product ({mm_macs / 1e6:.0f} M MAC, "
                      f"{dt_mm:.1f} s wall)"},
            "oracle": {"PA": lut["c4a"][1], "XA": lut["c4a"][2], "PB": lut["c4b"][1], "XB": lut["c4b"][2],
                       "Y_cols": _assemble(4096, 32, [w for w, _ in jobs], parts)}}
        # C5: the oracle attend on heads 0 and 31 (each its own KV head), torch's CPU softmax, reduces in the pool

        def reduce(pa, xa, pb, xb):
            rows = max(1, min(pa.shape[1], (1 << 14) // max(1, min(pb.shape[1], 64))))
            jobs = _tiles(pa, xa, pb, xb, rows, min(pb.shape[1], 64))
            parts = pool.map(_task_systolic, [j for _, j in jobs], chunksize=1)
            return _assemble(pa.shape[1], pb.shape[1], [w for w, _ in jobs], parts)

        qz = lambda V: ob.mxgemmini_quantize(V, "MXFP8_E4M3", 0)                  # noqa: E731
        side = oatt.Side(qz, qz, reduce)
        sm = lambda S: torch.softmax(torch.from_numpy(np.ascontiguousarray(S)), dim=-1).numpy()   # noqa: E731
        hs = list(C5_HEADS)
        t0 = time.perf_counter()
        o = oatt.attend(inp["q"][:, hs].numpy(), inp["k"][:, hs].numpy(), inp["v"][:, hs].numpy(),
                        inp["mask"].numpy(), 128 ** -0.5, side, side, sm)
        dt = time.perf_counter() - t0
        macs = 2 * len(hs) * 2048 * 2048 * 128
        out["c5"] = {"cpu_baseline": {
            "value": round(2 * macs / dt / 1e9, 4), "unit": "emulated GOP/s", "cores": cores, "kind": "port",
            "ms_whole_call_estimate": round(dt * 32 / len(hs) * 1e3, 0),
            "sample": f"oracle attend (quantizers, systolic reducer, torch CPU softmax) on heads 0 and 31 of the "
                      f"32 (a 1/16 slice: each head is its own KV head), every key computed as the reference "
                      f"does; {macs / 1e9:.2f} G MAC in {dt:.1f} s wall; the whole call's time is x16"},
            "oracle": o}
    _DATA.clear()
    return out


# -------------------------------------------------------------------------------------------- GPU timing
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


def _warm(fn, calls=10):
    """Untimed calls, so the timed ones start with the clocks up after the host-side work between lines."""
    import torch
    for _ in range(calls):
        fn()
    torch.cuda.synchronize()


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


def _capture(fn, entry):
    """Run fn once; return (its result, the argument tuples of its calls of library entry point `entry`, every
    tensor whose address it passed to the library).  The caller keeps the last alive while it replays."""
    from mxq import _lib
    calls, held, run, ptr = [], [], _lib.run, _lib.ptr

    def record(name, *args):
        if name == entry:
            calls.append(args)
        return run(name, *args)

    def hold(t):
        held.append(t)
        return ptr(t)
    _lib.run, _lib.ptr = record, hold
    try:
        res = fn()
    finally:
        _lib.run, _lib.ptr = run, ptr
    return res, calls, held


def _replay_ms(calls, entry, reps, stream):
    """Kernel time per launch of `entry` by replay: the recorded calls (whose buffers the caller keeps alive)
    issued `reps` times back to back between one pair of HIP events, so the events' own cost, some 15-20 us per
    pair (as much as a short kernel takes), is paid once instead of at every launch."""
    import torch

    from mxq import _lib
    f = getattr(_lib.load(), entry)
    torch.cuda.synchronize()
    for a in calls:                                          # warm
        _lib.check(f(*a), entry)
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record(stream)
    rcs = [f(*calls[k % len(calls)]) for k in range(reps)]
    end.record(stream)
    torch.cuda.synchronize()
    for rc in rcs:
        _lib.check(rc, entry)
    return start.elapsed_time(end) / reps


def _profile_value(name, key):
    """`key: N` from profiles/<name>.txt, else None."""
    path = os.path.join(REPO, "profiles", f"{name}.txt")
    try:
        with open(path) as f:
            for line in f:
                if line.startswith(f"{key}:"):
                    return float(line.split(":", 1)[1].split()[0])
    except (OSError, ValueError):
        pass
    return None


def quantize_lines(torch, steps, inp):
    """block.mxgemmini on bf16 8192 x 8192 (5 formats, rne) and block.ocp quantize + dequantize on 4096 x 512
    fp32 with rotating buffers past the 256 MB last-level cache: GB/s of algorithmic bytes.  Returns the line
    and the outputs the parity check compares."""
    from mxq import block
    dev = torch.device("cuda", 0)
    V = inp["c3"].to(dev)
    s = torch.cuda.current_stream(dev)
    out, kern, outputs = {}, {}, {}
    bytes_c3 = 8192 * 8192 * 2 + 8192 * 8192 * 4 + 256 * 8192 * 4
    for fmt in C3_FORMATS:
        fn = lambda: block.mxgemmini.quantize(V, fmt, axis=0, rounding_mode="rne")   # noqa: E731
        outputs[fmt] = _slice_digests(*(t.cpu().numpy() for t in fn()), 512)
        _warm(fn)
        ms = _events_ms(fn, steps, s)
        out[fmt] = round(bytes_c3 / ms / 1e6, 1)
        res, calls, held = _capture(fn, "mxq_block_quantize")
        kms = _replay_ms(calls, "mxq_block_quantize", steps, s)
        kern[fmt] = round(bytes_c3 / kms / 1e6, 1)
        del res, calls, held
    # the same quantize written as code and E8M0 bytes in one pass (mxq.packed, not in the reference)
    import mxq
    bytes_pk = 8192 * 8192 * 2 + 8192 * 8192 + 256 * 8192
    pk, pk_kern = {}, {}
    for fmt in C3_FORMATS:
        fn = lambda: mxq.packed.quantize(V, fmt, rounding_mode="rne", check=False)            # noqa: E731
        _warm(fn)
        ms = _events_ms(fn, steps, s)
        pk[fmt] = round(bytes_pk / ms / 1e6, 1)
        res, calls, held = _capture(fn, "mxq_block_quantize_packed")
        kms = _replay_ms(calls, "mxq_block_quantize_packed", steps, s)
        pk_kern[fmt] = round(bytes_pk / kms / 1e6, 1)
        del res, calls, held
    del V
    # 17 MB per call: rotate over 64 inputs (1.1 GB with outputs) so HBM, not the cache, serves them; the first
    # is the seeded input the parity check and the CPU baseline use
    g = torch.Generator(device=dev).manual_seed(11)
    rot = [inp["c1"].to(dev)] + [torch.randn(4096, 512, device=dev, generator=g) for _ in range(63)]
    bytes_c1 = 4096 * 512 * 4 * 2 + 128 * 512 * 4
    i = [0]

    def q1():
        r = block.ocp.quantize(rot[i[0] % 64], "MXFP8_E4M3", axis=0)
        i[0] += 1
        return r
    _warm(q1, 64)
    ms1 = _events_ms(q1, 256, s)
    c1_calls, c1_keep = [], []
    for k in range(64):
        res, calls, held = _capture(q1, "mxq_block_quantize")
        c1_keep.append((res, held))
        c1_calls += calls
    kms1 = _replay_ms(c1_calls, "mxq_block_quantize", 256, s)
    del c1_calls, c1_keep
    P, X = block.ocp.quantize(rot[0], "MXFP8_E4M3", axis=0)
    outputs["c1"] = _slice_digests(P.cpu().numpy(), X.cpu().numpy(), 32)
    ms1d = _events_ms(lambda: block.ocp.dequantize(P, X, axis=0), 64, s)
    return {"mxgemmini_bf16_8192x8192_rne_GBs": out, "mxgemmini_bf16_8192x8192_rne_kernel_GBs": kern,
            "mxgemmini_bytes_per_call": bytes_c3,
            "packed_bf16_8192x8192_rne_GBs": pk, "packed_bf16_8192x8192_rne_kernel_GBs": pk_kern,
            "packed_bytes_per_call": bytes_pk,
            "ocp_e4m3_4096x512_quantize_GBs": round(bytes_c1 / ms1 / 1e6, 1),
            "ocp_e4m3_4096x512_quantize_kernel_GBs": round(bytes_c1 / kms1 / 1e6, 1) if kms1 else None,
            "ocp_e4m3_4096x512_dequantize_GBs_cache_resident": round(bytes_c1 / ms1d / 1e6, 1),
            "peak_GBs": HBM_PEAK_GBS}, outputs


def lut_line(torch, steps, inp):
    """block.lut MXFP6_E3M2 (rne, 2^-23, group 1, 50 iterations) on two fp32 4096 x 4096 operands, then the
    systolic MXGEMMINI HW_FINAL product of the two LUT operands (K = M = N = 4096)."""
    from mxq import block, matmul
    dev = torch.device("cuda", 0)
    s = torch.cuda.current_stream(dev)
    A, B = inp["c4a"].to(dev), inp["c4b"].to(dev)
    q = lambda V: block.lut.quantize(V, "MXFP6_E3M2", 0, 32, rounding_mode="rne", scale_floor=2.0 ** -23,  # noqa
                                     group=1, max_iters=50)
    PA, XA = q(A)
    PB, XB = q(B)
    ms_q = _events_ms(lambda: q(A), steps, s)
    # the one-call path's kernels: quantize (fp32 in, code bytes, float32 scales and per-split counts out),
    # k-means, and the pick (code bytes in, float32 entries out)
    kl = {name: _kernel_ms(lambda: q(A), steps, name)[0] for name in ("lut_quant", "lut_kmeans", "lut_pick_codes")}
    elems = 4096 * 4096
    quant_bytes = elems * 4 + elems + elems // 32 * 4                 # V read; codes and scales written
    pick_bytes = elems + elems * 4                                    # codes read, entries written
    mm = lambda: matmul.systolic(PA, XA, PB, XB, matmul.MXGEMMINI(), matmul.HW_FINAL)        # noqa: E731
    Y = mm()
    _warm(mm, 3)
    ms_mm = _events_ms(mm, max(steps, 5), s)
    kms, _ = _kernel_ms(mm, max(steps, 5), "systolic_fast")
    macs = 4096 ** 3
    line = {"workload": "block.lut MXFP6_E3M2 4096x4096 (quantize and count, k-means, pick) + systolic 4096^3",
            "lut_quantize_ms": round(ms_q, 3),
            "lut_kernels_us": {k: round(v * 1e3, 2) if v else None for k, v in kl.items()},
            "lut_quant_kernel_GBs": round(quant_bytes / kl["lut_quant"] / 1e6, 1) if kl["lut_quant"] else None,
            "lut_pick_kernel_GBs": round(pick_bytes / kl["lut_pick_codes"] / 1e6, 1) if kl["lut_pick_codes"] else None,
            "lut_pick_kernel_frac": (round(pick_bytes / kl["lut_pick_codes"] / 1e6 / HBM_PEAK_GBS, 3)
                                     if kl["lut_pick_codes"] else None),
            "systolic_ms": round(ms_mm, 3),
            "systolic_TOPs": round(2 * macs / ms_mm / 1e9, 3),
            "systolic_kernel_TOPs": round(2 * macs / kms / 1e9, 3) if kms else None,
            "systolic_kernel_frac": round(2 * macs / kms / 1e9 / VALU_ROOF_TOPS, 4) if kms else None}
    outputs = {k: t.cpu().numpy() for k, t in (("PA", PA), ("XA", XA), ("PB", PB), ("XB", XB))}
    outputs["Y_cols"] = Y[:, 4064:].cpu().numpy()
    return line, outputs


def causal_computed_fraction(T=2048, tile=64):
    """The share of attend C5's MACs its kernels compute: on the causal mask the batched launches run on
    64 x 64 output tiles (32 problems of 2048 x 2048 scores, 32 x 32 tiles each, at least 8 per CU), Q K^T skips
    the tiles wholly above the diagonal and P V stops each 64-query tile's reduction at its last key: both
    compute n (n + 1) / 2 of n^2 tile-units, n = T / tile."""
    n = T // tile
    return n * (n + 1) / 2 / (n * n)


def attend_line(torch, steps, inp):
    """mxq.nn.attend, Llama-3-8B-shaped: 1 x 32 heads x 2048 x 128, causal HF eager mask, Q K^T and P V through
    the MXGEMMINI MXFP8_E4M3 Scheme, softmax in fp32; and its GQA variant with 8 KV heads."""
    from functools import partial

    import mxq
    from mxq import Scheme, block, matmul
    dev = torch.device("cuda", 0)
    s = torch.cuda.current_stream(dev)
    qz = partial(block.mxgemmini.quantize, fmt="MXFP8_E4M3", axis=0)
    hw = Scheme("hw", a=qz, b=qz, reduce=partial(matmul.systolic, arith=matmul.MXGEMMINI(), schedule=matmul.HW_FINAL))
    q, k, v, mask = (inp[n].to(dev) for n in ("q", "k", "v", "mask"))
    fn = lambda: mxq.nn.attend(q, k, v, mask, 128 ** -0.5, hw, hw)                      # noqa: E731
    o = fn()
    for _ in range(4):                     # past the allocator's growth and the clock ramp of a cold start
        fn()
    ms = _events_ms(fn, steps, s)
    kq, _ = _kernel_ms(fn, steps, "systolic_fast")
    k8, v8 = k[:, :8].contiguous(), v[:, :8].contiguous()
    fn8 = lambda: mxq.nn.attend(q, k8, v8, mask, 128 ** -0.5, hw, hw)                   # noqa: E731
    for _ in range(4):                     # its own buffers' first allocation, as for the call above
        fn8()
    ms8 = _events_ms(fn8, steps, s)
    macs = 2 * 32 * 2048 * 2048 * 128
    done = macs * causal_computed_fraction()
    line = {"workload": "nn.attend 1x32x2048x128 causal, MXGEMMINI MXFP8_E4M3 Scheme for QK^T and PV",
            "ms": round(ms, 3), "emulated_TOPs": round(2 * macs / ms / 1e9, 3),
            "computed_macs": int(done),
            "computed_TOPs": round(2 * done / ms / 1e9, 3),
            "computed_frac_whole_call": round(2 * done / ms / 1e9 / VALU_ROOF_TOPS, 4),
            "systolic_fast_kernels_ms": round(2 * kq, 3) if kq else None,
            "computed_frac_kernels": round(2 * done / (2 * kq) / 1e9 / VALU_ROOF_TOPS, 4) if kq else None,
            "gqa8_ms": round(ms8, 3),
            "note": "emulated_TOPs counts every MAC of the call (the reference computes them all); computed_* count "
                    "the MACs the kernels run after the exact causal skip"}
    return line, o[:, :, list(C5_HEADS)].cpu().numpy()


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


def c2_variants_line(torch, steps, inp):
    """C2's systolic product on its other operands: seed 1, and seed 0 quantized as the tapeout recipe does
    (rne, scale floor 2^-23).  GOP/s per call and the fast kernel's rate against the same roof.  Returns the
    line and each variant's first 32 output columns for the parity check."""
    from mxq import block, matmul
    dev = torch.device("cuda", 0)
    ar = matmul.MXGEMMINI()
    s = torch.cuda.current_stream(dev)
    out, cols = {}, {}
    for name, (xk, wk, kw) in C2_VARIANTS.items():
        P_A, X_A = block.mxgemmini.quantize(inp[xk].t().contiguous().to(dev), "MXFP8_E4M3", axis=0, **kw)
        P_B, X_B = block.mxgemmini.quantize(inp[wk].t().contiguous().to(dev), "MXFP8_E4M3", axis=0, **kw)
        Y = [None]

        def step():
            Y[0] = matmul.systolic(P_A, X_A, P_B, X_B, ar, matmul.HW_FINAL)
        for _ in range(3):
            step()
        ms = _events_ms(step, steps, s)
        kms, _ = _kernel_ms(step, steps, "systolic_fast")
        macs = 512 * 4096 * 4096
        k_tops = 2 * macs / (kms / 1e3) / 1e12 if kms else None
        out[name] = {"quantizer": "block.mxgemmini MXFP8_E4M3" + (f" {kw}" if kw else " (defaults)"),
                     "inputs": "seed 1" if xk == "x1" else "seed 0", "ms": round(ms, 4),
                     "GOPs": round(2 * macs / (ms / 1e3) / 1e9, 2), "kernel_ms": round(kms, 4) if kms else None,
                     "kernel_TOPs": round(k_tops, 3) if k_tops else None,
                     "frac": round(k_tops / VALU_ROOF_TOPS, 4) if k_tops else None}
        cols[name] = Y[0][:, :32].cpu().numpy()
    return out, cols


def mfma_line(torch, steps, P_A, X_A, P_B, X_B, inp):
    """mfma_accum (the matrix-core comparison product) on the benchmark's own codes: pack both operands to FP8
    and E8M0 bytes, then V_MFMA_SCALE_F32_32X32X64_F8F6F4.  The kernel rate is held against MI355X's dense FP8
    peak, 5.0 PFLOP/s.  With the inputs, the same x and W quantized to MXFP6_E2M3 and MXFP4 travel as FP6 and
    FP4 operands, against the 10.1 PFLOP/s dense FP6/FP4 peak."""
    import mxq
    from mxq import block
    dev = P_A.device
    s = torch.cuda.current_stream(dev)
    flops = 2 * P_A.shape[0] * P_A.shape[1] * P_B.shape[1]

    def timed(ops, fmt, peak, packed=None):
        fn = lambda: mxq.mfma_accum(*ops, fmt)                                    # noqa: E731
        _warm(fn)
        ms = _events_ms(fn, steps, s)
        res, calls, held = _capture(fn, "mxq_mx_mfma")           # held: the packed operands
        kms = _replay_ms(calls, "mxq_mx_mfma", steps, s)
        del res, calls, held
        k_tf = flops / (kms / 1e3) / 1e12 if kms else None
        line = {"ms": round(ms, 4), "kernel_ms": round(kms, 4) if kms else None,
                "kernel_TFLOPs": round(k_tf, 2) if k_tf else None, "peak_TFLOPs": peak,
                "frac": round(k_tf / peak, 4) if k_tf else None}
        if packed is not None:                                   # the same operands as mxq.packed bytes
            fb = lambda: mxq.mfma_accum_packed(*packed, fmt, check=False)        # noqa: E731
            _warm(fb)
            line["from_bytes_ms"] = round(_events_ms(fb, steps, s), 4)
        return line
    xt, wt = inp["x"].t().contiguous().to(dev), inp["W"].t().contiguous().to(dev)
    by = lambda fmt: (*mxq.packed.quantize(xt, fmt), *mxq.packed.quantize(wt, fmt))    # noqa: E731
    out = {"workload": "mfma_accum on the same MXFP8_E4M3 codes (M = 512, N = 4096, K = 4096); from_bytes_ms: "
                       "mfma_accum_packed on the same codes and scales as mxq.packed bytes", "kernel": "k_mx_mfma",
           **timed((P_A, X_A, P_B, X_B), "MXFP8_E4M3", FP8_PEAK_TFLOPS, by("MXFP8_E4M3"))}
    for fmt in ("MXFP6_E2M3", "MXFP4"):
        a, b = block.mxgemmini.quantize(xt, fmt, axis=0), block.mxgemmini.quantize(wt, fmt, axis=0)
        out[fmt] = timed((a[0], a[1], b[0], b[1]), fmt, FP6_FP4_PEAK_TFLOPS, by(fmt))
    return out


def valu_rates():
    """gfx950's VALU issue rate per instruction kind (mxq_valu_probe: 8192 workgroups x 256 threads, 64 x 2000
    independent instructions each): lane-operations per second over the chip against the 78.6 T of the vector
    FP32 peak; then, with one wave per SIMD (256 workgroups), the time from one instruction to the next that
    depends on it."""
    import torch

    from mxq import _lib
    wg, iters = 8192, 2000
    out = torch.empty(wg * 256, device="cuda")
    st = torch.cuda.current_stream()
    res = {}
    for kind, name in enumerate(VALU_PROBE_KINDS):
        def f():
            _lib.run("mxq_valu_probe", kind, iters, wg, _lib.ptr(out), _lib.stream(out.device))
        f()
        ms = _events_ms(f, 3, st)
        rate = wg * 256 * 64 * iters / (ms / 1e3)
        res[name] = {"ms": round(ms, 4), "lane_ops_per_s_T": round(rate / 1e12, 1),
                     "frac_of_78.6T": round(rate / VALU_LANE_OPS, 3)}
    chains = {}
    for j, name in enumerate(VALU_CHAIN_KINDS):
        kind = len(VALU_PROBE_KINDS) + j
        def f():
            _lib.run("mxq_valu_probe", kind, iters, 256, _lib.ptr(out), _lib.stream(out.device))
        f()
        ns = _events_ms(f, 3, st) * 1e6 / (64 * iters)
        chains[name] = {"ns_per_dependent_instruction": round(ns, 3), "clocks_at_2.4GHz": round(ns * 2.4, 2)}
    print(json.dumps({"valu_rates": res, "dependent_chains": chains}), flush=True)


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


# -------------------------------------------------------------------------------------------- parity
def _slice_digests(P, X, width):
    """Digests of P's and X's column slices of `width` columns, as the CPU baseline's jobs cut them."""
    return [(c, c + width, _digest(P[:, c:c + width]), _digest(X[:, c:c + width])) for c in range(0, P.shape[1], width)]


def _slices_equal(gpu, oracle):
    """The GPU's P and X against the oracle's, slice by slice, by digest."""
    return len(gpu) == len(oracle) and all(
        (c0, c1, dp, dx) == (j[2], j[3], op, ox) for (c0, c1, dp, dx), (j, op, ox) in zip(gpu, oracle))


def _bits_equal(a, b):
    import numpy as np
    a, b = np.ascontiguousarray(a, np.float32), np.ascontiguousarray(b, np.float32)
    return a.shape == b.shape and bool(np.array_equal(a.view(np.uint32), b.view(np.uint32)))


def _softmax_tolerance(got, want):
    """attend against the oracle run with torch's CPU softmax: the GPU's softmax may differ in the last bits;
    at most 2 % of outputs may differ, none by more than 2^-4 of the largest |output|."""
    import numpy as np
    differ = float((got != want).mean())
    worst = float(np.abs(got - want).max() / max(np.abs(want).max(), 1e-30))
    return {"equal_frac": round(1 - differ, 5), "max_rel_to_largest": worst,
            "within_tolerance": differ <= 0.02 and worst <= 2.0 ** -4}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    # the GPU's clock ramps over its first ~20 launches of the C2 kernel (1.32 ms falling to a steady 1.155 ms in
    # a kernel trace), so the default warm-up covers that before the timed steps
    ap.add_argument("--warmup", type=int, default=25)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baselines and the parity checks")
    ap.add_argument("--no-extra", action="store_true", help="only the systolic line (no quantize, LUT, attend)")
    ap.add_argument("--copy-calibration", action="store_true", help="run only the counter-calibration copy")
    ap.add_argument("--valu-rates", action="store_true", help="run only the VALU issue-rate probe")
    ap.add_argument("--only", choices=("quantize", "lut", "attend", "mfma", "trees", "llm"),
                    help="run one extra line alone (for profiling) and print it; not the benchmark line")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU; --gpus {args.gpus} is not supported (the systolic path "
              "would shard over output columns with one final all-gather)", file=sys.stderr)
        sys.exit(2)
    if args.valu_rates:
        valu_rates()
        return
    if args.copy_calibration:
        copy_calibration()
        return

    import torch

    inp = make_inputs(torch)
    cores = max(1, min(MAX_POOL, len(os.sched_getaffinity(0))))
    # the CPU baselines fork their worker pool, so they run before anything touches the GPU
    cpu = cpu_baselines(inp, cores) if not args.no_cpu and args.only is None else None
    print(f"bench: inputs ready{', CPU baselines done' if cpu else ''}", file=sys.stderr, flush=True)

    import mxq  # noqa: F401
    from mxq import block, matmul
    dev = torch.device("cuda", 0)
    if args.only in ("quantize", "lut", "attend", "llm"):
        fn = {"quantize": lambda: quantize_lines(torch, max(10, args.steps), inp)[0],
              "lut": lambda: lut_line(torch, 3, inp)[0], "attend": lambda: attend_line(torch, 10, inp)[0],
              "llm": lambda: llm_line(torch, 2)}[args.only]
        print(json.dumps({"only": args.only, args.only: fn()}), flush=True)
        return
    M, N, K = 512, 4096, 4096
    P_A, X_A = block.mxgemmini.quantize(inp["x"].t().contiguous().to(dev), "MXFP8_E4M3", axis=0)
    P_B, X_B = block.mxgemmini.quantize(inp["W"].t().contiguous().to(dev), "MXFP8_E4M3", axis=0)
    ar = matmul.MXGEMMINI()
    if args.only in ("mfma", "trees"):
        fn = {"mfma": lambda: mfma_line(torch, max(5, args.steps // 2), P_A, X_A, P_B, X_B, inp),
              "trees": lambda: trees_line(torch, 3, P_A, X_A, P_B, X_B)}[args.only]
        print(json.dumps({"only": args.only, args.only: fn()}), flush=True)
        return
    Y = [None]

    def step():
        Y[0] = matmul.systolic(P_A, X_A, P_B, X_B, ar, matmul.HW_FINAL)
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
    ops_per_mac = _profile_value("systolic_fast_c2_valu", "valu_lane_ops_per_mac")
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
                     "frac_survey_model": round(k_tops / MODEL10_ROOF_TOPS, 4) if k_tops else None,
                     "traffic": _profile_value("systolic_fast_c2_traffic", "bytes_per_launch"),
                     "kernel": "k_systolic_fast64<16, true, true, 2>", "kernel_ms": round(kms, 4) if kms else None,
                     "kernel_launches_timed": launches,
                     "executed": None if not (ops_per_mac and k_tops) else {
                         "valu_lane_ops_per_mac": ops_per_mac,
                         "valu_lane_ops_per_s_T": round(k_tops / 2 * ops_per_mac, 2),
                         "frac": round(k_tops * 1e12 / 2 * ops_per_mac / VALU_LANE_OPS, 4),
                         "source": "SQ_INSTS_VALU x 64 / emulated MACs, profiles/systolic_fast_c2_valu.txt"},
                     "note": "VALU-bound emulation (neither HBM nor MFMA): achieved = 2 x 8,589,934,592 emulated "
                             "MACs / the fast kernel's average duration; peak = MI355X vector FP32 157.3 TFLOP/s = "
                             "78.6 T full-rate lane-slots/s, / 8 slots per emulated MAC (an e4 lane step on gfx950: "
                             "multiply, mask, the add and subtract that round to the lane's step, the exact add and "
                             "a 3-op nearest-even split, one slot each) x 2 ops per MAC; frac_survey_model prices every "
                             "MAC at 10 lane-operations (15.73 TOP/s), a model the kernel's 8-operation step beats; "
                             "`executed.frac` holds the counted instructions (full- and half-rate alike) against "
                             "the 78.6 T lane rate"},
    }
    extra = {}
    if not args.no_extra:
        line["quantize"], extra["quantize"] = quantize_lines(torch, max(10, args.steps), inp)
        line["lut_c4"], extra["lut"] = lut_line(torch, 3, inp)
        line["attend_c5"], extra["attend"] = attend_line(torch, 10, inp)
        line["mfma_c2"] = mfma_line(torch, max(5, args.steps // 2), P_A, X_A, P_B, X_B, inp)
        line["trees_c2"] = trees_line(torch, 3, P_A, X_A, P_B, X_B)
        line["c2_variants"], extra["c2_variants"] = c2_variants_line(torch, 10, inp)
    if cpu is not None:
        line["cpu_baseline"] = cpu["c2"]["cpu_baseline"]
        ncol = cpu["c2"]["cols"]
        line["parity"] = {"checked": f"the timed output's columns 0..{ncol - 1} (all 512 rows) against the oracle",
                          "bit_exact": _bits_equal(Y[0][:, :ncol].cpu().numpy(), cpu["c2"]["oracle"])}
        if "quantize" in extra:
            q = extra["quantize"]
            line["quantize"]["cpu_baseline"] = {"c1_ocp_4096x512": cpu["c1"]["cpu_baseline"],
                                                "c3_mxgemmini_bf16_8192x8192": cpu["c3"]["cpu_baseline"]}
            line["quantize"]["parity"] = {
                "checked": "P and X of C1 and of C3 (every format), whole tensors, against the oracle's",
                "c1_bit_exact": _slices_equal(q["c1"], cpu["c1"]["oracle"]),
                "c3_bit_exact": {f: _slices_equal(q[f], cpu["c3"]["oracle"][f]) for f in C3_FORMATS}}
        if "lut" in extra:
            o, w = extra["lut"], cpu["c4"]["oracle"]
            line["lut_c4"]["cpu_baseline"] = cpu["c4"]["cpu_baseline"]
            line["lut_c4"]["parity"] = {
                "checked": "both LUT operands (P, X) whole, and the product's last 32 columns, against the oracle",
                "lut_operands_bit_exact": all(_bits_equal(o[k], w[k]) for k in ("PA", "XA", "PB", "XB")),
                "systolic_columns_bit_exact": _bits_equal(o["Y_cols"], w["Y_cols"])}
        if "c2_variants" in extra:
            line["c2_variants"]["parity"] = {
                "checked": "each variant's columns 0..31 (all 512 rows) against the oracle on the same operands",
                **{f"{k}_bit_exact": _bits_equal(extra["c2_variants"][k], cpu["c2_variants"][k])
                   for k in C2_VARIANTS}}
        if "attend" in extra:
            line["attend_c5"]["cpu_baseline"] = cpu["c5"]["cpu_baseline"]
            line["attend_c5"]["parity"] = {"checked": "heads 0 and 31 against the oracle with torch's CPU softmax "
                                                      "(bit for bit with the GPU's softmax: tests/test_nn_gpu.py)",
                                           **_softmax_tolerance(extra["attend"], cpu["c5"]["oracle"])}
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
