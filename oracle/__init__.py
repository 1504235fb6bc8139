"""CPU oracle: an independent numpy restatement of mxq's block quantization, LUT and systolic-emulation path.

TEST INFRASTRUCTURE ONLY.  Nothing in the product (the `mxq` package and its HIP library) imports, calls or
loads anything here.  The only users are tests/, __graft_entry__.smoke() (as the checker of one small GPU
call) and bench.py's cpu_baseline leg (timed as the CPU port of the reference's algorithm).

Every function follows the reference's own step order with numpy float32/float64 operations that have the
same IEEE roundings as the torch CPU kernels the reference runs (file:line citations are relative to the
reference repository).  It deliberately does NOT share code or technique with the HIP kernels: the kernels
work on integer bit patterns and lookup tables, the oracle on float arithmetic in the reference's order.

    numerics   rounding, float_em grids, microxcaling element step, scale factors, arith, Arithmetics
    block      compose / dequantize and the four named quantizers
    lut        formats tables, k-means tables, pick, lookup, finder
    systolic   the PE-column reducer with MXGEMMINI and MXQUANT
    fp64       fp64_accum
    brute      exact-rational scalar models used to pin the above on small inputs

What pins each function (closed forms, brute force, torch library pins, golden fixtures written by the
reference itself) is listed in each module's header and tested in tests/test_oracle_*.py.
"""
