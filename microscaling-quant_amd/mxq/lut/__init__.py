"""mxq.lut -- MX-Gemmini's look-up tables (mxq/lut/__init__.py:1-24), on the GPU.

A LUT format sends each element as a 4-bit index into a 16-entry table of element values, one table per 2^G
columns of a K x n operand (rows of A, columns of B), each spanning all of K.  The operand is MX block
quantized first (block.mxgemmini); the table is a second, coarser step.

    T = tables(P, fmt, group=G, max_iters=50)     P: K x n block codes; T: ceil(n / 2^G) x 16, rows ascending
    I = pick(P, T, group=G)                        nearest entry, ties to the lower index
    I = finder(codes, T, fmt, group=G)             the chip's finder, from element codes
    P_lut = lookup(I, T, group=G)
    P, X = block.lut.quantize(V, fmt, axis=0, ...) all of the above behind the block quantizer contract
"""
from .formats import FORMATS, SIZE, decode, encode, finder, values
from .kmeans import lookup, pick, tables

__all__ = ["FORMATS", "SIZE", "decode", "encode", "finder", "values", "tables", "pick", "lookup"]
