"""mxq -- microscaling (MX) quantization and bit-exact MX matmul emulation, with gfx950 kernels.

The API is mxq's own (chloe-wong/microscaling-quant, mxq/__init__.py:1-36); every computation runs as a
hand-written HIP kernel of libmxq_hip.so on an AMD Instinct MI355X.

    scale_factor      step 1: mxquant(amax) | ocp(amax, emax) | ocp_below_top | ocp_no_clip
    element_quant     step 2: float_em (grids qtorch | ieee | ocp), microsoft (microxcaling's element step)
    block             steps 1 + 2 fused: compose(V, scale=, elem=, axis); mxquant, mxgemmini, ocp, lut
    lut               MX-Gemmini's look-up tables: tables, pick, lookup, finder, decode, encode, values
    rounding          ties_away | rne | truncate on float32 bit patterns or integers; bf16
    arith             exact_add, truncate_significand, flush_product, saturate
    matmul            systolic: Y = A^T B from codes and scales in the hardware's summation order, with the
                      MXGEMMINI or MXQUANT Arithmetic and a per-lane accumulator schedule
    fp64_accum        the same codes with no rounding inside the multiply: the error floor
    mfma_accum        the same comparison on the gfx950 matrix cores, within mfma_tolerance(K) * sum |a b|;
                      mfma_accum_packed takes the codes and scales as mxq.packed bytes
    schedule          one float(e, m) per accumulator position: load(csv), fixed(e, m), HW_FINAL
    scheme            Scheme(name, a, b, reduce): one explicit chain for one matmul
    nn                MXLinear, patch, attend: Schemes inside a model
"""
__version__ = "0.1.0"

import torch  # noqa: F401  (first: libmxq_hip.so binds to the HIP runtime torch loads)

from . import rounding, arith, schedule, scale_factor, element_quant, lut, block, matmul, scheme, nn, packed
from .block import BLOCK
from ._fp64_accum import fp64_accum
from ._mfma_accum import mfma_accum, mfma_accum_packed, mfma_tolerance
from .element_quant.formats import Format
from .scheme import Scheme

__all__ = ["rounding", "arith", "schedule", "scale_factor", "element_quant", "lut", "block", "matmul", "scheme", "nn",
           "packed", "BLOCK", "Format", "Scheme", "fp64_accum", "mfma_accum", "mfma_accum_packed", "mfma_tolerance"]
