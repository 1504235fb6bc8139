"""mxq.element_quant -- step 2 of block quantization: snap scaled values onto a format's codes.

    formats     the format table (name -> e, m, emax, max_norm)
    float_em    float(e, m) on the qtorch, ieee or ocp grid
    microsoft   microxcaling's _quantize_elemwise, the OCP reference's element step

float_em is also the quantizer of products and accumulators, which are float(e, m) too.
"""
from . import formats, float_em, microsoft

__all__ = ["formats", "float_em", "microsoft"]
