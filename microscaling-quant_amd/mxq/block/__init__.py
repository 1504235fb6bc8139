"""mxq.block -- block quantization: step 1 (scale_factor) and step 2 (element_quant) composed, fused on gfx950.

    P, X = block.compose(V, scale=f, elem=g, axis=0, block_size=BLOCK)   any pair: X = f(amax), P = g(block / X)
    P, X = block.<name>.quantize(V, fmt, axis=0, block_size=BLOCK)        P: V's shape; X: ceil(len/BLOCK) along axis
    V_hat = block.<name>.dequantize(P, X, axis=0)                          = P * expand(X)

    mxquant      scale_factor.mxquant + float_em grid=qtorch      MXQuant's simulation codes
    mxgemmini    scale_factor.mxquant + float_em grid=ocp         MX-Gemmini's operand codes
    ocp          scale_factor.ocp     + microxcaling element step OCP MX v1.0
    lut          mxgemmini + mxq.lut tables                       MX-Gemmini's LUT operand
"""
from ._driver import BLOCK, compose, dequantize
from . import mxquant, mxgemmini, ocp, lut

__all__ = ["BLOCK", "compose", "dequantize", "mxquant", "mxgemmini", "ocp", "lut"]
