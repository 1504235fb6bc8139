// Block quantization to element-code and E8M0 scale bytes for f16_t inputs (one translation unit per input type).
#include "quantize_impl.h"

// ce, cm: the element format of the code bytes.
int mxq_quantize_packed_f16(const void* V, uint8_t* P, uint8_t* X, int32_t* err, int ce, int cm, int64_t outer,
                             int64_t n, int64_t inner, int64_t bs, const mxq_block_spec& q, hipStream_t st) {
  const mxq_quant::CodeConsts k = mxq_quant::code_consts(ce, cm);
  const mxq_quant::ByteSink out{P, X, err, ce, cm, k, (k.maxbits >> k.nshift) - k.nsub};
  return mxq_quant::dispatch_elem(static_cast<const mxq_quant::f16_t*>(V), out, outer, n, inner, bs, q,
                                  st);
}
