// Block-quantize kernels for f16_t inputs (one translation unit per input type, compiled in parallel).
#include "quantize_impl.h"

int mxq_quantize_f16(const void* V, float* P, float* X, int64_t outer, int64_t n, int64_t inner, int64_t bs,
                      const mxq_block_spec& q, hipStream_t st) {
  return mxq_quant::dispatch_elem(static_cast<const mxq_quant::f16_t*>(V), mxq_quant::FloatSink{P, X}, outer, n, inner, bs, q, st);
}
