// Block-quantize kernels for float inputs (one translation unit per input type, compiled in parallel).
#include "quantize_impl.h"

int mxq_quantize_f32(const void* V, float* P, float* X, int64_t outer, int64_t n, int64_t inner, int64_t bs,
                      const mxq_block_spec& q, hipStream_t st) {
  return mxq_quant::dispatch_elem(static_cast<const float*>(V), mxq_quant::FloatSink{P, X}, outer, n, inner, bs, q, st);
}
