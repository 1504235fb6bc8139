// The fused LUT-operand quantize kernels for one input type (the types compile in parallel).
#include "lut_operand_impl.h"

int mxq_lut_quant_bf16(const void* V, const mxq_lut::LutQuantArgs& a, const mxq_block_spec& s, int cw,
                       int64_t ntiles, int64_t nsplit, hipStream_t st) {
  return mxq_lut::launch_lut_quant(static_cast<const mxq_quant::bf16_t*>(V), a, s, cw, ntiles, nsplit, st);
}
