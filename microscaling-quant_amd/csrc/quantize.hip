// C entry points of block quantization and dequantization; the kernels live in quantize_impl.h and are
// instantiated per input type in quantize_{f32,bf16,f16}.hip.
#include "quantize_impl.h"

int mxq_quantize_f32(const void*, float*, float*, int64_t, int64_t, int64_t, int64_t, const mxq_block_spec&, hipStream_t);
int mxq_quantize_bf16(const void*, float*, float*, int64_t, int64_t, int64_t, int64_t, const mxq_block_spec&, hipStream_t);
int mxq_quantize_f16(const void*, float*, float*, int64_t, int64_t, int64_t, int64_t, const mxq_block_spec&, hipStream_t);
int mxq_quantize_packed_f32(const void*, uint8_t*, uint8_t*, int32_t*, int, int, int64_t, int64_t, int64_t, int64_t,
                            const mxq_block_spec&, hipStream_t);
int mxq_quantize_packed_bf16(const void*, uint8_t*, uint8_t*, int32_t*, int, int, int64_t, int64_t, int64_t, int64_t,
                             const mxq_block_spec&, hipStream_t);
int mxq_quantize_packed_f16(const void*, uint8_t*, uint8_t*, int32_t*, int, int, int64_t, int64_t, int64_t, int64_t,
                            const mxq_block_spec&, hipStream_t);

extern "C" int mxq_block_quantize(const void* V, int32_t v_dtype, float* P, float* X, int64_t outer, int64_t n,
                                  int64_t inner, int64_t block_size, const mxq_block_spec* spec,
                                  mxq_stream_t stream) {
  if (!spec) return mxq::invalid("mxq_block_quantize: spec is NULL");
  if (outer < 0 || n < 0 || inner < 0 || block_size < 1) return mxq::invalid("mxq_block_quantize: bad shape");
  if (int rc = mxq_quant::validate(*spec)) return rc;
  if (outer == 0 || n == 0 || inner == 0) return MXQ_OK;
  if (!V || !P || !X) return mxq::invalid("mxq_block_quantize: NULL pointer");
  const mxq_block_spec q = *spec;
  hipStream_t st = mxq::as_stream(stream);
  switch (v_dtype) {
    case MXQ_DT_F32: return mxq_quantize_f32(V, P, X, outer, n, inner, block_size, q, st);
    case MXQ_DT_BF16: return mxq_quantize_bf16(V, P, X, outer, n, inner, block_size, q, st);
    case MXQ_DT_F16: return mxq_quantize_f16(V, P, X, outer, n, inner, block_size, q, st);
    default: return mxq::invalid("mxq_block_quantize: unsupported input dtype");
  }
}

// The transposed layout goes through the same per-type dispatch, flagged by a negative block size.
extern "C" int mxq_block_quantize_t(const void* M, int32_t v_dtype, float* P, float* X, int64_t n, int64_t inner,
                                    int64_t block_size, const mxq_block_spec* spec, mxq_stream_t stream) {
  if (!spec) return mxq::invalid("mxq_block_quantize_t: spec is NULL");
  if (n < 0 || inner < 0) return mxq::invalid("mxq_block_quantize_t: bad shape");
  if (block_size != 32) return mxq::invalid("mxq_block_quantize_t: block_size must be 32");
  if (int rc = mxq_quant::validate(*spec)) return rc;
  if (n == 0 || inner == 0) return MXQ_OK;
  if (!M || !P || !X) return mxq::invalid("mxq_block_quantize_t: NULL pointer");
  const mxq_block_spec q = *spec;
  hipStream_t st = mxq::as_stream(stream);
  switch (v_dtype) {
    case MXQ_DT_F32: return mxq_quantize_f32(M, P, X, 1, n, inner, -32, q, st);
    case MXQ_DT_BF16: return mxq_quantize_bf16(M, P, X, 1, n, inner, -32, q, st);
    case MXQ_DT_F16: return mxq_quantize_f16(M, P, X, 1, n, inner, -32, q, st);
    default: return mxq::invalid("mxq_block_quantize_t: unsupported input dtype");
  }
}

extern "C" int mxq_block_dequantize(const float* P, const float* X, float* out, int64_t outer, int64_t n,
                                    int64_t inner, int64_t block_size, mxq_stream_t stream) {
  if (outer < 0 || n < 0 || inner < 0 || block_size < 1) return mxq::invalid("mxq_block_dequantize: bad shape");
  if (outer == 0 || n == 0 || inner == 0) return MXQ_OK;
  if (!P || !X || !out) return mxq::invalid("mxq_block_dequantize: NULL pointer");
  const int64_t nb = mxq::ceil_div(n, block_size);
  const uintptr_t ap = reinterpret_cast<uintptr_t>(P), ax = reinterpret_cast<uintptr_t>(X),
                  ao = reinterpret_cast<uintptr_t>(out);
  auto aligned = [&](int vec) { return inner % vec == 0 && (ap | ax | ao) % (vec * 4) == 0; };
  const int vec = aligned(4) ? 4 : (aligned(2) ? 2 : 1);
  const int64_t count = outer * n * (inner / vec), xcount = outer * nb * inner;
  hipStream_t st = mxq::as_stream(stream);
  auto go = [&](auto vec_const, auto idx) {
    constexpr int VEC = decltype(vec_const)::value;
    using I = decltype(idx);
    mxq_quant::k_dequant_flat<VEC, I><<<mxq::grid_for(count, 256), 256, 0, st>>>(
        P, X, out, (I)count, (I)(inner / VEC), (I)n, (I)block_size, (I)nb);
  };
  const bool narrow = count * vec < ((int64_t)1 << 31) && xcount < ((int64_t)1 << 31);   // no wrap near the end
  if (vec == 4) narrow ? go(std::integral_constant<int, 4>{}, uint32_t{}) : go(std::integral_constant<int, 4>{}, int64_t{});
  else if (vec == 2) narrow ? go(std::integral_constant<int, 2>{}, uint32_t{}) : go(std::integral_constant<int, 2>{}, int64_t{});
  else narrow ? go(std::integral_constant<int, 1>{}, uint32_t{}) : go(std::integral_constant<int, 1>{}, int64_t{});
  return mxq::check_launch("mxq_block_dequantize");
}

// The element format of the code bytes a spec's element rule produces: float_em's widths for the qtorch and ocp
// grids, the microxcaling step's mbits less its sign and implicit bits; false unless it is an OCP MX format.
static bool code_format(const mxq_block_spec& q, int* ce, int* cm) {
  *ce = q.e;
  *cm = q.elem == MXQ_ELEM_MICROSOFT ? q.m - 2 : q.m;
  const int e = *ce, m = *cm;
  return (e == 4 && m == 3) || (e == 5 && m == 2) || (e == 3 && m == 2) || (e == 2 && m == 3) || (e == 2 && m == 1);
}

extern "C" int mxq_block_quantize_packed(const void* V, int32_t v_dtype, uint8_t* codes, uint8_t* scales,
                                         int32_t* err, int64_t outer, int64_t n, int64_t inner, int64_t block_size,
                                         const mxq_block_spec* spec, mxq_stream_t stream) {
  if (!spec) return mxq::invalid("mxq_block_quantize_packed: spec is NULL");
  if (outer < 0 || n < 0 || inner < 0 || block_size < 1) return mxq::invalid("mxq_block_quantize_packed: bad shape");
  if (int rc = mxq_quant::validate(*spec)) return rc;
  int ce, cm;
  if (spec->elem != MXQ_ELEM_QTORCH && spec->elem != MXQ_ELEM_OCP && spec->elem != MXQ_ELEM_MICROSOFT)
    return mxq::invalid("mxq_block_quantize_packed: the element rule has no byte format");
  if (!code_format(*spec, &ce, &cm)) return mxq::invalid("mxq_block_quantize_packed: not an OCP MX element format");
  if (outer == 0 || n == 0 || inner == 0) return MXQ_OK;
  if (!V || !codes || !scales || !err) return mxq::invalid("mxq_block_quantize_packed: NULL pointer");
  const mxq_block_spec q = *spec;
  hipStream_t st = mxq::as_stream(stream);
  switch (v_dtype) {
    case MXQ_DT_F32: return mxq_quantize_packed_f32(V, codes, scales, err, ce, cm, outer, n, inner, block_size, q, st);
    case MXQ_DT_BF16: return mxq_quantize_packed_bf16(V, codes, scales, err, ce, cm, outer, n, inner, block_size, q, st);
    case MXQ_DT_F16: return mxq_quantize_packed_f16(V, codes, scales, err, ce, cm, outer, n, inner, block_size, q, st);
    default: return mxq::invalid("mxq_block_quantize_packed: unsupported input dtype");
  }
}
