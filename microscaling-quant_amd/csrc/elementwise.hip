// Elementwise entry points: the datapath primitives (rounding, float_em grids, the microxcaling element step,
// scale factors, arith) as standalone kernels over flat arrays.  The block quantizer and the systolic kernels
// inline the same device functions (mxq_numerics.h); these entry points serve the public per-tensor API.
// Grid-stride loops, 256 threads per block, one element per thread per iteration.
#include "mxq_common.h"
#include "mxq_numerics.h"

namespace {

constexpr int kThreads = 256;

inline dim3 ew_grid(int64_t n) {
  int64_t blocks = mxq::ceil_div(n, kThreads);
  if (blocks > 65536) blocks = 65536;
  return dim3((unsigned)(blocks < 1 ? 1 : blocks));
}

#define MXQ_EW_LOOP(n) for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < (n); i += (int64_t)gridDim.x * blockDim.x)

__global__ void k_round_bits(const int64_t* bits, const int64_t* keep, int keep_scalar, int64_t* out, int64_t n,
                             int mode) {
  MXQ_EW_LOOP(n) {
    const int kp = keep ? (int)keep[i] : keep_scalar;
    out[i] = (int64_t)round_bits32((uint32_t)bits[i], kp, mode);
  }
}

template <typename T>
__global__ void k_round_int(const T* k, T* out, int64_t n, int mode) {
  MXQ_EW_LOOP(n) {
    const T x = k[i];
    T r;
    if (mode == MXQ_RNE) {
      r = rint(x);
    } else if (mode == MXQ_TIES_AWAY) {
      const T s = (x > T(0)) ? T(1) : ((x < T(0)) ? T(-1) : T(0));
      r = s * floor(fabs(x) + T(0.5));
    } else {
      r = trunc(x);
    }
    out[i] = r;
  }
}

__global__ void k_bf16(const float* x, float* out, int64_t n) {
  MXQ_EW_LOOP(n) out[i] = bf16_rne(x[i]);
}

__global__ void k_float_em32(const float* z, float* out, int64_t n, int e, int m, int mode, int grid, float max_norm) {
  MXQ_EW_LOOP(n) out[i] = float_em_quantize32(z[i], e, m, mode, grid, max_norm);
}
__global__ void k_float_em64(const double* z, float* out, int64_t n, int e, int m, int mode, int grid, float max_norm) {
  MXQ_EW_LOOP(n) out[i] = float_em_quantize64(z[i], e, m, mode, grid, max_norm);
}

__global__ void k_microsoft(const float* z, float* out, int64_t n, int ebits, int mbits, float max_norm, int mode,
                            int saturate) {
  MXQ_EW_LOOP(n) out[i] = microsoft_quantize(z[i], ebits, mbits, max_norm, mode, saturate != 0);
}

__global__ void k_scale(const float* amax, float* out, int64_t n, mxq_block_spec s) {
  MXQ_EW_LOOP(n) {
    const float a = amax[i];
    float x;
    if (s.scale_rule == MXQ_SCALE_MXQUANT) x = scale_mxquant(a, s.scale_floor);
    else if (s.scale_rule == MXQ_SCALE_OCP) x = scale_ocp(a, s.scale_emax, s.scale_bits);
    else x = scale_ocp_no_clip(a, s.scale_emax, s.scale_bits, s.e, s.m, s.max_norm, s.rounding);
    out[i] = x;
  }
}

__global__ void k_exact_add(const float* a, const float* b, float* out, int64_t n, int e, int m, int mode, int grid,
                            float max_norm) {
  MXQ_EW_LOOP(n) out[i] = exact_add(a[i], b[i], e, m, mode, grid, max_norm);
}

__global__ void k_truncate(const float* x, float* out, int64_t n, int m) {
  MXQ_EW_LOOP(n) out[i] = truncate_significand(x[i], m);
}
__global__ void k_flush(const float* x, float* out, int64_t n, float thr) {
  MXQ_EW_LOOP(n) out[i] = flush_product(x[i], thr);
}
__global__ void k_saturate(const float* x, float* out, int64_t n, float limit, float value) {
  MXQ_EW_LOOP(n) out[i] = saturate(x[i], limit, value);
}

bool widths_ok(int e, int m) { return (e == 8 && m == 23) || (e >= 1 && e <= 8 && m >= 1 && m <= 22); }

}  // namespace

#define MXQ_EW_PRE(name)                                             \
  if (n < 0) return mxq::invalid(name ": negative length");         \
  if (n == 0) return MXQ_OK;                                         \
  hipStream_t st = mxq::as_stream(stream)

extern "C" int mxq_round_bits(const int64_t* bits, const int64_t* keep, int32_t keep_scalar, int64_t* out, int64_t n,
                              int32_t mode, mxq_stream_t stream) {
  MXQ_EW_PRE("mxq_round_bits");
  if (mode < 0 || mode > 2) return mxq::invalid("mxq_round_bits: bad mode");
  if (!keep && (keep_scalar < 0 || keep_scalar > 22)) return mxq::invalid("keep must be in [0, 22]");
  k_round_bits<<<ew_grid(n), kThreads, 0, st>>>(bits, keep, keep_scalar, out, n, mode);
  return mxq::check_launch("mxq_round_bits");
}

extern "C" int mxq_round_int(const void* k, int32_t dtype, void* out, int64_t n, int32_t mode, mxq_stream_t stream) {
  MXQ_EW_PRE("mxq_round_int");
  if (mode < 0 || mode > 2) return mxq::invalid("mxq_round_int: bad mode");
  if (dtype == 0)
    k_round_int<float><<<ew_grid(n), kThreads, 0, st>>>((const float*)k, (float*)out, n, mode);
  else if (dtype == 3)
    k_round_int<double><<<ew_grid(n), kThreads, 0, st>>>((const double*)k, (double*)out, n, mode);
  else
    return mxq::invalid("mxq_round_int: dtype must be float32 (0) or float64 (3)");
  return mxq::check_launch("mxq_round_int");
}

extern "C" int mxq_bf16(const float* x, float* out, int64_t n, mxq_stream_t stream) {
  MXQ_EW_PRE("mxq_bf16");
  k_bf16<<<ew_grid(n), kThreads, 0, st>>>(x, out, n);
  return mxq::check_launch("mxq_bf16");
}

extern "C" int mxq_float_em(const void* z, int32_t dtype, float* out, int64_t n, int32_t e, int32_t m, int32_t mode,
                            int32_t grid, float max_norm, mxq_stream_t stream) {
  MXQ_EW_PRE("mxq_float_em");
  if (!widths_ok(e, m)) return mxq::invalid("unsupported widths e=" + std::to_string(e) + ", m=" + std::to_string(m));
  if (mode < 0 || mode > 2 || grid < 0 || grid > 2) return mxq::invalid("mxq_float_em: bad mode or grid");
  if (dtype == 0)
    k_float_em32<<<ew_grid(n), kThreads, 0, st>>>((const float*)z, out, n, e, m, mode, grid, max_norm);
  else if (dtype == 3)
    k_float_em64<<<ew_grid(n), kThreads, 0, st>>>((const double*)z, out, n, e, m, mode, grid, max_norm);
  else
    return mxq::invalid("mxq_float_em: dtype must be float32 (0) or float64 (3)");
  return mxq::check_launch("mxq_float_em");
}

extern "C" int mxq_microsoft(const float* z, float* out, int64_t n, int32_t ebits, int32_t mbits, float max_norm,
                             int32_t mode, int32_t saturate, mxq_stream_t stream) {
  MXQ_EW_PRE("mxq_microsoft");
  if (ebits < 2 || ebits > 8 || mbits < 2 || mbits > 24 || mode < 0 || mode > 2)
    return mxq::invalid("mxq_microsoft: bad format or mode");
  k_microsoft<<<ew_grid(n), kThreads, 0, st>>>(z, out, n, ebits, mbits, max_norm, mode, saturate);
  return mxq::check_launch("mxq_microsoft");
}

extern "C" int mxq_scale_factor(const float* amax, float* out, int64_t n, const mxq_block_spec* spec,
                                mxq_stream_t stream) {
  MXQ_EW_PRE("mxq_scale_factor");
  if (!spec || spec->scale_rule < MXQ_SCALE_MXQUANT || spec->scale_rule > MXQ_SCALE_OCP_NO_CLIP)
    return mxq::invalid("mxq_scale_factor: bad scale rule");
  k_scale<<<ew_grid(n), kThreads, 0, st>>>(amax, out, n, *spec);
  return mxq::check_launch("mxq_scale_factor");
}

extern "C" int mxq_exact_add(const float* a, const float* b, float* out, int64_t n, int32_t e, int32_t m,
                             int32_t mode, int32_t grid, float max_norm, mxq_stream_t stream) {
  MXQ_EW_PRE("mxq_exact_add");
  if (!widths_ok(e, m)) return mxq::invalid("unsupported widths e=" + std::to_string(e) + ", m=" + std::to_string(m));
  if (mode < 0 || mode > 2 || grid < 0 || grid > 2) return mxq::invalid("mxq_exact_add: bad mode or grid");
  k_exact_add<<<ew_grid(n), kThreads, 0, st>>>(a, b, out, n, e, m, mode, grid, max_norm);
  return mxq::check_launch("mxq_exact_add");
}

extern "C" int mxq_truncate_significand(const float* x, float* out, int64_t n, int32_t m, mxq_stream_t stream) {
  MXQ_EW_PRE("mxq_truncate_significand");
  if (m < 0) return mxq::invalid("mxq_truncate_significand: m must be >= 0");
  k_truncate<<<ew_grid(n), kThreads, 0, st>>>(x, out, n, m);
  return mxq::check_launch("mxq_truncate_significand");
}

extern "C" int mxq_flush_product(const float* x, float* out, int64_t n, float threshold, mxq_stream_t stream) {
  MXQ_EW_PRE("mxq_flush_product");
  k_flush<<<ew_grid(n), kThreads, 0, st>>>(x, out, n, threshold);
  return mxq::check_launch("mxq_flush_product");
}

extern "C" int mxq_saturate(const float* x, float* out, int64_t n, float limit, float value, mxq_stream_t stream) {
  MXQ_EW_PRE("mxq_saturate");
  k_saturate<<<ew_grid(n), kThreads, 0, st>>>(x, out, n, limit, value);
  return mxq::check_launch("mxq_saturate");
}
