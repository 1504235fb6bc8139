// Packed wire formats of block-quantized tensors: one element-code byte per element (OCP MX layout, see
// mx_encode) and one E8M0 byte per block scale, a quarter of the float32 codes' bytes.  The layout is the
// float32 one's: (outer, n, inner) with blocks of block_size along n, codes shaped like P, scales like X.
//
//   k_pack             float32 P and X -> bytes; one thread per block column (it needs the whole block to
//                      know whether a scale E8M0 lacks belongs to an all-zero block)
//   k_unpack_codes     bytes -> float32 P, and k_unpack_scales -> float32 X
//   k_dequant_packed   bytes -> the dequantized float32 values P * X, without materialising either
#include "mxq_common.h"
#include "mxq_numerics.h"

namespace {

bool code_format_ok(int e, int m) {
  return (e == 4 && m == 3) || (e == 5 && m == 2) || (e == 3 && m == 2) || (e == 2 && m == 3) || (e == 2 && m == 1);
}

// (o, b, c) of a flat index over outer * nb * inner (32-bit arithmetic while everything fits).
__device__ __forceinline__ void block_col(int64_t t, int64_t inner, int64_t nb, int64_t& o, int64_t& b, int64_t& c) {
  if (t < 0x7FFFFFFF && inner < 0x7FFFFFFF && nb < 0x7FFFFFFF) {
    const uint32_t tt = (uint32_t)t, ii = (uint32_t)inner, nn = (uint32_t)nb;
    const uint32_t ob = tt / ii;
    c = tt - ob * ii;
    o = ob / nn;
    b = ob - (uint32_t)o * nn;
  } else {
    const int64_t ob = t / inner;
    c = t - ob * inner;
    o = ob / nb;
    b = ob - o * nb;
  }
}

__global__ void __launch_bounds__(256) k_pack(const float* __restrict__ P, const float* __restrict__ X,
                                              uint8_t* __restrict__ codes, uint8_t* __restrict__ scales,
                                              int32_t* __restrict__ err, int64_t outer, int64_t n, int64_t inner,
                                              int64_t bs, int64_t nb, int e, int m) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= outer * nb * inner) return;
  int64_t o, b, c;
  block_col(t, inner, nb, o, b, c);
  const int64_t k0 = b * bs, rows = (n - k0 < bs) ? n - k0 : bs;
  const int64_t off = (o * n + k0) * inner + c;
  bool ok = true, zero = true;
  for (int64_t r = 0; r < rows; ++r) {
    const float q = P[off + r * inner];
    zero = zero && (f2u(q) & 0x7FFFFFFFu) == 0u;
    codes[off + r * inner] = (uint8_t)mx_encode(q, e, m, &ok);
  }
  if (!ok) atomicOr(err, 1);
  bool sok = true;
  scales[t] = (uint8_t)e8m0_encode(X[t], zero, &sok);
  if (!sok) atomicOr(err, 2);
}

__global__ void __launch_bounds__(256) k_unpack_codes(const uint8_t* __restrict__ codes, float* __restrict__ P,
                                                      int64_t count, int e, int m) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < count; i += (int64_t)gridDim.x * blockDim.x)
    P[i] = mx_decode(codes[i], e, m);
}

__global__ void __launch_bounds__(256) k_unpack_scales(const uint8_t* __restrict__ scales, float* __restrict__ X,
                                                       int64_t count) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < count; i += (int64_t)gridDim.x * blockDim.x)
    X[i] = e8m0_decode(scales[i]);
}

// One thread per block column: decode, scale, store (the float32 multiply mxq/block/_driver.py:66-72 makes of
// the float32 codes and scales).
__global__ void __launch_bounds__(256) k_dequant_packed(const uint8_t* __restrict__ codes,
                                                        const uint8_t* __restrict__ scales, float* __restrict__ out,
                                                        int64_t outer, int64_t n, int64_t inner, int64_t bs,
                                                        int64_t nb, int e, int m) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= outer * nb * inner) return;
  int64_t o, b, c;
  block_col(t, inner, nb, o, b, c);
  const int64_t k0 = b * bs, rows = (n - k0 < bs) ? n - k0 : bs;
  const int64_t off = (o * n + k0) * inner + c;
  const float x = e8m0_decode(scales[t]);
  for (int64_t r = 0; r < rows; ++r) out[off + r * inner] = mx_decode(codes[off + r * inner], e, m) * x;
}

int check_shape(int64_t outer, int64_t n, int64_t inner, int64_t bs, int e, int m, const char* who) {
  if (outer < 0 || n < 0 || inner < 0 || bs < 1) return mxq::invalid(std::string(who) + ": bad shape");
  if (!code_format_ok(e, m)) return mxq::invalid(std::string(who) + ": not an OCP MX element format");
  return MXQ_OK;
}

dim3 grid_cap(int64_t threads) {
  const int64_t blocks = mxq::ceil_div(threads, 256);
  return dim3((unsigned)(blocks < (1 << 20) ? blocks : (1 << 20)));
}

}  // namespace

extern "C" int mxq_pack(const float* P, const float* X, uint8_t* codes, uint8_t* scales, int32_t* err, int64_t outer,
                        int64_t n, int64_t inner, int64_t block_size, int32_t e, int32_t m, mxq_stream_t stream) {
  if (int rc = check_shape(outer, n, inner, block_size, e, m, "mxq_pack")) return rc;
  if (outer == 0 || n == 0 || inner == 0) return MXQ_OK;
  if (!P || !X || !codes || !scales || !err) return mxq::invalid("mxq_pack: NULL pointer");
  const int64_t nb = mxq::ceil_div(n, block_size), threads = outer * nb * inner;
  k_pack<<<mxq::grid_for(threads, 256), 256, 0, mxq::as_stream(stream)>>>(P, X, codes, scales, err, outer, n, inner,
                                                                           block_size, nb, e, m);
  return mxq::check_launch("mxq_pack");
}

extern "C" int mxq_unpack(const uint8_t* codes, const uint8_t* scales, float* P, float* X, int64_t outer, int64_t n,
                          int64_t inner, int64_t block_size, int32_t e, int32_t m, mxq_stream_t stream) {
  if (int rc = check_shape(outer, n, inner, block_size, e, m, "mxq_unpack")) return rc;
  if (outer == 0 || n == 0 || inner == 0) return MXQ_OK;
  if ((P && !codes) || (X && !scales)) return mxq::invalid("mxq_unpack: NULL pointer");
  hipStream_t st = mxq::as_stream(stream);
  const int64_t count = outer * n * inner, scount = outer * mxq::ceil_div(n, block_size) * inner;
  if (P) k_unpack_codes<<<grid_cap(count), 256, 0, st>>>(codes, P, count, e, m);
  if (X) k_unpack_scales<<<grid_cap(scount), 256, 0, st>>>(scales, X, scount);
  return mxq::check_launch("mxq_unpack");
}

extern "C" int mxq_dequantize_packed(const uint8_t* codes, const uint8_t* scales, float* out, int64_t outer,
                                     int64_t n, int64_t inner, int64_t block_size, int32_t e, int32_t m,
                                     mxq_stream_t stream) {
  if (int rc = check_shape(outer, n, inner, block_size, e, m, "mxq_dequantize_packed")) return rc;
  if (outer == 0 || n == 0 || inner == 0) return MXQ_OK;
  if (!codes || !scales || !out) return mxq::invalid("mxq_dequantize_packed: NULL pointer");
  const int64_t nb = mxq::ceil_div(n, block_size), threads = outer * nb * inner;
  k_dequant_packed<<<mxq::grid_for(threads, 256), 256, 0, mxq::as_stream(stream)>>>(codes, scales, out, outer, n, inner,
                                                                                     block_size, nb, e, m);
  return mxq::check_launch("mxq_dequantize_packed");
}
