// Fused MX block quantization and dequantization for gfx950.
//
// A tensor is viewed as (outer, n, inner) with the block axis n in the middle.  Two layouts:
//   strided  (inner > 1, or any block size): one thread owns VEC adjacent columns of one block and walks the
//            block's rows; adjacent threads own adjacent columns, so every row access of a wavefront is one
//            contiguous run (64 * VEC elements).  The block stays in registers between the amax and the
//            element step when the block size is the compile-time 32; other sizes read the block twice.
//   contig32 (inner == 1, block 32, n % 32 == 0): eight lanes own one contiguous 128-byte block, four
//            elements each, and combine their amax with three cross-lane exchanges.
// Step 1 (the scale) runs once per block and column; step 2 (the element grid) once per element.  The
// division by the scale is a multiply by its reciprocal when the scale is a normal power of two (then both
// are the same correctly rounded value) and an IEEE division otherwise (the 1e-38 floor is not a power of two).
#include "mxq_common.h"
#include "mxq_numerics.h"

namespace {


struct bf16_t { uint16_t v; };
struct f16_t { uint16_t v; };

__device__ __forceinline__ float to_f32(float x) { return x; }
__device__ __forceinline__ float to_f32(bf16_t x) { return u2f((uint32_t)x.v << 16); }
__device__ __forceinline__ float to_f32(f16_t x) { return (float)__builtin_bit_cast(_Float16, x.v); }

template <typename T, int VEC>
struct alignas(sizeof(T) * VEC) VecT { T v[VEC]; };

template <typename T, int VEC>
__device__ __forceinline__ void load_vec(const T* p, float (&out)[VEC]) {
  const VecT<T, VEC> r = *reinterpret_cast<const VecT<T, VEC>*>(p);
#pragma unroll
  for (int j = 0; j < VEC; ++j) out[j] = to_f32(r.v[j]);
}

template <int VEC>
__device__ __forceinline__ void store_vec(float* p, const float (&in)[VEC]) {
  VecT<float, VEC> r;
#pragma unroll
  for (int j = 0; j < VEC; ++j) r.v[j] = in[j];
  *reinterpret_cast<VecT<float, VEC>*>(p) = r;
}

// (o, b, column group) of a flat thread index over outer * nb * groups.
__device__ __forceinline__ void split_index(int64_t t, int64_t groups, int64_t nb, int64_t& o, int64_t& b,
                                            int64_t& g) {
  if (t < 0x7FFFFFFF && groups < 0x7FFFFFFF && nb < 0x7FFFFFFF) {
    const uint32_t tt = (uint32_t)t, gg = (uint32_t)groups, nn = (uint32_t)nb;
    const uint32_t ob = tt / gg;
    g = tt - ob * gg;
    o = ob / nn;
    b = ob - (uint32_t)o * nn;
  } else {
    const int64_t ob = t / groups;
    g = t - ob * groups;
    o = ob / nb;
    b = ob - o * nb;
  }
}

template <typename T, int ELEM, int VEC, int BS>
__global__ void __launch_bounds__(256) k_quant_strided(const T* __restrict__ V, float* __restrict__ P,
                                                       float* __restrict__ X, int64_t outer, int64_t n,
                                                       int64_t inner, int64_t bs_rt, int64_t nb, mxq_block_spec s) {
  const int64_t groups = inner / VEC;
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= outer * nb * groups) return;
  int64_t o, b, g;
  split_index(t, groups, nb, o, b, g);
  const int64_t bs = BS ? (int64_t)BS : bs_rt;
  const int64_t k0 = b * bs;
  const int64_t rows = (n - k0 < bs) ? n - k0 : bs;
  const int64_t off = (o * n + k0) * inner + g * VEC;
  const T* vp = V + off;
  float* pp = P + off;

  float amax[VEC];
#pragma unroll
  for (int j = 0; j < VEC; ++j) amax[j] = 0.0f;

  if constexpr (BS > 0) {
    float v[BS][VEC];
#pragma unroll
    for (int r = 0; r < BS; ++r) {
      if (r < rows) {
        load_vec<T, VEC>(vp + (int64_t)r * inner, v[r]);
      } else {
#pragma unroll
        for (int j = 0; j < VEC; ++j) v[r][j] = 0.0f;
      }
#pragma unroll
      for (int j = 0; j < VEC; ++j) amax[j] = amax_combine(amax[j], fabsf(v[r][j]));
    }
    Div d[VEC];
    float xs[VEC];
#pragma unroll
    for (int j = 0; j < VEC; ++j) {
      xs[j] = block_scale(amax[j], s);
      d[j] = make_div(xs[j]);
    }
#pragma unroll
    for (int r = 0; r < BS; ++r) {
      if (r < rows) {
        float q[VEC];
#pragma unroll
        for (int j = 0; j < VEC; ++j) q[j] = elem_q<ELEM>(s.scale_rule ? apply_div(v[r][j], d[j]) : v[r][j], s);
        store_vec<VEC>(pp + (int64_t)r * inner, q);
      }
    }
    store_vec<VEC>(X + (o * nb + b) * inner + g * VEC, xs);
  } else {
    for (int64_t r = 0; r < rows; ++r) {
      float v[VEC];
      load_vec<T, VEC>(vp + r * inner, v);
#pragma unroll
      for (int j = 0; j < VEC; ++j) amax[j] = amax_combine(amax[j], fabsf(v[j]));
    }
    Div d[VEC];
    float xs[VEC];
#pragma unroll
    for (int j = 0; j < VEC; ++j) {
      xs[j] = block_scale(amax[j], s);
      d[j] = make_div(xs[j]);
    }
    for (int64_t r = 0; r < rows; ++r) {
      float v[VEC], q[VEC];
      load_vec<T, VEC>(vp + r * inner, v);
#pragma unroll
      for (int j = 0; j < VEC; ++j) q[j] = elem_q<ELEM>(s.scale_rule ? apply_div(v[j], d[j]) : v[j], s);
      store_vec<VEC>(pp + r * inner, q);
    }
    store_vec<VEC>(X + (o * nb + b) * inner + g * VEC, xs);
  }
}

// inner == 1, blocks of 32 contiguous elements, n % 32 == 0: eight lanes per block, four elements per lane.
template <typename T, int ELEM>
__global__ void __launch_bounds__(256) k_quant_contig32(const T* __restrict__ V, float* __restrict__ P,
                                                        float* __restrict__ X, int64_t nblocks, mxq_block_spec s) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t blk = t >> 3;
  const bool live = blk < nblocks;
  const int64_t off = t * 4;
  float v[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  if (live) load_vec<T, 4>(V + off, v);
  float a = 0.0f;
#pragma unroll
  for (int j = 0; j < 4; ++j) a = amax_combine(a, fabsf(v[j]));
  // all 64 lanes take part in the exchanges; lanes past the end hold 0 and belong to no live block
  a = amax_combine(a, __shfl_xor(a, 1, 8));
  a = amax_combine(a, __shfl_xor(a, 2, 8));
  a = amax_combine(a, __shfl_xor(a, 4, 8));
  if (!live) return;
  const float xs = block_scale(a, s);
  const Div d = make_div(xs);
  float q[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) q[j] = elem_q<ELEM>(s.scale_rule ? apply_div(v[j], d) : v[j], s);
  store_vec<4>(P + off, q);
  if ((t & 7) == 0) X[blk] = xs;
}

template <int VEC>
__global__ void __launch_bounds__(256) k_dequant_strided(const float* __restrict__ P, const float* __restrict__ X,
                                                         float* __restrict__ out, int64_t outer, int64_t n,
                                                         int64_t inner, int64_t bs, int64_t nb) {
  const int64_t groups = inner / VEC;
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= outer * nb * groups) return;
  int64_t o, b, g;
  split_index(t, groups, nb, o, b, g);
  const int64_t k0 = b * bs;
  const int64_t rows = (n - k0 < bs) ? n - k0 : bs;
  const int64_t off = (o * n + k0) * inner + g * VEC;
  float xs[VEC];
  {
    VecT<float, VEC> r = *reinterpret_cast<const VecT<float, VEC>*>(X + (o * nb + b) * inner + g * VEC);
#pragma unroll
    for (int j = 0; j < VEC; ++j) xs[j] = r.v[j];
  }
  for (int64_t r = 0; r < rows; ++r) {
    float v[VEC];
    load_vec<float, VEC>(P + off + r * inner, v);
#pragma unroll
    for (int j = 0; j < VEC; ++j) v[j] = v[j] * xs[j];
    store_vec<VEC>(out + off + r * inner, v);
  }
}

// ------------------------------------------------------------------------------------------ host side
int validate(const mxq_block_spec& s) {
  using mxq::invalid;
  if (s.scale_rule < MXQ_SCALE_NONE || s.scale_rule > MXQ_SCALE_OCP_NO_CLIP) return invalid("bad scale_rule");
  if (s.elem < MXQ_ELEM_NONE || s.elem > MXQ_ELEM_MICROSOFT) return invalid("bad elem rule");
  if (s.rounding < 0 || s.rounding > 2) return invalid("bad rounding code");
  if ((s.scale_rule == MXQ_SCALE_OCP || s.scale_rule == MXQ_SCALE_OCP_NO_CLIP) && (s.scale_bits < 1 || s.scale_bits > 30))
    return invalid("bad scale_bits");
  if (s.scale_rule == MXQ_SCALE_OCP_NO_CLIP && s.elem != MXQ_ELEM_MICROSOFT)
    return invalid("ocp_no_clip needs the microsoft element rule's format");
  if (s.elem == MXQ_ELEM_QTORCH || s.elem == MXQ_ELEM_IEEE) {
    if (!((s.e == 8 && s.m == 23) || (s.e >= 1 && s.e <= 8 && s.m >= 1 && s.m <= 22)))
      return invalid("unsupported widths e=" + std::to_string(s.e) + ", m=" + std::to_string(s.m));
  }
  if (s.elem == MXQ_ELEM_OCP) {
    if (!(s.e >= 2 && s.e <= 5 && s.m >= 1 && s.m <= 3)) return invalid("ocp grid needs an OCP element format");
    if (s.via_e && !((s.via_e == 8 && s.via_m == 23) || (s.via_e >= 1 && s.via_e <= 8 && s.via_m >= 1 && s.via_m <= 22)))
      return invalid("unsupported via widths");
  }
  if (s.elem == MXQ_ELEM_MICROSOFT && !(s.e >= 2 && s.e <= 8 && s.m >= 2 && s.m <= 24))
    return invalid("bad microxcaling format parameters");
  return MXQ_OK;
}

template <typename T, int ELEM>
int launch_quant(const T* V, float* P, float* X, int64_t outer, int64_t n, int64_t inner, int64_t bs,
                 const mxq_block_spec& q, hipStream_t st) {
  const int64_t nb = mxq::ceil_div(n, bs);
  const uintptr_t av = reinterpret_cast<uintptr_t>(V), ap = reinterpret_cast<uintptr_t>(P),
                  ax = reinterpret_cast<uintptr_t>(X);
  if (inner == 1 && bs == 32 && n % 32 == 0 && av % (4 * sizeof(T)) == 0 && ap % 16 == 0) {
    const int64_t nblocks = outer * nb;
    k_quant_contig32<T, ELEM><<<mxq::grid_for(nblocks * 8, 256), 256, 0, st>>>(V, P, X, nblocks, q);
    return mxq::check_launch("mxq_block_quantize");
  }
  auto aligned = [&](int vec) {
    return inner % vec == 0 && av % (vec * sizeof(T)) == 0 && ap % (vec * 4) == 0 && ax % (vec * 4) == 0;
  };
  const int vec = aligned(4) ? 4 : (aligned(2) ? 2 : 1);
  const int64_t threads = outer * nb * (inner / vec);
#define MXQ_Q_LAUNCH(VEC, BS)                                                                        \
  k_quant_strided<T, ELEM, VEC, BS><<<mxq::grid_for(threads, 256), 256, 0, st>>>(V, P, X, outer, n, inner, \
                                                                                 bs, nb, q)
  if (bs == 32) {
    if (vec == 4) MXQ_Q_LAUNCH(4, 32);
    else if (vec == 2) MXQ_Q_LAUNCH(2, 32);
    else MXQ_Q_LAUNCH(1, 32);
  } else {
    if (vec == 4) MXQ_Q_LAUNCH(4, 0);
    else if (vec == 2) MXQ_Q_LAUNCH(2, 0);
    else MXQ_Q_LAUNCH(1, 0);
  }
#undef MXQ_Q_LAUNCH
  return mxq::check_launch("mxq_block_quantize");
}

template <typename T>
int dispatch_elem(const T* V, float* P, float* X, int64_t outer, int64_t n, int64_t inner, int64_t bs,
                  const mxq_block_spec& q, hipStream_t st) {
  switch (q.elem) {
    case MXQ_ELEM_QTORCH: return launch_quant<T, MXQ_ELEM_QTORCH>(V, P, X, outer, n, inner, bs, q, st);
    case MXQ_ELEM_IEEE: return launch_quant<T, MXQ_ELEM_IEEE>(V, P, X, outer, n, inner, bs, q, st);
    case MXQ_ELEM_OCP: return launch_quant<T, MXQ_ELEM_OCP>(V, P, X, outer, n, inner, bs, q, st);
    case MXQ_ELEM_MICROSOFT: return launch_quant<T, MXQ_ELEM_MICROSOFT>(V, P, X, outer, n, inner, bs, q, st);
    default: return launch_quant<T, MXQ_ELEM_NONE>(V, P, X, outer, n, inner, bs, q, st);
  }
}

}  // namespace

extern "C" int mxq_block_quantize(const void* V, int32_t v_dtype, float* P, float* X, int64_t outer, int64_t n,
                                  int64_t inner, int64_t block_size, const mxq_block_spec* spec,
                                  mxq_stream_t stream) {
  if (!spec) return mxq::invalid("mxq_block_quantize: spec is NULL");
  if (outer < 0 || n < 0 || inner < 0 || block_size < 1) return mxq::invalid("mxq_block_quantize: bad shape");
  if (int rc = validate(*spec)) return rc;
  if (outer == 0 || n == 0 || inner == 0) return MXQ_OK;
  if (!V || !P || !X) return mxq::invalid("mxq_block_quantize: NULL pointer");
  const mxq_block_spec q = *spec;
  hipStream_t st = mxq::as_stream(stream);
  switch (v_dtype) {
    case MXQ_DT_F32: return dispatch_elem(static_cast<const float*>(V), P, X, outer, n, inner, block_size, q, st);
    case MXQ_DT_BF16: return dispatch_elem(static_cast<const bf16_t*>(V), P, X, outer, n, inner, block_size, q, st);
    case MXQ_DT_F16: return dispatch_elem(static_cast<const f16_t*>(V), P, X, outer, n, inner, block_size, q, st);
    default: return mxq::invalid("mxq_block_quantize: unsupported input dtype");
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
  const int64_t threads = outer * nb * (inner / vec);
  hipStream_t st = mxq::as_stream(stream);
  if (vec == 4)
    k_dequant_strided<4><<<mxq::grid_for(threads, 256), 256, 0, st>>>(P, X, out, outer, n, inner, block_size, nb);
  else if (vec == 2)
    k_dequant_strided<2><<<mxq::grid_for(threads, 256), 256, 0, st>>>(P, X, out, outer, n, inner, block_size, nb);
  else
    k_dequant_strided<1><<<mxq::grid_for(threads, 256), 256, 0, st>>>(P, X, out, outer, n, inner, block_size, nb);
  return mxq::check_launch("mxq_block_dequantize");
}
