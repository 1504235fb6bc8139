// microxcaling's "dither" rounding (mxq/microxcaling/elemwise.py:41-43): the element step rounds
// sign(A) * floor(|A| + u) with u drawn by torch.rand_like(A) for every element of the tensor it rounds.  The
// draws come from the caller (the Python layer draws them with torch, as the reference does, in its order and
// on its device); these kernels apply them.
//   mxq_microsoft_dither        the element step on a flat tensor, u[i] for element i
//   mxq_scale_factor_dither     scale_factor.ocp_no_clip, u[i] for block maximum i (its rounding of amax / X)
//   mxq_block_quantize_dither   block.ocp: amax, the scale rule (ocp_no_clip rounding amax / X with u_amax),
//                               the division and the element step, one thread per block column.  The draws
//                               are indexed as the reference's blocked tensors hold them: V viewed as (outer,
//                               n, inner) becomes (outer * inner, nb, block) with the block axis last (moved,
//                               then zero-padded), so element (o, k, i) takes u[((o * inner + i) * nb + k / bs) *
//                               bs + k % bs] and its block's maximum u_amax[(o * inner + i) * nb + k / bs].
// Dither is a rounding for experiments, not a hot path: the block kernel is a plain one, coalesced across the
// inner columns.
#include "mxq_common.h"
#include "mxq_numerics.h"
#include "quantize_impl.h"

namespace {

constexpr int kThreads = 256;

__global__ void __launch_bounds__(kThreads) k_microsoft_dither(const float* __restrict__ z, const float* __restrict__ u,
                                                              float* __restrict__ out, int64_t n, int ebits, int mbits,
                                                              float max_norm, int saturate) {
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += (int64_t)gridDim.x * kThreads)
    out[i] = microsoft_quantize_t<MXQ_DITHER>(z[i], ebits, mbits, max_norm, saturate != 0, u[i]);
}

__global__ void __launch_bounds__(kThreads) k_scale_dither(const float* __restrict__ amax, const float* __restrict__ u,
                                                          float* __restrict__ out, int64_t n, mxq_block_spec s) {
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += (int64_t)gridDim.x * kThreads)
    out[i] = scale_ocp_no_clip(amax[i], s.scale_emax, s.scale_bits, s.e, s.m, s.max_norm, MXQ_DITHER, u[i]);
}

template <typename T>
__global__ void __launch_bounds__(kThreads) k_quant_dither(const T* __restrict__ V, const float* __restrict__ u_amax,
                                                          const float* __restrict__ u, float* __restrict__ P,
                                                          float* __restrict__ X, int64_t outer, int64_t n,
                                                          int64_t inner, int64_t bs, int64_t nb, mxq_block_spec s) {
  const int64_t total = outer * nb * inner;
  for (int64_t t = (int64_t)blockIdx.x * kThreads + threadIdx.x; t < total; t += (int64_t)gridDim.x * kThreads) {
    const int64_t i = t % inner, ob = t / inner, b = ob % nb, o = ob / nb;
    const int64_t k0 = b * bs, k1 = k0 + bs < n ? k0 + bs : n;
    const T* src = V + o * n * inner + i;
    uint32_t am = 0u;                                  // |v| bit patterns: NaN lies above +Inf and wins
    for (int64_t k = k0; k < k1; ++k) am = max(am, f2u(mxq_quant::to_f32(src[k * inner])) & 0x7FFFFFFFu);
    const int64_t blk = (o * inner + i) * nb + b;     // the block's index in the reference's (..., nb) layout
    float xs = 1.0f;
    if (s.scale_rule == MXQ_SCALE_OCP_NO_CLIP)
      xs = scale_ocp_no_clip(u2f(am), s.scale_emax, s.scale_bits, s.e, s.m, s.max_norm, MXQ_DITHER, u_amax[blk]);
    else if (s.scale_rule)
      xs = block_scale(u2f(am), s);
    X[(o * nb + b) * inner + i] = xs;
    const Div d = make_div(xs);
    for (int64_t k = k0; k < k1; ++k) {
      const float v = mxq_quant::to_f32(src[k * inner]);
      const float z = s.scale_rule ? apply_div(v, d) : v;
      P[(o * n + k) * inner + i] = microsoft_quantize_t<MXQ_DITHER>(z, s.e, s.m, s.max_norm, true, u[blk * bs + k - k0]);
    }
  }
}

dim3 grid_of(int64_t n) {
  int64_t blocks = mxq::ceil_div(n, kThreads);
  if (blocks > 65536) blocks = 65536;
  return dim3((unsigned)(blocks < 1 ? 1 : blocks));
}

bool ms_format_ok(int ebits, int mbits) { return ebits >= 2 && ebits <= 8 && mbits >= 2 && mbits <= 24; }

}  // namespace

extern "C" int mxq_microsoft_dither(const float* z, const float* u, float* out, int64_t n, int32_t ebits,
                                    int32_t mbits, float max_norm, int32_t saturate, mxq_stream_t stream) {
  if (n < 0 || !ms_format_ok(ebits, mbits)) return mxq::invalid("mxq_microsoft_dither: bad size or format");
  if (n == 0) return MXQ_OK;
  if (!z || !u || !out) return mxq::invalid("mxq_microsoft_dither: NULL pointer");
  k_microsoft_dither<<<grid_of(n), kThreads, 0, mxq::as_stream(stream)>>>(z, u, out, n, ebits, mbits, max_norm,
                                                                          saturate);
  return mxq::check_launch("mxq_microsoft_dither");
}

extern "C" int mxq_scale_factor_dither(const float* amax, const float* u, float* out, int64_t n,
                                       const mxq_block_spec* spec, mxq_stream_t stream) {
  if (!spec || spec->scale_rule != MXQ_SCALE_OCP_NO_CLIP || !ms_format_ok(spec->e, spec->m) ||
      spec->scale_bits < 1 || spec->scale_bits > 30 || n < 0)
    return mxq::invalid("mxq_scale_factor_dither: the spec must be ocp_no_clip's with a microxcaling format");
  if (n == 0) return MXQ_OK;
  if (!amax || !u || !out) return mxq::invalid("mxq_scale_factor_dither: NULL pointer");
  k_scale_dither<<<grid_of(n), kThreads, 0, mxq::as_stream(stream)>>>(amax, u, out, n, *spec);
  return mxq::check_launch("mxq_scale_factor_dither");
}

extern "C" int mxq_block_quantize_dither(const void* V, int32_t v_dtype, const float* u_amax, const float* u,
                                         float* P, float* X, int64_t outer, int64_t n, int64_t inner,
                                         int64_t block_size, const mxq_block_spec* spec, mxq_stream_t stream) {
  if (!spec) return mxq::invalid("mxq_block_quantize_dither: spec is NULL");
  if (outer < 0 || n < 0 || inner < 0 || block_size < 1) return mxq::invalid("mxq_block_quantize_dither: bad shape");
  mxq_block_spec q = *spec;
  if (q.elem != MXQ_ELEM_MICROSOFT || !ms_format_ok(q.e, q.m))
    return mxq::invalid("mxq_block_quantize_dither: the element rule must be microxcaling's");
  q.rounding = MXQ_RNE;                                // validated as a plain mode; the kernel rounds by dither
  if (int rc = mxq_quant::validate(q)) return rc;
  if (outer == 0 || n == 0 || inner == 0) return MXQ_OK;
  if (!V || !u || !P || !X || (q.scale_rule == MXQ_SCALE_OCP_NO_CLIP && !u_amax))
    return mxq::invalid("mxq_block_quantize_dither: NULL pointer");
  const int64_t nb = mxq::ceil_div(n, block_size), total = outer * nb * inner;
  const dim3 g = grid_of(total);
  hipStream_t st = mxq::as_stream(stream);
  switch (v_dtype) {
    case MXQ_DT_F32:
      k_quant_dither<float><<<g, kThreads, 0, st>>>(static_cast<const float*>(V), u_amax, u, P, X, outer, n, inner,
                                                    block_size, nb, q);
      break;
    case MXQ_DT_BF16:
      k_quant_dither<mxq_quant::bf16_t><<<g, kThreads, 0, st>>>(static_cast<const mxq_quant::bf16_t*>(V), u_amax, u,
                                                                P, X, outer, n, inner, block_size, nb, q);
      break;
    case MXQ_DT_F16:
      k_quant_dither<mxq_quant::f16_t><<<g, kThreads, 0, st>>>(static_cast<const mxq_quant::f16_t*>(V), u_amax, u,
                                                               P, X, outer, n, inner, block_size, nb, q);
      break;
    default: return mxq::invalid("mxq_block_quantize_dither: unsupported input dtype");
  }
  return mxq::check_launch("mxq_block_quantize_dither");
}
