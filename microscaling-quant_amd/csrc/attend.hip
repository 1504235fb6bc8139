// Score glue of the batched attention path (mxq/nn/_attention.py:128-139): the steps between the two systolic
// launches that are not matmuls, each one pass over the Z x n*m x Tk scores.
//
//   k_scores_scale_mask  S <- r(r(S * scale) + mask row), in place: the float32 multiply, the rounding r (none,
//                        or bf16 RNE for vector precision "bf16"), the float32 add of the query's mask row, r
//                        again -- the reference's two elementwise steps with their two roundings, read and
//                        written once
//   k_transpose          out (C x R) = in (R x C)^T through 64 x 64 LDS tiles (row padding against bank
//                        conflicts): P^T for the P-side quantizer, whose blocks run along the keys
#include "mxq_common.h"
#include "mxq_numerics.h"

namespace {

constexpr int TT = 64;   // transpose tile

// Scores in groups of G (G = 4: Tk % 4 == 0, one 16-byte load and store per thread; else G = 1), group index
// of type I (uint32 when the scores fit it: cheap divisions).  mask: the row of query j of pair z is
// mask + ((z0 + z) / z_per_b - z0 / z_per_b) * mask_b_stride + j * mask_row_stride (keys contiguous).
template <int G, typename I>
__global__ void __launch_bounds__(256) k_scores_scale_mask(float* __restrict__ S, I groups, I Tk, I n, I m,
                                                           float scale, const float* __restrict__ mask,
                                                           int64_t mask_b_stride, int64_t mask_row_stride,
                                                           int64_t z0, int64_t z_per_b, int bf16) {
  const I t = (I)blockIdx.x * 256 + threadIdx.x;
  if (t >= groups) return;
  const I row = t / (Tk / G);                                     // row = (z * n + i) * m + j
  float v[G];
  float* s = S + (int64_t)t * G;
  if constexpr (G == 4) {
    const float4 q = *reinterpret_cast<const float4*>(s);
    v[0] = q.x, v[1] = q.y, v[2] = q.z, v[3] = q.w;
  } else {
    v[0] = s[0];
  }
#pragma unroll
  for (int e = 0; e < G; ++e) {
    v[e] = v[e] * scale;
    if (bf16) v[e] = bf16_rne(v[e]);
  }
  if (mask) {
    const I j = row % m, z = row / (n * m), k = (I)(t * G - row * Tk);
    const float* mr = mask + ((z0 + (int64_t)z) / z_per_b - z0 / z_per_b) * mask_b_stride +
                      (int64_t)j * mask_row_stride + k;
#pragma unroll
    for (int e = 0; e < G; ++e) {
      v[e] = v[e] + mr[e];
      if (bf16) v[e] = bf16_rne(v[e]);
    }
  }
  if constexpr (G == 4) {
    *reinterpret_cast<float4*>(s) = make_float4(v[0], v[1], v[2], v[3]);
  } else {
    s[0] = v[0];
  }
}

template <typename I>
void launch_scores(float* S, int64_t rows, int64_t n, int64_t m, int64_t Tk, float scale, const float* mask,
                   int64_t mbs, int64_t mrs, int64_t z0, int64_t zpb, int bf16, hipStream_t st) {
  const bool vec = Tk % 4 == 0 && reinterpret_cast<uintptr_t>(S) % 16 == 0;
  const int64_t groups = rows * Tk / (vec ? 4 : 1);
  const dim3 grid = mxq::grid_for(groups, 256);
  if (vec)
    k_scores_scale_mask<4, I><<<grid, 256, 0, st>>>(S, (I)groups, (I)Tk, (I)n, (I)m, scale, mask, mbs, mrs, z0, zpb,
                                                    bf16);
  else
    k_scores_scale_mask<1, I><<<grid, 256, 0, st>>>(S, (I)groups, (I)Tk, (I)n, (I)m, scale, mask, mbs, mrs, z0, zpb,
                                                    bf16);
}

// One 64 x 64 tile per workgroup, tiles numbered row-major over the ceil(R/64) x ceil(C/64) tile grid.
__global__ void __launch_bounds__(256) k_transpose(const float* __restrict__ in, float* __restrict__ out, int64_t R,
                                                   int64_t C, int64_t tiles_c) {
  __shared__ float tile[TT][TT + 1];
  const int64_t tr = blockIdx.x / tiles_c, tc = blockIdx.x - tr * tiles_c;
  const int64_t r0 = tr * TT, c0 = tc * TT;
  const int tx = threadIdx.x % TT, ty = threadIdx.x / TT;          // 64 x 4 threads
#pragma unroll
  for (int i = 0; i < TT; i += 4) {
    const int64_t r = r0 + ty + i, c = c0 + tx;
    if (r < R && c < C) tile[ty + i][tx] = in[r * C + c];
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < TT; i += 4) {
    const int64_t c = c0 + ty + i, r = r0 + tx;
    if (c < C && r < R) out[c * R + r] = tile[tx][ty + i];
  }
}

}  // namespace

extern "C" int mxq_scores_scale_mask(float* S, int64_t Z, int64_t n, int64_t m, int64_t Tk, float scale,
                                     const float* mask, int64_t mask_b_stride, int64_t mask_row_stride, int64_t z0,
                                     int64_t z_per_b, int32_t round_bf16, mxq_stream_t stream) {
  if (Z < 0 || n < 0 || m < 0 || Tk < 0 || z0 < 0 || z_per_b < 1)
    return mxq::invalid("mxq_scores_scale_mask: bad shape");
  const int64_t rows = Z * n * m;
  if (rows == 0 || Tk == 0) return MXQ_OK;
  if (!S) return mxq::invalid("mxq_scores_scale_mask: NULL scores");
  if (mxq::ceil_div(rows * Tk, 256) > INT32_MAX) return mxq::invalid("mxq_scores_scale_mask: too many scores");
  if (mask && (mask_row_stride < 0 || mask_b_stride < 0))
    return mxq::invalid("mxq_scores_scale_mask: bad mask strides");
  if (rows * Tk < ((int64_t)1 << 31))             // thread indices stay far from uint32 wrap-around
    launch_scores<uint32_t>(S, rows, n, m, Tk, scale, mask, mask_b_stride, mask_row_stride, z0, z_per_b,
                            round_bf16 ? 1 : 0, mxq::as_stream(stream));
  else
    launch_scores<int64_t>(S, rows, n, m, Tk, scale, mask, mask_b_stride, mask_row_stride, z0, z_per_b,
                           round_bf16 ? 1 : 0, mxq::as_stream(stream));
  return mxq::check_launch("mxq_scores_scale_mask");
}

extern "C" int mxq_transpose(const float* in, float* out, int64_t R, int64_t C, mxq_stream_t stream) {
  if (R < 0 || C < 0) return mxq::invalid("mxq_transpose: bad shape");
  if (R == 0 || C == 0) return MXQ_OK;
  if (!in || !out) return mxq::invalid("mxq_transpose: NULL pointer");
  const int64_t tiles_c = mxq::ceil_div(C, TT), tiles = mxq::ceil_div(R, TT) * tiles_c;
  if (tiles > INT32_MAX) return mxq::invalid("mxq_transpose: matrix too large");
  k_transpose<<<dim3((unsigned)tiles), 256, 0, mxq::as_stream(stream)>>>(in, out, R, C, tiles_c);
  return mxq::check_launch("mxq_transpose");
}
