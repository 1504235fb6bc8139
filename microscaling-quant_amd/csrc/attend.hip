// Glue of the batched attention path (mxq/nn/_attention.py:108-141), around the two systolic launches:
//   k_group_amax         per contraction row, the max over each column group of |code| * its block scale (the
//                        masked-key bound's factors, one group per call)
//   k_attend_windows     per call, the masked-key bound and whether the call keeps every key (its first and last
//                        key blocks each hold a key some query still sees)
//   k_scores_scale_mask  S <- r(r(S * scale) + mask row) in place over the Z x n*m x Tk scores: the float32
//                        multiply, the rounding r (none, or bf16 RNE for vector precision "bf16"), the float32
//                        add of the query's mask row, r again -- the reference's two elementwise steps with their
//                        two roundings, read and written once.
//   k_mask_minabs        per mask batch row, 32-row group of a call's n*m score rows and 32-key group, the
//                        smallest |mask| (0 for a NaN) and the largest mask value
//   k_attend_hints       the two batched launches' hints (include/mxq_hip.h mxq_systolic_hints) from those and
//                        each call's masked-key bound b: a 32 x 32 group of scores is not needed when its
//                        smallest |mask| c absorbs 2b (c + 2b == c and c - 2b == c in float32), for then every
//                        mask value there absorbs every score the call can produce, r(r(s * scale) + mask) is
//                        r(mask) whatever s is, and a +0 score gives the same; k_end of a 64-row group is the
//                        end of its last key group that some of its rows still see, and the largest mask value
//                        past it (the largest score there, for the softmax).  Where every key of a row is
//                        masked softmax is uniform, not zero, and the systolic kernel's check of the rows past
//                        k_end sends that tile to the general kernel.
#include "mxq_common.h"
#include "mxq_numerics.h"

namespace {

constexpr int ZCH = 8;   // problems per thread

// One thread per group of G scores (G = 4: Tk % 4 == 0, 16-byte loads and stores; else G = 1) of one row of the
// n*m x Tk score matrix, for ZCH consecutive problems: the mask values are loaded once per batch row of the mask
// and the ZCH score loads are issued together.  Index type I: uint32 when the counts fit it (cheap divisions).
// The mask row of query j of problem z: mask + ((z0 + z) / z_per_b - z0 / z_per_b) * mask_b_stride
// + j * mask_row_stride, keys contiguous.
template <int G, typename I>
__global__ void __launch_bounds__(256) k_scores_scale_mask(float* __restrict__ S, I per_problem, I Z, I Tk, I m,
                                                           I zchunks, float scale, const float* __restrict__ mask,
                                                           int64_t mask_b_stride, int64_t mask_row_stride,
                                                           int64_t z0, int64_t z_per_b, int bf16) {
  const I t = (I)blockIdx.x * 256 + threadIdx.x;
  if (t >= per_problem * zchunks) return;
  const I zc = t / per_problem, g = t - zc * per_problem;   // g: group within one problem's n*m x Tk scores
  const I row = g / (Tk / G), k = g * G - row * Tk;         // row = i * m + j
  const I j = row % m;
  const I zb = zc * ZCH;
  float v[ZCH][G];
#pragma unroll
  for (int u = 0; u < ZCH; ++u) {
    if (zb + u < Z) {
      const float* s = S + ((int64_t)(zb + u) * per_problem + g) * G;
      if constexpr (G == 4) {
        const float4 q = *reinterpret_cast<const float4*>(s);
        v[u][0] = q.x, v[u][1] = q.y, v[u][2] = q.z, v[u][3] = q.w;
      } else {
        v[u][0] = s[0];
      }
    }
  }
  float mv[G];
  int64_t b_prev = -1;
#pragma unroll
  for (int u = 0; u < ZCH; ++u) {
    if (zb + u >= Z) break;
#pragma unroll
    for (int e = 0; e < G; ++e) {
      v[u][e] = v[u][e] * scale;
      if (bf16) v[u][e] = bf16_rne(v[u][e]);
    }
    if (mask) {
      const int64_t b = (z0 + (int64_t)(zb + u)) / z_per_b - z0 / z_per_b;
      if (b != b_prev) {
        const float* mr = mask + b * mask_b_stride + (int64_t)j * mask_row_stride + k;
#pragma unroll
        for (int e = 0; e < G; ++e) mv[e] = mr[e];
        b_prev = b;
      }
#pragma unroll
      for (int e = 0; e < G; ++e) {
        v[u][e] = v[u][e] + mv[e];
        if (bf16) v[u][e] = bf16_rne(v[u][e]);
      }
    }
    float* s = S + ((int64_t)(zb + u) * per_problem + g) * G;
    if constexpr (G == 4) {
      *reinterpret_cast<float4*>(s) = make_float4(v[u][0], v[u][1], v[u][2], v[u][3]);
    } else {
      s[0] = v[u][0];
    }
  }
}

template <typename I>
void launch_scores(float* S, int64_t Z, int64_t n, int64_t m, int64_t Tk, float scale, const float* mask,
                   int64_t mbs, int64_t mrs, int64_t z0, int64_t zpb, int bf16, hipStream_t st) {
  const bool vec = Tk % 4 == 0 && reinterpret_cast<uintptr_t>(S) % 16 == 0;
  const int64_t per_problem = n * m * Tk / (vec ? 4 : 1), zchunks = mxq::ceil_div(Z, ZCH);
  const dim3 grid = mxq::grid_for(per_problem * zchunks, 256);
  if (vec)
    k_scores_scale_mask<4, I><<<grid, 256, 0, st>>>(S, (I)per_problem, (I)Z, (I)Tk, (I)m, (I)zchunks, scale, mask,
                                                    mbs, mrs, z0, zpb, bf16);
  else
    k_scores_scale_mask<1, I><<<grid, 256, 0, st>>>(S, (I)per_problem, (I)Z, (I)Tk, (I)m, (I)zchunks, scale, mask,
                                                    mbs, mrs, z0, zpb, bf16);
}

// One workgroup per (contraction row k, column group g): out[k * groups + g] = max over the group's columns c of
// |P[k, c]| * X[k / bs, c] (float32 products, as float64).  The max is taken over the products' bit patterns:
// non-negative floats order like their patterns and every NaN pattern lies above +Inf, so a NaN wins as
// torch.amax's does.
__global__ void __launch_bounds__(256) k_group_amax(const float* __restrict__ P, const float* __restrict__ X,
                                                    int64_t cols, int64_t groups, int64_t bs, double* __restrict__ out) {
  __shared__ uint32_t part[4];
  const int64_t k = blockIdx.x / groups, g = blockIdx.x - k * groups;
  const int64_t per = cols / groups;
  const float* p = P + k * cols + g * per;
  const float* x = X + (k / bs) * cols + g * per;
  uint32_t am = 0u;
  // eight columns a thread per round, every load issued before the first product
  constexpr int PER = 8;
  for (int64_t c0 = threadIdx.x; c0 < per; c0 += 256 * PER) {
    float pv[PER], xv[PER];
#pragma unroll
    for (int u = 0; u < PER; ++u) {
      const int64_t c = c0 + 256 * u;
      pv[u] = c < per ? p[c] : 0.0f;
      xv[u] = c < per ? x[c] : 0.0f;
    }
#pragma unroll
    for (int u = 0; u < PER; ++u) am = max(am, f2u(fabsf(pv[u]) * xv[u]) & 0x7FFFFFFFu);
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) am = max(am, (uint32_t)__shfl_xor((int)am, off, 64));
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = am;
  __syncthreads();
  if (threadIdx.x == 0) out[blockIdx.x] = (double)u2f(max(max(part[0], part[1]), max(part[2], part[3])));
}

// Workgroup (z, chunk) of the Z x chunks grid checks query rows [chunk * WROWS, +WROWS) of call z.  Its bound:
// max(slack_scale * sum over d of amax_a[d, z] * amax_k[d, z], FLT_MIN) in float64, b32 = float(bound); a mask
// value c absorbs the call's scores when c + b32 == c and c - b32 == c (float32).  Its word of flags
// (z * chunks + chunk, written whole: nothing to clear first) holds bit 0 when some checked row leaves a key of
// the first key block unabsorbed, bit 1 for the last block; Tk <= block sets both.  The mask row of query j of
// call z as in k_scores_scale_mask.
constexpr int WROWS = 64;

// Thread 0 gets the masked-key bound of call z: slack_scale * the float64 sum over d, in d order, of
// amax_a[d * lda + z] * amax_k[d * ldk + z], at least the smallest normal float32 (a NaN stays NaN).  The whole
// workgroup loads and multiplies 256 terms at a time into `terms`; thread 0 adds them in order.  Every thread
// of the workgroup must call it.
__device__ double call_bound(const double* __restrict__ amax_a, int64_t lda, const double* __restrict__ amax_k,
                             int64_t ldk, int64_t D, int64_t z, double slack_scale, double* terms) {
  double sum = 0.0;
  for (int64_t d0 = 0; d0 < D; d0 += 256) {
    const int64_t d = d0 + threadIdx.x;
    if (d < D) terms[threadIdx.x] = amax_a[d * lda + z] * amax_k[d * ldk + z];
    __syncthreads();
    if (threadIdx.x == 0) {
      const int64_t n = D - d0 < 256 ? D - d0 : 256;
      for (int64_t e = 0; e < n; ++e) sum += terms[e];
    }
    __syncthreads();
  }
  double bound = slack_scale * sum;
  if (bound < 1.1754943508222875e-38) bound = 1.1754943508222875e-38;
  return bound;
}

__global__ void __launch_bounds__(256) k_attend_windows(const double* __restrict__ amax_a, int64_t lda,
                                                        const double* __restrict__ amax_k, int64_t ldk, int64_t D,
                                                        double slack_scale, const float* __restrict__ mask,
                                                        int64_t mask_b_stride, int64_t mask_row_stride, int64_t z0,
                                                        int m, int Tk, int block, int chunks,
                                                        int64_t z_per_b, int32_t* __restrict__ flags) {
  __shared__ float b32;
  const int z = blockIdx.x / chunks, chunk = blockIdx.x - z * chunks;
  if (Tk <= block) {
    if (threadIdx.x == 0) flags[blockIdx.x] = 3;
    return;
  }
  __shared__ double terms[256];
  const double bound = call_bound(amax_a, lda, amax_k, ldk, D, z, slack_scale, terms);
  if (threadIdx.x == 0) b32 = (float)bound;
  __syncthreads();
  const float bnd = b32;
  const float* rows = mask + ((z0 + z) / z_per_b - z0 / z_per_b) * mask_b_stride;
  const int last0 = (Tk - 1) / block * block, j0 = chunk * WROWS;
  const int nrows = min(WROWS, m - j0);
  int live = 0;
  // eight elements of each of the two blocks a thread per round, every load issued before any is tested
  constexpr int PER = 8;
  const int total = nrows * block;
  for (int i0 = threadIdx.x; i0 < total; i0 += 256 * PER) {
    float c[PER], e[PER];
    bool in[PER], in_last[PER];
#pragma unroll
    for (int u = 0; u < PER; ++u) {
      const int i = i0 + 256 * u;
      in[u] = i < total;
      const int j = in[u] ? i / block : 0, key = in[u] ? i - j * block : 0;
      const float* r = rows + (int64_t)(j0 + j) * mask_row_stride;
      c[u] = in[u] ? r[key] : 0.0f;                           // key < block < Tk
      in_last[u] = in[u] && last0 + key < Tk;
      e[u] = in_last[u] ? r[last0 + key] : 0.0f;
    }
#pragma unroll
    for (int u = 0; u < PER; ++u) {
      if (in[u] && !((c[u] + bnd) == c[u] && (c[u] - bnd) == c[u])) live |= 1;
      if (in_last[u] && !((e[u] + bnd) == e[u] && (e[u] - bnd) == e[u])) live |= 2;
    }
  }
  const int first = __syncthreads_or(live & 1), last = __syncthreads_or(live & 2);
  if (threadIdx.x == 0) flags[blockIdx.x] = (first ? 1 : 0) | (last ? 2 : 0);
}

__global__ void __launch_bounds__(256) k_mask_minabs(const float* __restrict__ mask, int64_t mask_b_stride,
                                                     int64_t mask_row_stride, int64_t rows, int64_t m, int64_t Tk,
                                                     int64_t rgroups, int64_t kgroups, float* __restrict__ out,
                                                     float* __restrict__ maxval) {
  const int64_t bb = blockIdx.z, rg = blockIdx.y, key = (int64_t)blockIdx.x * 256 + threadIdx.x;
  float mn = f_inf(), mx = -f_inf();                           // keys past Tk take no part
  if (key < Tk) {
    const int64_t r0 = rg * 32, q0 = r0 % m;
    if (r0 + 32 <= rows && q0 + 32 <= m) {
      // 32 consecutive mask rows: every load issued before the first is used
      const float* col = mask + bb * mask_b_stride + q0 * mask_row_stride + key;
      float c[32];
#pragma unroll
      for (int i = 0; i < 32; ++i) c[i] = col[i * mask_row_stride];
#pragma unroll
      for (int i = 0; i < 32; ++i) {
        mn = fminf(mn, c[i] != c[i] ? 0.0f : fabsf(c[i]));
        mx = fmaxf(mx, c[i]);                                  // a NaN takes no part
      }
    } else {
      for (int i = 0; i < 32; ++i) {
        const int64_t r = r0 + i;
        if (r >= rows) break;
        const float c = mask[bb * mask_b_stride + (r % m) * mask_row_stride + key];
        mn = fminf(mn, c != c ? 0.0f : fabsf(c));
        mx = fmaxf(mx, c);                                     // a NaN takes no part
      }
    }
  }
  for (int off = 16; off > 0; off >>= 1) {
    mn = fminf(mn, __shfl_xor(mn, off, 32));
    mx = fmaxf(mx, __shfl_xor(mx, off, 32));
  }
  const int64_t kg = key >> 5;
  if ((threadIdx.x & 31) == 0 && kg < kgroups) {
    out[(bb * rgroups + rg) * kgroups + kg] = mn;
    if (maxval) maxval[(bb * rgroups + rg) * kgroups + kg] = mx;
  }
}

// Workgroup (t, z): 64-row group t of call z.  The bound as k_attend_windows takes it.
__global__ void __launch_bounds__(256) k_attend_hints(const double* __restrict__ amax_a, int64_t lda,
                                                      const double* __restrict__ amax_k, int64_t ldk, int64_t D,
                                                      double slack_scale, const float* __restrict__ minabs,
                                                      int64_t z0, int64_t z_per_b, int batched, int64_t rgroups,
                                                      int64_t kgroups, int64_t tgroups, uint8_t* __restrict__ skip,
                                                      int32_t* __restrict__ k_end, const float* __restrict__ maxval,
                                                      float* __restrict__ tail_max) {
  __shared__ float b2;
  __shared__ int last;
  __shared__ float tmax[4];
  const int64_t t = blockIdx.x, z = blockIdx.y;
  const int64_t bb = batched ? (z0 + z) / z_per_b - z0 / z_per_b : 0;
  // with at most 256 key groups a thread tests one of each of the two row groups: its minimum (and largest
  // value) loaded before the bound is formed, so their latency and the bound's overlap
  const bool one = kgroups <= 256;
  float pre_c[2] = {0.0f, 0.0f}, pre_v[2] = {-f_inf(), -f_inf()};
  bool pre_in[2] = {false, false};
#pragma unroll
  for (int g = 0; g < 2; ++g) {
    const int64_t rg = 2 * t + g;
    pre_in[g] = one && rg < rgroups && threadIdx.x < kgroups;
    if (pre_in[g]) {
      pre_c[g] = minabs[(bb * rgroups + rg) * kgroups + threadIdx.x];
      if (maxval) pre_v[g] = maxval[(bb * rgroups + rg) * kgroups + threadIdx.x];
    }
  }
  __shared__ double terms[256];
  const double bound = call_bound(amax_a, lda, amax_k, ldk, D, z, slack_scale, terms);
  if (threadIdx.x == 0) {
    b2 = (float)(2.0 * bound);
    last = -1;
  }
  __syncthreads();
  const float b = b2;
  const bool usable = is_finite_f(b);
  int mine = -1;
  if (one) {
#pragma unroll
    for (int g = 0; g < 2; ++g) {
      if (!pre_in[g]) continue;
      const float c = pre_c[g];
      const bool sk = usable && (c + b) == c && (c - b) == c;
      skip[(z * rgroups + 2 * t + g) * kgroups + threadIdx.x] = sk ? 1 : 0;
      if (!sk) mine = (int)threadIdx.x;
    }
  } else {
    for (int64_t rg = 2 * t; rg < 2 * t + 2 && rg < rgroups; ++rg) {
      const float* mrow = minabs + (bb * rgroups + rg) * kgroups;
      uint8_t* srow = skip + (z * rgroups + rg) * kgroups;
      for (int64_t kg = threadIdx.x; kg < kgroups; kg += 256) {
        const float c = mrow[kg];
        const bool sk = usable && (c + b) == c && (c - b) == c;
        srow[kg] = sk ? 1 : 0;
        if (!sk && kg > mine) mine = (int)kg;
      }
    }
  }
  atomicMax(&last, mine);
  __syncthreads();
  if (threadIdx.x == 0) k_end[z * tgroups + t] = (int32_t)((last + 1) * 32);
  if (!tail_max) return;
  // the largest mask value of the groups past k_end (every one of them skipped): the largest score there
  float tm = -f_inf();
  if (one) {
    const int lst = last;
#pragma unroll
    for (int g = 0; g < 2; ++g)
      if (pre_in[g] && (int)threadIdx.x > lst) tm = fmaxf(tm, pre_v[g]);
  } else {
    for (int64_t rg = 2 * t; rg < 2 * t + 2 && rg < rgroups; ++rg) {
      const float* vrow = maxval + (bb * rgroups + rg) * kgroups;
      for (int64_t kg = last + 1 + threadIdx.x; kg < kgroups; kg += 256) tm = fmaxf(tm, vrow[kg]);
    }
  }
  for (int off = 32; off > 0; off >>= 1) tm = fmaxf(tm, __shfl_xor(tm, off, 64));
  if ((threadIdx.x & 63) == 0) tmax[threadIdx.x >> 6] = tm;
  __syncthreads();
  if (threadIdx.x == 0) tail_max[z * tgroups + t] = fmaxf(fmaxf(tmax[0], tmax[1]), fmaxf(tmax[2], tmax[3]));
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
  if (mxq::ceil_div(n * m * Tk * mxq::ceil_div(Z, ZCH), 256) > INT32_MAX)
    return mxq::invalid("mxq_scores_scale_mask: too many scores");
  if (mask && (mask_row_stride < 0 || mask_b_stride < 0))
    return mxq::invalid("mxq_scores_scale_mask: bad mask strides");
  if (rows * Tk < ((int64_t)1 << 31))             // thread indices stay far from uint32 wrap-around
    launch_scores<uint32_t>(S, Z, n, m, Tk, scale, mask, mask_b_stride, mask_row_stride, z0, z_per_b,
                            round_bf16 ? 1 : 0, mxq::as_stream(stream));
  else
    launch_scores<int64_t>(S, Z, n, m, Tk, scale, mask, mask_b_stride, mask_row_stride, z0, z_per_b,
                           round_bf16 ? 1 : 0, mxq::as_stream(stream));
  return mxq::check_launch("mxq_scores_scale_mask");
}

extern "C" int mxq_group_amax(const float* P, const float* X, int64_t K, int64_t cols, int64_t groups,
                              int64_t block_size, double* out, mxq_stream_t stream) {
  if (K < 0 || cols < 0 || groups < 1 || block_size < 1 || cols % groups)
    return mxq::invalid("mxq_group_amax: bad shape");
  if (K == 0) return MXQ_OK;
  if (!P || !X || !out) return mxq::invalid("mxq_group_amax: NULL pointer");
  if (K * groups > INT32_MAX) return mxq::invalid("mxq_group_amax: too many groups");
  k_group_amax<<<dim3((unsigned)(K * groups)), 256, 0, mxq::as_stream(stream)>>>(P, X, cols, groups, block_size, out);
  return mxq::check_launch("mxq_group_amax");
}

extern "C" int mxq_attend_windows(const double* amax_a, int64_t lda, const double* amax_k, int64_t ldk, int64_t D,
                                  int64_t Z, double slack_scale, const float* mask, int64_t mask_b_stride,
                                  int64_t mask_row_stride, int64_t z0, int64_t z_per_b, int64_t m, int64_t Tk,
                                  int64_t block, int32_t* flags, mxq_stream_t stream) {
  if (D < 0 || Z < 0 || m < 1 || Tk < 0 || block < 1 || z0 < 0 || z_per_b < 1 || lda < Z || ldk < Z ||
      mask_b_stride < 0 || mask_row_stride < 0)
    return mxq::invalid("mxq_attend_windows: bad shape");
  if (Z == 0) return MXQ_OK;
  if (!amax_a || !amax_k || !mask || !flags) return mxq::invalid("mxq_attend_windows: NULL pointer");
  const int64_t chunks = mxq::ceil_div(m, WROWS);
  if (Tk > INT32_MAX || m * block > INT32_MAX || Z * chunks > INT32_MAX)
    return mxq::invalid("mxq_attend_windows: too large");
  k_attend_windows<<<dim3((unsigned)(Z * chunks)), 256, 0, mxq::as_stream(stream)>>>(
      amax_a, lda, amax_k, ldk, D, slack_scale, mask, mask_b_stride, mask_row_stride, z0, (int)m, (int)Tk,
      (int)block, (int)chunks, z_per_b, flags);
  return mxq::check_launch("mxq_attend_windows");
}

extern "C" int mxq_mask_minabs(const float* mask, int64_t mask_b_stride, int64_t mask_row_stride, int64_t batches,
                               int64_t rows, int64_t m, int64_t Tk, float* out, float* maxval, mxq_stream_t stream) {
  if (batches < 0 || rows < 0 || m < 1 || Tk < 0 || mask_b_stride < 0 || mask_row_stride < 0)
    return mxq::invalid("mxq_mask_minabs: bad shape");
  if (batches == 0 || rows == 0 || Tk == 0) return MXQ_OK;
  if (!mask || !out) return mxq::invalid("mxq_mask_minabs: NULL pointer");
  const int64_t rgroups = mxq::ceil_div(rows, 32), kgroups = mxq::ceil_div(Tk, 32);
  if (rgroups > 65535 || batches > 65535 || mxq::ceil_div(Tk, 256) > INT32_MAX)
    return mxq::invalid("mxq_mask_minabs: too large");
  const dim3 grid((unsigned)mxq::ceil_div(Tk, 256), (unsigned)rgroups, (unsigned)batches);
  k_mask_minabs<<<grid, 256, 0, mxq::as_stream(stream)>>>(mask, mask_b_stride, mask_row_stride, rows, m, Tk, rgroups,
                                                          kgroups, out, maxval);
  return mxq::check_launch("mxq_mask_minabs");
}

extern "C" int mxq_attend_hints(const double* amax_a, int64_t lda, const double* amax_k, int64_t ldk, int64_t D,
                                int64_t Z, double slack_scale, const float* minabs, int64_t z0, int64_t z_per_b,
                                int32_t batched, int64_t rows, int64_t Tk, uint8_t* skip, int32_t* k_end,
                                const float* maxval, float* tail_max, mxq_stream_t stream) {
  if (D < 0 || Z < 0 || rows < 0 || Tk < 0 || z0 < 0 || z_per_b < 1 || lda < Z || ldk < Z)
    return mxq::invalid("mxq_attend_hints: bad shape");
  if (Z == 0 || rows == 0) return MXQ_OK;
  if (!amax_a || !amax_k || !minabs || !skip || !k_end) return mxq::invalid("mxq_attend_hints: NULL pointer");
  if (tail_max && !maxval) return mxq::invalid("mxq_attend_hints: tail_max needs maxval");
  const int64_t rgroups = mxq::ceil_div(rows, 32), kgroups = mxq::ceil_div(Tk, 32), tgroups = mxq::ceil_div(rows, 64);
  if (tgroups > INT32_MAX || Z > 65535 || kgroups > INT32_MAX / 32) return mxq::invalid("mxq_attend_hints: too large");
  k_attend_hints<<<dim3((unsigned)tgroups, (unsigned)Z), 256, 0, mxq::as_stream(stream)>>>(
      amax_a, lda, amax_k, ldk, D, slack_scale, minabs, z0, z_per_b, batched ? 1 : 0, rgroups, kgroups, tgroups, skip,
      k_end, maxval, tail_max);
  return mxq::check_launch("mxq_attend_hints");
}
