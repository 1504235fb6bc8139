// MX-Gemmini look-up tables on gfx950 (mxq/lut/kmeans.py:27-152, mxq/lut/formats.py:140-159).
//
//   k_lut_hist    counts of each distinct code value per column group: the group's columns of a K-row stripe
//                 are binned into an LDS histogram (the grid bin read off a code's bits, or a binary search of
//                 the sorted grid with an exact-match check), then added into the global counts with one atomic
//                 per nonzero bin
//   k_lut_kmeans  one wavefront per group: quantile seeds (or the present values when 16 or fewer), weighted
//                 Lloyd passes in float64 until two passes agree (numpy.allclose's tolerances) or max_iters,
//                 snap to the nearest finder-safe value, pad with unused safe values smallest magnitude first,
//                 sort.  Lanes own grid bins for the assignment step; the sums are exact in float64 (counts times
//                 grid values have few significant bits), so their order does not matter
//   k_lut_pick    nearest table entry per code (ties to the lower index): int64 index, the entry's value, or
//                 4-bit indices two to a byte (the wire format: adjacent lanes hold adjacent columns and pair
//                 up through a shuffle)
//   k_lut_lookup  the entries named by int64 indices; k_lut_lookup4 by 4-bit ones
//   k_lut_finder  the chip's finder: nearest in fixed point with the format's |difference| mask, first index
#include <cmath>

#include "lut_impl.h"

using mxq_lut::kMaxGrid;
using mxq_lut::kSize;
using mxq_lut::stream_rows;
using mxq_lut::stripe_rows;

namespace {

// lower_bound in a sorted float array: the first index with a[i] >= v (NaN compares false: count of a[i] < v)
__device__ __forceinline__ int lower_bound_f(const float* a, int n, float v) {
  int lo = 0, hi = n;
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    if (a[mid] < v) lo = mid + 1;
    else hi = mid;
  }
  return lo;
}

// The nearest entry of an ascending row of `width` values to v (mxq/lut/kmeans.py:125-138): the insertion point
// `hi` of v (the count of entries below it) clamped to [1, width - 1], then lo = hi - 1 unless v is strictly
// nearer row[hi]; ties to the lower index.
__device__ __forceinline__ int nearest_entry(const float* row, int width, float v) {
  int hi = lower_bound_f(row, width, v);
  hi = hi < 1 ? 1 : (hi > width - 1 ? width - 1 : hi);
  const int lo = hi - 1;
  return (fabsf(v - row[lo]) <= fabsf(row[hi] - v)) ? lo : hi;
}

// nearest_entry for a row of kSize = 16: the count of entries below v in four fixed probes (8, 4, 2, 1 ahead
// of the count so far), no loop.
__device__ __forceinline__ int nearest16(const float* row, float v) {
  int below = 0;
#pragma unroll
  for (int step = kSize / 2; step >= 1; step >>= 1)
    if (row[below + step - 1] < v) below += step;
  const int hi = below < 1 ? 1 : (below > kSize - 1 ? kSize - 1 : below);
  return (fabsf(v - row[hi - 1]) <= fabsf(row[hi] - v)) ? hi - 1 : hi;
}

// Where a float32 value that is a code of a LUT format sits in the format's value grid (mxq_lut::CodeGrid's
// order): the code's bits read off the value (normal values by their exponent and mantissa fields, subnormal
// ones as multiples of the smallest step).  A value that is no code of the format gets -1.  ok == 0: the grid
// is not a LUT format's (the callers search it instead).  Built on the host by grid_index_of.
struct GridIndex {
  int ok;
  int m, nneg;
  uint32_t nmin, nsub, lowmask, maxbits;
  float sub_mul;
};

__device__ __forceinline__ int grid_index(float v, const GridIndex& g) {
  const uint32_t u = f2u(v), a = u & 0x7FFFFFFFu;
  int c;
  bool good;
  if (a >= g.nmin) {
    c = (int)((a >> (23 - g.m)) - g.nsub);
    good = (a & g.lowmask) == 0u && a <= g.maxbits;
  } else {
    const float t = u2f(a) * g.sub_mul;
    c = (int)t;
    good = (float)c == t;
  }
  return good ? g.nneg + ((u >> 31) ? -c : c) : -1;
}

// A group's slot in a block's per-group LDS arrays: the even groups first, then the odd ones, so the two groups
// of a lane's four columns (group 1) land half an array apart and a wave's 64 lanes spread over the banks.
__device__ __forceinline__ int group_slot(int gl, int half) { return (gl & 1) * half + (gl >> 1); }

// blockDim = 256; CB columns per block, 256 / CB row lanes per column; rows [k0, k0 + rows_per_block).
// INDEXED: a code's bin is read off its bits (grid_index); otherwise found by binary search in the grid.  A
// value is counted only when it equals a grid value (-0 counts as the 0 bin, as == says); anything else sets
// the error flag.
template <int VEC, bool INDEXED>
__global__ void __launch_bounds__(256) k_lut_hist(const float* __restrict__ P, int64_t K, int64_t n, int group,
                                                  const float* __restrict__ grid, int nv, GridIndex gi, int CB,
                                                  int64_t rows_per_block, int* __restrict__ counts,
                                                  int* __restrict__ err) {
  extern __shared__ int hist[];                      // per group slot nv counts (2 * half slots)
  __shared__ float g_s[kMaxGrid];
  const int64_t c0 = (int64_t)blockIdx.x * CB;
  const int64_t k0 = (int64_t)blockIdx.y * rows_per_block;
  const int gpb = (CB >> group) > 0 ? (CB >> group) : 1;
  const int half = (gpb + 1) / 2;
  for (int i = threadIdx.x; i < 2 * half * nv; i += blockDim.x) hist[i] = 0;
  if constexpr (!INDEXED)
    for (int i = threadIdx.x; i < nv; i += blockDim.x) g_s[i] = grid[i];
  __syncthreads();
  // a lane bins VEC adjacent columns (one VEC-wide load per row); CB / VEC lanes span the block's columns and
  // the 256 / (CB / VEC) row lanes split its rows
  const int lanes_x = CB / VEC;
  const int col = (threadIdx.x % lanes_x) * VEC, rl = threadIdx.x / lanes_x, nrl = blockDim.x / lanes_x;
  const int64_t j = c0 + col;
  const int64_t g0 = c0 >> group;
  bool bad = false;
  if (j < n) {
    int* h[VEC];
#pragma unroll
    for (int e = 0; e < VEC; ++e) h[e] = hist + group_slot((int)(((j + e < n ? j + e : j) >> group) - g0), half) * nv;
    const int64_t kend = (k0 + rows_per_block < K) ? k0 + rows_per_block : K;
    const int64_t kfirst = k0 + rl;                    // this lane's rows: kfirst, kfirst + nrl, ... < kend
    const int64_t rows = kfirst < kend ? (kend - kfirst + nrl - 1) / nrl : 0;
    const float* src = P + kfirst * n + j;
    const int64_t rstep = (int64_t)nrl * n;
    constexpr int U = VEC == 4 ? 8 : 16;               // rows per batch
    using Buf = float[U][VEC];
    auto load = [&](Buf& v, int64_t batch, int count) {
      const float* p = src + batch * U * rstep;
#pragma unroll
      for (int t = 0; t < U; ++t) {
        if constexpr (VEC == 4) {
          float4 q = make_float4(0.f, 0.f, 0.f, 0.f);
          if (t < count) q = *reinterpret_cast<const float4*>(p + t * rstep);
          v[t][0] = q.x; v[t][1] = q.y; v[t][2] = q.z; v[t][3] = q.w;
        } else {
          v[t][0] = t < count ? p[t * rstep] : 0.0f;
        }
      }
    };
    auto bin = [&](const Buf& v, int64_t, int count) {
#pragma unroll
      for (int t = 0; t < U; ++t) {
        if (t >= count) break;
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
          int b;
          if constexpr (INDEXED) {
            b = grid_index(v[t][e], gi);
          } else {
            b = lower_bound_f(g_s, nv, v[t][e]);
            if (b >= nv || !(g_s[b] == v[t][e])) b = -1;
          }
          if (b < 0) bad = true;
          else atomicAdd(&h[e][b], 1);
        }
      }
    };
    stream_rows<U, Buf>(rows, load, bin);
  }
  if (bad) atomicOr(err, 1);
  __syncthreads();
  const int64_t ng = (n + (1 << group) - 1) >> group;
  for (int i = threadIdx.x; i < gpb * nv; i += blockDim.x) {
    const int c = hist[group_slot(i / nv, half) * nv + i % nv];
    const int64_t g = g0 + i / nv;
    if (c && g < ng) atomicAdd(&counts[g * nv + (i % nv)], c);
  }
}

// The 16 values held by lanes 0..15 sorted ascending across those lanes (bitonic network), equal values kept
// in lane order, as a stable sort leaves them.  Lanes 16..63 take part in
// their own 16-lane groups and are ignored.
__device__ __forceinline__ double sort16_lanes(double v, int lane) {
  int idx = lane;
#pragma unroll
  for (int k = 2; k <= kSize; k <<= 1) {
#pragma unroll
    for (int j = k >> 1; j > 0; j >>= 1) {
      const double pv = __shfl_xor(v, j, 64);
      const int pi = __shfl_xor(idx, j, 64);
      const bool up = (lane & k) == 0;                     // this pair sorts ascending
      const bool lower = (lane & j) == 0;                  // this lane is the pair's lower position
      const bool p_first = pv < v || (pv == v && pi < idx);
      // the lower position of an ascending pair takes the first of the two; the upper takes the second
      const bool take = (lower == up) ? p_first : !p_first;
      if (take) {
        v = pv;
        idx = pi;
      }
    }
  }
  return v;
}

__device__ __forceinline__ bool is_finite_d(double x) { return (d2u(x) & 0x7FF0000000000000ull) != 0x7FF0000000000000ull; }

// Wave-wide helpers for the table kernel (one 64-lane wavefront per table).
// Number of lanes below this one whose flag is set.
__device__ __forceinline__ int lanes_below(bool flag, int lane) {
  const unsigned long long m = __ballot(flag);
  return __popcll(m & ((1ull << lane) - 1ull));
}
// Inclusive prefix sum of one double per lane (exact here: integer counts).
__device__ __forceinline__ double wave_scan(double v, int lane) {
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const double u = __shfl_up(v, off, 64);
    if (lane >= off) v += u;
  }
  return v;
}

// One 64-lane workgroup per table; lane i handles grid bins i, i + 64, ... (nv <= 256: four rounds).
//   seeds   the present values when 16 or fewer (in grid order); else the quantile seeds: bin cdf =
//           cumsum(counts) / total (exact integer prefix sums, the same float64 division per bin), seed i the
//           first bin whose cdf reaches (i + 0.5) / 16, found with ballots; then a sort, duplicate
//           removal and sort, across lanes 0..15
//   Lloyd   lanes own bins for the nearest-centre step (first minimum), float64 LDS sums (exact, so their
//           order does not matter), lane c < 16 updates centre c, the same dedupe, allclose by wave vote
//   snap    lane c < 16: the nearest safe value to centre c (first minimum); the distinct ones are the table's
//           members; the unused safe values in safe_order order fill it to 16 (ranks by ballot); the members
//           are written in ascending order, +Inf past them
//   code map (when not NULL) per element code c of the format: the bits of the table entry pick chooses for
//           the code's value (NaN for a code with no grid bin), at code_map[g * ncodes + c]
// The counts of group g are summed from src (mxq_lut::CountSource): every split's units of the group.
__global__ void __launch_bounds__(64) k_lut_kmeans(mxq_lut::CountSource src, int nv, const float* __restrict__ grid,
                                                   const float* __restrict__ safe, int ns,
                                                   const int* __restrict__ safe_order, int max_iters,
                                                   float* __restrict__ T, uint32_t* __restrict__ code_map,
                                                   mxq_lut::CodeGrid cg, int exact) {
  constexpr int kRounds = kMaxGrid / 64;
  __shared__ double x_s[kMaxGrid];
  __shared__ double w_s[kMaxGrid];
  __shared__ double C[kSize];
  __shared__ double sums[kSize], wsum[kSize];
  __shared__ double pw[kMaxGrid], pwx[kMaxGrid];     // inclusive prefix sums of the counts and counts x values
  __shared__ int lo_s[kSize], hi_s[kSize];           // a pass's cluster ranges of bins (lo -1: empty)
  __shared__ int lab_s[kMaxGrid];                    // a pass's cluster of each bin (sums not exact)
  __shared__ float safe_s[kMaxGrid];
  __shared__ int order_s[kMaxGrid];
  __shared__ unsigned char member[kMaxGrid];
  __shared__ float T_s[kSize];
  const int g = blockIdx.x, lane = threadIdx.x;
  // rounds of 64 lanes over the grid's bins and over the safe values (a loop over them stops at these)
  const int nr = (nv + 63) >> 6, nsr = (ns + 63) >> 6;
  const int64_t u0 = (int64_t)g << src.shift;
  const int64_t u1 = ((int64_t)(g + 1) << src.shift) < src.nunits ? ((int64_t)(g + 1) << src.shift) : src.nunits;
  // every load in flight before the stores into LDS: grid, safe values and order, and each bin's count, the
  // sum over every split and owned unit, eight loads at a time
  float gv[kRounds], sv[kRounds];
  int ov[kRounds];
  int64_t cv[kRounds];
  const int64_t nu = u1 - u0, terms = (int64_t)src.nsplit * nu;
#pragma unroll
  for (int r = 0; r < kRounds; ++r) {
    const int i = r * 64 + lane;
    gv[r] = i < nv ? grid[i] : 0.0f;
    sv[r] = i < ns ? safe[i] : 0.0f;
    ov[r] = i < ns ? safe_order[i] : 0;
  }
#pragma unroll
  for (int r = 0; r < kRounds; ++r) {
    const int i = r * 64 + lane;
    cv[r] = 0;
    if (r >= nr) break;
    for (int64_t t0 = 0; t0 < terms; t0 += 8) {
      int v[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const int64_t t = t0 + k;
        const int64_t sp = t / nu, u = u0 + (t - sp * nu);
        v[k] = (t < terms && i < nv) ? src.p[sp * src.split_stride + u * nv + i] : 0;
      }
#pragma unroll
      for (int k = 0; k < 8; ++k) cv[r] += v[k];
    }
  }
#pragma unroll
  for (int r = 0; r < kRounds; ++r) {
    const int i = r * 64 + lane;
    if (i < nv) {
      x_s[i] = (double)gv[r];
      w_s[i] = (double)cv[r];
    }
    if (i < ns) {
      safe_s[i] = sv[r];
      order_s[i] = ov[r];
      member[i] = 0;
    }
  }
  __syncthreads();

  // ---- seeds
  int npres = 0;
#pragma unroll
  for (int r = 0; r < kRounds; ++r) {
    if (r >= nr) break;
    const int i = r * 64 + lane;
    npres += __popcll(__ballot(i < nv && w_s[i] > 0.0));
  }
  double cen = d_inf();                                // lane c < 16: centre c
  bool stop;
  if (npres <= kSize) {
    int base = 0;
#pragma unroll
    for (int r = 0; r < kRounds; ++r) {
      if (r >= nr) break;
      const int i = r * 64 + lane;
      const bool pres = i < nv && w_s[i] > 0.0;
      const int rank = base + lanes_below(pres, lane);
      if (pres) C[rank] = x_s[i];
      base += __popcll(__ballot(pres));
    }
    if (lane >= npres && lane < kSize) C[lane] = d_inf();
    __syncthreads();
    if (lane < kSize) cen = C[lane];
    stop = true;
  } else {
    double cum[kRounds];
    double carry = 0.0;
#pragma unroll
    for (int r = 0; r < kRounds; ++r) {
      if (r >= nr) break;
      const int i = r * 64 + lane;
      const double incl = wave_scan(i < nv ? w_s[i] : 0.0, lane) + carry;
      cum[r] = incl;
      carry = __shfl(incl, 63, 64);
    }
    const double total = carry;
    double carry_x = 0.0;
#pragma unroll
    for (int r = 0; r < kRounds; ++r) {
      if (r >= nr) break;
      const int i = r * 64 + lane;
      const double incl = wave_scan(i < nv ? w_s[i] * x_s[i] : 0.0, lane) + carry_x;
      if (i < nv) {
        pw[i] = cum[r];
        pwx[i] = incl;
      }
      carry_x = __shfl(incl, 63, 64);
    }
    double cdf[kRounds];
#pragma unroll
    for (int r = 0; r < kRounds; ++r) cdf[r] = r < nr ? cum[r] / total : 0.0;
    // seed q is the first bin whose cdf reaches (q + 0.5) / 16.  The cdf never decreases along the bins, so
    // with k = the number of probes a bin's cdf reaches, seed q's bin is the number of bins with k <= q (nv:
    // none reaches it, the last bin then).  The seeds come out ascending, so the reference's sort is the
    // identity and its dedupe-and-sort keeps the distinct ones in order, +Inf after them.
    int kreach[kRounds];
#pragma unroll
    for (int r = 0; r < kRounds; ++r) {
      kreach[r] = 0;
#pragma unroll
      for (int q = 0; q < kSize; ++q) kreach[r] += cdf[r] >= (double)(2 * q + 1) * 0.03125 ? 1 : 0;  // (q+.5)/16
    }
    int seed_bin = nv;                                 // lane q < 16: seed q's bin
#pragma unroll
    for (int q = 0; q < kSize; ++q) {
      int below_q = 0;
#pragma unroll
      for (int r = 0; r < kRounds; ++r) {
        if (r >= nr) break;
        below_q += __popcll(__ballot(r * 64 + lane < nv && kreach[r] <= q));
      }
      if (lane == q) seed_bin = below_q;
    }
    cen = d_inf();
    if (lane < kSize) cen = x_s[seed_bin < nv ? seed_bin : nv - 1];
    const double below = __shfl_up(cen, 1, 64);
    const bool keep = lane < kSize && (lane == 0 || cen != below);
    const int rank = lanes_below(keep, lane);
    if (lane < kSize) C[lane] = d_inf();
    __syncthreads();
    if (keep) C[rank] = cen;
    stop = max_iters <= 0;
  }
  __syncthreads();

  // ---- Lloyd passes
  // A pass assigns each bin its nearest centre (first minimum).  The centres are ascending and the bins too, so
  // the assignment is non-decreasing along the bins and every cluster is a run of bins: its sums are then
  // differences of the prefix sums (exact while sums_exact holds).  A pass whose assignment is not monotone
  // (rounding at a near-tie could make one) adds its bins into the sums by LDS atomics instead; groups whose
  // sums may round add each cluster's bins in bin order, a lane a cluster, as the reference does.  The new
  // centres are sorted and deduplicated only when they need it (a stable sort of ascending, distinct values
  // is the identity).
  for (int it = 0; it < max_iters && !stop; ++it) {
    double cen_r[kSize];
#pragma unroll
    for (int c = 0; c < kSize; ++c) cen_r[c] = C[c];
    int best[kRounds];
#pragma unroll
    for (int r = 0; r < kRounds; ++r) best[r] = kSize;  // past the bins: above every cluster
    bool mono = true;
#pragma unroll
    for (int r = 0; r < kRounds; ++r) {
      if (r >= nr) break;
      const int i = r * 64 + lane;
      if (i < nv) {
        // the first minimum of the 16 distances as a tree: the later of a pair wins only when strictly
        // nearer, which is the linear scan's choice (distances are never NaN: the values are finite)
        const double xv = x_s[i];
        double d[kSize];
        int bi[kSize];
#pragma unroll
        for (int c = 0; c < kSize; ++c) {
          d[c] = fabs(xv - cen_r[c]);
          bi[c] = c;
        }
#pragma unroll
        for (int step = 1; step < kSize; step <<= 1)
#pragma unroll
          for (int c = 0; c < kSize; c += 2 * step)
            if (d[c + step] < d[c]) {
              d[c] = d[c + step];
              bi[c] = bi[c + step];
            }
        best[r] = bi[0];
      }
      // every lane takes part in each exchange (a lane a shuffle reads from must be active)
      const int up = __shfl_up(best[r], 1, 64);
      const int last = r > 0 ? __shfl(best[r > 0 ? r - 1 : 0], 63, 64) : -1;
      const int prev = lane > 0 ? up : last;
      mono = mono && best[r] >= prev;
    }
    if (lane < kSize) { lo_s[lane] = -1; hi_s[lane] = -1; sums[lane] = 0.0; wsum[lane] = 0.0; }
    __syncthreads();
    const bool all_runs = __all(mono);
    const bool runs = exact && all_runs;
    if (!exact) {
#pragma unroll
      for (int r = 0; r < kRounds; ++r) {
        const int i = r * 64 + lane;
        if (r < nr && i < nv) lab_s[i] = best[r];
      }
    } else if (runs) {
#pragma unroll
      for (int r = 0; r < kRounds; ++r) {
        if (r >= nr) break;
        const int i = r * 64 + lane;
        const int up = __shfl_up(best[r], 1, 64), dn = __shfl_down(best[r], 1, 64);
        const int last = r > 0 ? __shfl(best[r > 0 ? r - 1 : 0], 63, 64) : -1;
        const int first = r + 1 < nr ? __shfl(best[r + 1 < kRounds ? r + 1 : r], 0, 64) : kSize;
        const int prev = lane > 0 ? up : last;
        const int next = lane < 63 ? dn : first;
        if (i < nv && best[r] != prev) lo_s[best[r]] = i;
        if (i < nv && best[r] != next) hi_s[best[r]] = i;
      }
    } else {
#pragma unroll
      for (int r = 0; r < kRounds; ++r) {
        if (r >= nr) break;
        const int i = r * 64 + lane;
        if (i < nv && w_s[i] != 0.0) {
          atomicAdd(&sums[best[r]], w_s[i] * x_s[i]);
          atomicAdd(&wsum[best[r]], w_s[i]);
        }
      }
    }
    __syncthreads();
    // lane c < 16: the new centre c (the old one when its cluster is empty), the dedupe, allclose by vote
    double cn = d_inf();
    if (lane < kSize) {
      double sw = wsum[lane], swx = sums[lane];
      if (runs) {
        const int lo = lo_s[lane], hi = hi_s[lane];
        sw = lo < 0 ? 0.0 : pw[hi] - (lo > 0 ? pw[lo - 1] : 0.0);
        swx = lo < 0 ? 0.0 : pwx[hi] - (lo > 0 ? pwx[lo - 1] : 0.0);
      } else if (!exact) {
        // the reference's scatter_add order: the cluster's bins one by one, in bin order
        sw = 0.0;
        swx = 0.0;
        for (int i = 0; i < nv; ++i)
          if (lab_s[i] == lane) {
            sw += w_s[i];
            swx += w_s[i] * x_s[i];
          }
      }
      cn = (sw > 0.0) ? swx / sw : C[lane];
    }
    const double below0 = __shfl_up(cn, 1, 64);
    const bool in_order = lane == 0 || lane >= kSize || below0 < cn || (below0 == cn && cn == d_inf());
    if (!__all(in_order)) {
      cn = sort16_lanes(cn, lane);
      const double below = __shfl_up(cn, 1, 64);
      if (lane > 0 && lane < kSize && cn == below) cn = d_inf();
      cn = sort16_lanes(cn, lane);
    }
    bool same = true;
    if (lane < kSize) {
      const double old_c = C[lane];
      const bool valid = is_finite_d(old_c);
      if (is_finite_d(cn) != valid) same = false;
      if (valid && !(fabs(cn - old_c) <= 1e-8 + 1e-5 * fabs(old_c))) same = false;
    }
    stop = __all(same);
    __syncthreads();                                   // every lane has read C
    if (!stop && lane < kSize) C[lane] = cn;
    __syncthreads();
  }

  // ---- snap to the safe values, pad, write in ascending order
  if (lane < kSize) {
    const double c = C[lane];
    if (is_finite_d(c)) {
      // the first nearest safe value: a neighbour of c's insertion point, the lower on a tie (the safe values
      // lie at least a grid step apart, far above the distances' rounding, so no farther value ties)
      int lo = 0, hi = ns;
      while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if ((double)safe_s[mid] < c) lo = mid + 1;
        else hi = mid;
      }
      int best = lo;
      if (lo == ns) best = ns - 1;
      else if (lo > 0 && !(fabs(c - (double)safe_s[lo]) < fabs(c - (double)safe_s[lo - 1]))) best = lo - 1;
      member[best] = 1;
    }
  }
  __syncthreads();
  int cnt = 0;
#pragma unroll
  for (int r = 0; r < kRounds; ++r) {
    if (r >= nsr) break;
    const int i = r * 64 + lane;
    cnt += __popcll(__ballot(i < ns && member[i]));
  }
  int need = kSize - cnt;
  // unused safe values in safe_order order, the first `need` of them
  bool take[kRounds];
  int base = 0;
#pragma unroll
  for (int r = 0; r < kRounds; ++r) {
    take[r] = false;
    if (r >= nsr) continue;
    const int q = r * 64 + lane;
    const bool unused = q < ns && !member[order_s[q]];
    take[r] = unused && base + lanes_below(unused, lane) < need;
    base += __popcll(__ballot(unused));
  }
  __syncthreads();                                     // every lane has read member
#pragma unroll
  for (int r = 0; r < kRounds; ++r) {
    const int q = r * 64 + lane;
    if (take[r]) member[order_s[q]] = 1;
  }
  __syncthreads();
  base = 0;
#pragma unroll
  for (int r = 0; r < kRounds; ++r) {
    if (r >= nsr) break;
    const int i = r * 64 + lane;
    const bool mem = i < ns && member[i];
    const int rank = base + lanes_below(mem, lane);
    if (mem && rank < kSize) {
      T[(int64_t)g * kSize + rank] = safe_s[i];
      T_s[rank] = safe_s[i];
    }
    base += __popcll(__ballot(mem));
  }
  if (lane >= base && lane < kSize) {
    T[(int64_t)g * kSize + lane] = f_inf();
    T_s[lane] = f_inf();
  }
  if (!code_map) return;
  __syncthreads();
  const int ncodes = 2 << cg.sign_at;
  for (int c = lane; c < ncodes; c += 64) {
    const int b = mxq_lut::code_bin((uint32_t)c, cg);
    code_map[(int64_t)g * ncodes + c] = b >= 0 ? f2u(T_s[nearest16(T_s, (float)x_s[b])]) : 0x7FC00000u;
  }
}

// Nearest entry of each code's group table (ascending; ties to the lower index): int64 index to I, the entry's
// value to Pout, or I4: row k's byte j / 2 holds column j's index in its low nibble (j even) and column
// j + 1's in its high one (0 past n).  Exactly one of I, Pout, I4 is set.  W16: tables of kSize entries
// (nearest16); otherwise `width` entries, searched.
template <int VEC, bool W16>
__global__ void __launch_bounds__(256) k_lut_pick(const float* __restrict__ P, int64_t K, int64_t n, int group,
                                                  const float* __restrict__ T, int width, int64_t rows_per_block,
                                                  int64_t* __restrict__ I, float* __restrict__ Pout,
                                                  uint8_t* __restrict__ I4) {
  // (256 >> group, at least 1) rows of the block's tables, each `width` values and one float of padding (rows
  // an odd number of words apart: the lanes' searches in different rows fall in different LDS banks)
  extern __shared__ float rows_s[];
  const int stride = width + 1;
  const int64_t c0 = (int64_t)blockIdx.x * 256;
  const int64_t g0 = c0 >> group;
  const int64_t ng = (n + (1 << group) - 1) >> group;
  const int gpb = (256 >> group) > 0 ? (256 >> group) : 1;
  // the block's tables are T[g0 * width, + gpb * width): eight loads in flight per thread before their stores
  {
    const int total = gpb * width;
    const int64_t avail = (ng - g0) * width;
    for (int base = 0; base < total; base += 256 * 8) {
      float w[8];
#pragma unroll
      for (int f = 0; f < 8; ++f) {
        const int i = base + f * 256 + (int)threadIdx.x;
        w[f] = (i < total && i < avail) ? T[g0 * width + i] : 0.0f;
      }
#pragma unroll
      for (int f = 0; f < 8; ++f) {
        const int i = base + f * 256 + (int)threadIdx.x;
        if (i < total) rows_s[(i / width) * stride + i % width] = w[f];
      }
    }
  }
  __syncthreads();
  auto nearest = [&](const float* row, float v) { return W16 ? nearest16(row, v) : nearest_entry(row, width, v); };
  const int64_t k0 = (int64_t)blockIdx.y * rows_per_block;
  const int64_t kend = (k0 + rows_per_block < K) ? k0 + rows_per_block : K;
  if constexpr (VEC == 4) {
    // four adjacent columns per lane (16-byte loads and stores), 64 lanes across the block's 256 columns, four
    // row lanes; n % 4 == 0, so a lane's columns are all inside the tensor or all past it
    const int64_t j = c0 + (threadIdx.x & 63) * 4;
    if (j >= n) return;
    const int rl = threadIdx.x >> 6;
    const float* row[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) row[e] = rows_s + (int)(((j + e) >> group) - g0) * stride;
    // this wave's rows: kfirst, kfirst + 4, ... < kend
    const int64_t kfirst = k0 + rl;
    const int64_t rows = kfirst < kend ? (kend - kfirst + 3) / 4 : 0;
    const int64_t rstep = 4 * n;
    const int64_t at0 = kfirst * n + j;
    constexpr int U = 4;
    using Buf = float4[U];
    auto load = [&](Buf& v, int64_t batch, int count) {
      const float* p = P + at0 + batch * U * rstep;
#pragma unroll
      for (int t = 0; t < U; ++t)
        v[t] = t < count ? *reinterpret_cast<const float4*>(p + t * rstep) : make_float4(0.f, 0.f, 0.f, 0.f);
    };
    auto use = [&](const Buf& v, int64_t batch, int count) {
#pragma unroll
      for (int t = 0; t < U; ++t) {
        if (t >= count) break;
        const int64_t at = at0 + (batch * U + t) * rstep;
        const int p0 = nearest(row[0], v[t].x), p1 = nearest(row[1], v[t].y), p2 = nearest(row[2], v[t].z),
                  p3 = nearest(row[3], v[t].w);
        if (I) {
          *reinterpret_cast<longlong2*>(I + at) = make_longlong2(p0, p1);
          *reinterpret_cast<longlong2*>(I + at + 2) = make_longlong2(p2, p3);
        } else {
          *reinterpret_cast<float4*>(Pout + at) = make_float4(row[0][p0], row[1][p1], row[2][p2], row[3][p3]);
        }
      }
    };
    stream_rows<U, Buf>(rows, load, use);
    return;
  }
  const int64_t j = c0 + threadIdx.x;
  const bool live = j < n;
  if (!live && !I4) return;                          // the nibble output keeps every lane for its shuffle
  const int64_t jj = live ? j : n - 1;               // a column of this block (c0 < n)
  const float* row = rows_s + (int)((jj >> group) - g0) * stride;
  const int64_t nbytes = (n + 1) >> 1;
  constexpr int U = 8;
  using Buf = float[U];
  auto load = [&](Buf& v, int64_t batch, int count) {
    const float* p = P + (k0 + batch * U) * n + jj;
#pragma unroll
    for (int t = 0; t < U; ++t) v[t] = t < count ? p[t * n] : 0.0f;
  };
  auto use = [&](const Buf& v, int64_t batch, int count) {
#pragma unroll
    for (int t = 0; t < U; ++t) {
      if (t >= count) break;
      const int64_t k = k0 + batch * U + t;
      const int pick = nearest(row, v[t]);
      if (I4) {                                       // count is the block's: all lanes shuffle
        const int next = __shfl_xor(pick, 1, 64);
        if (live && (j & 1) == 0) I4[k * nbytes + (j >> 1)] = (uint8_t)(pick | ((j + 1 < n ? next : 0) << 4));
      } else if (I) {
        I[k * n + j] = pick;
      } else {
        Pout[k * n + j] = row[pick];
      }
    }
  };
  stream_rows<U, Buf>(kend - k0, load, use);
}

__global__ void __launch_bounds__(256) k_lut_lookup(const int64_t* __restrict__ I, int64_t K, int64_t n, int group,
                                                    const float* __restrict__ T, int width, float* __restrict__ out) {
  const int64_t total = K * n;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total; e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t j = e % n;
    out[e] = T[(j >> group) * width + I[e]];
  }
}

__global__ void __launch_bounds__(256) k_lut_lookup4(const uint8_t* __restrict__ I4, int64_t K, int64_t n,
                                                     int group, const float* __restrict__ T, int width,
                                                     float* __restrict__ out) {
  const int64_t total = K * n, nbytes = (n + 1) >> 1;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total; e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t k = e / n, j = e - k * n;
    const int idx = (I4[k * nbytes + (j >> 1)] >> ((j & 1) * 4)) & 0xF;
    out[e] = T[(j >> group) * width + idx];
  }
}

__global__ void __launch_bounds__(256) k_lut_finder(const int64_t* __restrict__ codes, int64_t K, int64_t n, int group,
                                                    const int64_t* __restrict__ fx_all, int ncodes,
                                                    const int64_t* __restrict__ lut_fx, int64_t mask,
                                                    int64_t* __restrict__ out) {
  __shared__ int64_t fx_s[kMaxGrid];
  for (int i = threadIdx.x; i < ncodes; i += blockDim.x) fx_s[i] = fx_all[i];
  __syncthreads();
  const int64_t total = K * n;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total; e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t j = e % n;
    const int64_t f = fx_s[codes[e]];
    const int64_t* lf = lut_fx + (j >> group) * kSize;
    int best = 0;
    int64_t bd = f - lf[0];
    bd = bd < 0 ? -bd : bd;
    if (mask) bd &= mask;
    for (int i = 1; i < kSize; ++i) {
      int64_t d = f - lf[i];
      d = d < 0 ? -d : d;
      if (mask) d &= mask;
      if (d < bd) { bd = d; best = i; }
    }
    out[e] = best;
  }
}

__global__ void k_fill_i32(int* p, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) p[i] = 0;
}

// The grid index of a LUT format (e, m) whose grid has nv values: ok == 0 unless nv is what the format gives.
GridIndex grid_index_of(int e, int m, int nv) {
  GridIndex g{};
  const mxq_lut::CodeGrid cg = mxq_lut::code_grid_of(e, m, nv);
  if (!cg.ok) return g;
  const int bias = (1 << (e - 1)) - 1, emin = 1 - bias;
  const int ex = cg.cmax >> m, man = cg.cmax & ((1 << m) - 1);
  g.maxbits = ((uint32_t)(ex - bias + 127) << 23) | ((uint32_t)man << (23 - m));
  g.nmin = (uint32_t)(emin + 127) << 23;
  g.nsub = (uint32_t)(127 - bias) << m;
  g.lowmask = (1u << (23 - m)) - 1u;
  g.sub_mul = std::ldexp(1.0f, m - emin);
  g.m = m;
  g.nneg = cg.cmax;
  g.ok = 1;
  return g;
}

int launch_pick(const float* P, int64_t K, int64_t n, int group, const float* T, int width, int64_t* I,
                float* P_lut, uint8_t* I4, bool vec4, hipStream_t st) {
  const int gpb = (256 >> group) > 0 ? (256 >> group) : 1;
  const size_t lds = (size_t)gpb * (width + 1) * sizeof(float);
  if (lds > 65536) return mxq::invalid("mxq_lut_pick: tables too wide");
  const int64_t col_blocks = mxq::ceil_div(n, 256);
  const int64_t rpb = stripe_rows(K, col_blocks, 1024);           // about four blocks per CU
  const dim3 grid((unsigned)col_blocks, (unsigned)mxq::ceil_div(K, rpb));
  const bool w16 = width == kSize;
  if (vec4 && w16) k_lut_pick<4, true><<<grid, 256, lds, st>>>(P, K, n, group, T, width, rpb, I, P_lut, I4);
  else if (vec4) k_lut_pick<4, false><<<grid, 256, lds, st>>>(P, K, n, group, T, width, rpb, I, P_lut, I4);
  else if (w16) k_lut_pick<1, true><<<grid, 256, lds, st>>>(P, K, n, group, T, width, rpb, I, P_lut, I4);
  else k_lut_pick<1, false><<<grid, 256, lds, st>>>(P, K, n, group, T, width, rpb, I, P_lut, I4);
  return MXQ_OK;
}

}  // namespace

namespace mxq_lut {

int launch_kmeans(const CountSource& src, int64_t ng, int nv, const float* grid, const float* safe, int ns,
                  const int* safe_order, int max_iters, float* T, uint32_t* code_map, const CodeGrid& cg,
                  bool exact_sums, hipStream_t st) {
  if (code_map && !cg.ok) return mxq::invalid("k-means: a code map needs the format's code grid");
  mxq::KernelTimer timer("lut_kmeans", st);
  k_lut_kmeans<<<dim3((unsigned)ng), 64, 0, st>>>(src, nv, grid, safe, ns, safe_order, max_iters, T, code_map, cg,
                                                  exact_sums ? 1 : 0);
  return mxq::check_launch("mxq_lut k-means");
}

}  // namespace mxq_lut

extern "C" int mxq_lut_tables(const float* P, int64_t K, int64_t n, int32_t group, int32_t max_iters,
                              const float* grid, int32_t nv, const float* safe, int32_t ns, const int32_t* safe_order,
                              int32_t fmt_e, int32_t fmt_m, float* T, int32_t* workspace, mxq_stream_t stream) {
  if (K < 0 || n < 0 || group < 0 || group > 30 || max_iters < 0) return mxq::invalid("mxq_lut_tables: bad arguments");
  if (nv < 1 || nv > kMaxGrid || ns < 1 || ns > kMaxGrid) return mxq::invalid("mxq_lut_tables: bad grid sizes");
  if (n == 0) return MXQ_OK;
  const GridIndex gi = grid_index_of(fmt_e, fmt_m, nv);
  const int64_t ng = (n + (int64_t(1) << group) - 1) >> group;
  hipStream_t st = mxq::as_stream(stream);
  int* counts = workspace;                              // ng * nv, then one error flag
  int* err = workspace + ng * nv;
  {
    int64_t nz = ng * nv + 1, blocks = mxq::ceil_div(nz, 256);
    k_fill_i32<<<dim3((unsigned)(blocks < 4096 ? blocks : 4096)), 256, 0, st>>>(workspace, nz);
  }
  if (K > 0) {
    // columns per block: the LDS histogram (group slots x nv ints) within 64 KiB
    auto slots = [&](int cb) { const int gpb = (cb >> group) > 0 ? (cb >> group) : 1; return (int64_t)(gpb + 1) / 2 * 2; };
    int CB = 256;
    while (CB > 1 && slots(CB) * nv * 4 > 65536) CB >>= 1;
    const int64_t col_blocks = mxq::ceil_div(n, CB);
    // about three blocks per CU (as many as their LDS lets a CU hold), each thread binning a long stripe with
    // many loads in flight; every block then adds its histogram into the global counts, one atomic per
    // nonzero bin
    const int64_t rpb = stripe_rows(K, col_blocks, 768);
    const dim3 hgrid((unsigned)col_blocks, (unsigned)mxq::ceil_div(K, rpb));
    const size_t lds = (size_t)(slots(CB) * nv * sizeof(int));
    // four adjacent columns per lane (16-byte loads) when rows are 16-byte aligned and the block spans 4 lanes
    const bool vec4 = n % 4 == 0 && reinterpret_cast<uintptr_t>(P) % 16 == 0 && CB >= 4 && 256 % (CB / 4) == 0;
    if (vec4 && gi.ok) k_lut_hist<4, true><<<hgrid, 256, lds, st>>>(P, K, n, group, grid, nv, gi, CB, rpb, counts, err);
    else if (vec4) k_lut_hist<4, false><<<hgrid, 256, lds, st>>>(P, K, n, group, grid, nv, gi, CB, rpb, counts, err);
    else if (gi.ok) k_lut_hist<1, true><<<hgrid, 256, lds, st>>>(P, K, n, group, grid, nv, gi, CB, rpb, counts, err);
    else k_lut_hist<1, false><<<hgrid, 256, lds, st>>>(P, K, n, group, grid, nv, gi, CB, rpb, counts, err);
    if (int rc = mxq::check_launch("mxq_lut_tables histogram")) return rc;
  }
  const mxq_lut::CountSource src{counts, 1, 0, ng, 0};
  const int64_t per_group = K * ((int64_t(1) << group) < n ? (int64_t(1) << group) : n);
  return mxq_lut::launch_kmeans(src, ng, nv, grid, safe, ns, safe_order, max_iters, T, nullptr, mxq_lut::CodeGrid{},
                                mxq_lut::sums_exact(per_group, fmt_e, fmt_m), st);
}

extern "C" int mxq_lut_pick(const float* P, int64_t K, int64_t n, int32_t group, const float* T, int32_t width,
                            int64_t* I, float* P_lut, mxq_stream_t stream) {
  if (K < 0 || n < 0 || group < 0 || group > 30 || width < 2 || width > 4096) return mxq::invalid("mxq_lut_pick: bad arguments");
  if ((I == nullptr) == (P_lut == nullptr)) return mxq::invalid("mxq_lut_pick: exactly one of I and P_lut");
  if (K == 0 || n == 0) return MXQ_OK;
  const uintptr_t out_addr = I ? reinterpret_cast<uintptr_t>(I) : reinterpret_cast<uintptr_t>(P_lut);
  const bool vec4 = n % 4 == 0 && (reinterpret_cast<uintptr_t>(P) | out_addr) % 16 == 0;
  if (int rc = launch_pick(P, K, n, group, T, width, I, P_lut, nullptr, vec4, mxq::as_stream(stream))) return rc;
  return mxq::check_launch("mxq_lut_pick");
}

extern "C" int mxq_lut_pick_packed(const float* P, int64_t K, int64_t n, int32_t group, const float* T, int32_t width,
                                   uint8_t* I4, mxq_stream_t stream) {
  if (K < 0 || n < 0 || group < 0 || group > 30 || width < 2 || width > kSize)
    return mxq::invalid("mxq_lut_pick_packed: bad arguments");
  if (K == 0 || n == 0) return MXQ_OK;
  if (!P || !T || !I4) return mxq::invalid("mxq_lut_pick_packed: NULL pointer");
  if (int rc = launch_pick(P, K, n, group, T, width, nullptr, nullptr, I4, false, mxq::as_stream(stream))) return rc;
  return mxq::check_launch("mxq_lut_pick_packed");
}

extern "C" int mxq_lut_lookup_packed(const uint8_t* I4, int64_t K, int64_t n, int32_t group, const float* T,
                                     int32_t width, float* out, mxq_stream_t stream) {
  if (K < 0 || n < 0 || group < 0 || group > 30 || width < 1 || width > kSize)
    return mxq::invalid("mxq_lut_lookup_packed: bad arguments");
  if (K == 0 || n == 0) return MXQ_OK;
  if (!I4 || !T || !out) return mxq::invalid("mxq_lut_lookup_packed: NULL pointer");
  int64_t blocks = mxq::ceil_div(K * n, 256);
  if (blocks > 65536) blocks = 65536;
  k_lut_lookup4<<<dim3((unsigned)blocks), 256, 0, mxq::as_stream(stream)>>>(I4, K, n, group, T, width, out);
  return mxq::check_launch("mxq_lut_lookup_packed");
}

extern "C" int mxq_lut_lookup(const int64_t* I, int64_t K, int64_t n, int32_t group, const float* T, int32_t width,
                              float* out, mxq_stream_t stream) {
  if (K < 0 || n < 0 || group < 0 || group > 30 || width < 1) return mxq::invalid("mxq_lut_lookup: bad arguments");
  if (K == 0 || n == 0) return MXQ_OK;
  int64_t blocks = mxq::ceil_div(K * n, 256);
  if (blocks > 65536) blocks = 65536;
  k_lut_lookup<<<dim3((unsigned)blocks), 256, 0, mxq::as_stream(stream)>>>(I, K, n, group, T, width, out);
  return mxq::check_launch("mxq_lut_lookup");
}

extern "C" int mxq_lut_finder(const int64_t* codes, int64_t K, int64_t n, int32_t group, const int64_t* fx_all,
                              int32_t ncodes, const int64_t* lut_fx, int64_t mask, int64_t* out, mxq_stream_t stream) {
  if (K < 0 || n < 0 || group < 0 || group > 30 || ncodes < 1 || ncodes > kMaxGrid)
    return mxq::invalid("mxq_lut_finder: bad arguments");
  if (K == 0 || n == 0) return MXQ_OK;
  int64_t blocks = mxq::ceil_div(K * n, 256);
  if (blocks > 65536) blocks = 65536;
  k_lut_finder<<<dim3((unsigned)blocks), 256, 0, mxq::as_stream(stream)>>>(codes, K, n, group, fx_all, ncodes, lut_fx,
                                                                           mask, out);
  return mxq::check_launch("mxq_lut_finder");
}
