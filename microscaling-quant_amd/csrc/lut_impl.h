// Shared by the LUT translation units: table sizes, where a code sits in its format's value grid, and the
// k-means launch (lut.hip) that both the standalone tables and the fused LUT operand path use.
#pragma once
#include <cmath>

#include "mxq_common.h"
#include "mxq_numerics.h"

namespace mxq_lut {

constexpr int kSize = 16;            // entries per table
constexpr int kMaxGrid = 256;        // distinct finite values of the largest LUT format (E5M2: 247)

// The value grid of a LUT format (e, m) read off its codes: the grid holds the distinct finite values
// ascending, one zero, symmetric about it, so magnitude code c (sign bit at bit e + m) sits at cmax + c and
// its negative at cmax - c, where cmax is the largest finite magnitude code.  E5M2's magnitudes above 0x7B are
// Inf and NaN: no bin.  (E4M3's S.1111.111 is 480 on MX-Gemmini: a bin like the rest.)  ok == 0: the grid
// of nv values is not this format's (callers then have no code bins).
struct CodeGrid {
  int ok;
  int sign_at;       // e + m
  int cmax;
};

// Whether a group's float64 sums of count x value are exact in any order: every such sum is a multiple of the
// format's smallest step and at most per_group x its largest value in magnitude, so it is exact while that bound
// over the step stays below 2^53 (always for E4M3, E3M2 and E2M3; for E5M2 up to about 2.4 M codes a group).
// Past it, k-means adds each cluster's bins one by one in bin order, as the reference's scatter_add does.
inline bool sums_exact(int64_t per_group, int e, int m) {
  double top = 0.0;
  if (e == 4 && m == 3) top = 448.0;
  else if (e == 5 && m == 2) top = 57344.0;
  else if (e == 3 && m == 2) top = 28.0;
  else if (e == 2 && m == 3) top = 7.5;
  if (top == 0.0) return false;
  const int bias = (1 << (e - 1)) - 1;
  const double step = std::ldexp(1.0, 1 - bias - m);
  return (double)per_group * top / step < 9007199254740992.0;
}

inline CodeGrid code_grid_of(int e, int m, int nv) {
  CodeGrid g{};
  if (e < 2 || e > 5 || m < 1 || m > 3) return g;
  const int cmax = (e == 5 && m == 2) ? 0x7B : (1 << (e + m)) - 1;
  if (nv != 2 * cmax + 1) return g;
  g.ok = 1;
  g.sign_at = e + m;
  g.cmax = cmax;
  return g;
}

// The grid bin of element code c (-1: not a finite value of the format).
__device__ __forceinline__ int code_bin(uint32_t c, const CodeGrid& g) {
  const int mag = (int)(c & ((1u << g.sign_at) - 1u));
  if (mag > g.cmax) return -1;
  return (c >> g.sign_at) & 1u ? g.cmax - mag : g.cmax + mag;
}

// Where k-means reads a group's counts: nsplit partial histograms (split_stride words apart), each of nunits
// units of nv counts in grid order; group g owns units [g << shift, (g + 1) << shift) below nunits, and its
// count of bin i is the sum over every split and owned unit.  The standalone tables: one split, one unit per
// group.
struct CountSource {
  const int* p;
  int nsplit;
  int64_t split_stride;
  int64_t nunits;
  int shift;
};

// A lane's stripe of `rows` rows in batches of U: use(buf, batch, count) on each batch, whose loads,
// load(buf, batch, count), were issued while the batch before it was in use.  Two buffers take turns with no
// copy between them (a copy would wait for the loads in flight), full batches load without per-row conditions
// (count == U folds them away), and the last rows % U rows come as one short batch.
template <int U, typename Buf, typename Load, typename Use>
__device__ __forceinline__ void stream_rows(int64_t rows, Load&& load, Use&& use) {
  Buf a, b;
  const int64_t full = rows / U;
  if (full > 0) load(a, 0, U);
  for (int64_t i = 0; i < full; i += 2) {
    if (i + 1 < full) load(b, i + 1, U);
    use(a, i, U);
    if (i + 1 >= full) break;
    if (i + 2 < full) load(a, i + 2, U);
    use(b, i + 1, U);
  }
  const int rest = (int)(rows - full * U);
  if (rest > 0) {
    load(a, full, rest);
    use(a, full, rest);
  }
}

// Rows per block of a column-striped kernel: about `target` blocks in all, long stripes, within the grid's
// y limit.
inline int64_t stripe_rows(int64_t K, int64_t col_blocks, int64_t target) {
  int64_t row_blocks = mxq::ceil_div(target, col_blocks);
  if (row_blocks > K) row_blocks = K;
  if (row_blocks < 1) row_blocks = 1;
  if (row_blocks > 65535) row_blocks = 65535;
  return mxq::ceil_div(K, row_blocks);
}

// k-means over each of ng groups (one 64-lane workgroup each): T (ng x kSize) and, when code_map is not NULL,
// per group and element code c < 2^(e+m+1) the bits of the entry pick chooses for the code's value (NaN for a
// code with no bin) at code_map[g * ncodes + c].  exact_sums: sums_exact() holds for the groups.
int launch_kmeans(const CountSource& src, int64_t ng, int nv, const float* grid, const float* safe, int ns,
                  const int* safe_order, int max_iters, float* T, uint32_t* code_map, const CodeGrid& cg,
                  bool exact_sums, hipStream_t st);

}  // namespace mxq_lut
