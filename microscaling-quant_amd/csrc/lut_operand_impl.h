// block.lut's first step fused with the histogram the tables are fitted to (mxq/block/lut.py:23-34 with
// mxq/lut/kmeans.py:46-60): one kernel quantizes a K x n tensor in blocks of 32 rows the MX-Gemmini way,
// keeps the element codes as bytes (the pick reads them back: a quarter of float32's traffic) and the scales
// as float32, and counts every code's grid bin per column group while the codes are in registers.
//
// Workgroup: 16 waves over one tile of CW columns and one split of the row blocks.  A wave covers 8 * VEC
// columns of a block: lane l takes rows 4 (l / 8) .. + 3 of the VEC columns (l % 8) * VEC .. + VEC - 1 (eight
// lanes share those columns' maxima through exchanges, as the split quantize kernel does).  The tile is
// CW / (8 VEC) waves wide; the 16 / that wave rows take the split's blocks in turn.  (VEC = 8, CW = 128: two
// waves side by side write a row's 128 code bytes, 64 each, at the same time.)  The histogram is LDS,
// (CW >> group, at least 1) units of nv counts, written whole into the split's slice of the partial counts
// at the end; k-means sums the splits.
#pragma once
#include "lut_impl.h"
#include "quantize_impl.h"

namespace mxq_lut {

struct LutQuantArgs {
  uint8_t* codes;            // K x n element codes
  float* X;                  // ceil(K / 32) x n scales
  int* partial;              // nsplit x (ntiles * units) x nv counts
  int* err;                  // bit 0: a value that is not a code of the format
  int64_t K, n;
  int group, nv, units;
  CodeGrid cg;
  int64_t blocks_per_split;
  int64_t split_stride;      // words between two splits' slices of `partial`
  mxq_quant::ByteSink sink;  // the element codes off nearest even (its X is unused)
};

template <typename T, int MODE, int VEC, int CW>
__global__ void __launch_bounds__(1024) k_lut_quant(const T* __restrict__ V, LutQuantArgs a, mxq_block_spec s) {
  constexpr int WX = CW / (8 * VEC);                 // waves across the tile
  constexpr int WY = 16 / WX;                        // wave rows: each takes every WY-th block of the split
  constexpr int PER = (VEC + 7) / 8;                 // scales each lane evaluates
  extern __shared__ int hist[];
  for (int i = threadIdx.x; i < a.units * a.nv; i += blockDim.x) hist[i] = 0;
  __syncthreads();
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int c = lane & 7, r = lane >> 3;
  const int64_t n = a.n;
  const int64_t j0 = (int64_t)blockIdx.x * CW + (w % WX) * (8 * VEC) + c * VEC;
  const int jt = (w % WX) * (8 * VEC) + c * VEC;     // that column within the tile
  const bool live = j0 < n;                          // n % VEC == 0: all VEC columns or none
  const int64_t nb = (a.K + 31) / 32;
  const int64_t b_lo = (int64_t)blockIdx.y * a.blocks_per_split;
  const int64_t b_hi = b_lo + a.blocks_per_split < nb ? b_lo + a.blocks_per_split : nb;
  bool bad = false;
  for (int64_t b = b_lo + w / WX; b < b_hi; b += WY) {
    const int64_t k0 = b * 32;
    const int rows = (int)(a.K - k0 < 32 ? a.K - k0 : 32);
    const T* src = V + (k0 + r * 4) * n + (live ? j0 : 0);
    float v[4][VEC];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (rows == 32 || r * 4 + i < rows) {
        mxq_quant::load_vec<T, VEC>(src + (int64_t)i * n, v[i]);
      } else {
#pragma unroll
        for (int j = 0; j < VEC; ++j) v[i][j] = 0.0f;
      }
    }
    // block maxima as |v| bit patterns (a NaN pattern lies above +Inf, so NaN wins as torch.amax's does)
    uint32_t am[VEC];
#pragma unroll
    for (int j = 0; j < VEC; ++j) {
      am[j] = f2u(v[0][j]) & 0x7FFFFFFFu;
#pragma unroll
      for (int i = 1; i < 4; ++i) am[j] = max(am[j], f2u(v[i][j]) & 0x7FFFFFFFu);
    }
#pragma unroll
    for (int step = 8; step < 64; step <<= 1)
#pragma unroll
      for (int j = 0; j < VEC; ++j) am[j] = max(am[j], (uint32_t)__shfl_xor((int)am[j], step, 64));
    // lane r evaluates the scales of columns r + 8q; column j's is then read from lane c + (j % 8) * 8
    float own[PER];
#pragma unroll
    for (int q = 0; q < PER; ++q) {
      uint32_t mine = am[8 * q];
#pragma unroll
      for (int jj = 1; jj < 8; ++jj)
        if (8 * q + jj < VEC) mine = (r == jj) ? am[8 * q + jj] : mine;
      own[q] = block_scale(u2f(mine), s);
    }
    // the scales: stored by the row-part-0 lanes, then the division by each (a multiply by the exact
    // reciprocal when every scale of the wave is a normal power of two, make_div's test; else IEEE division)
    float xs[VEC];
    bool p2 = true;
#pragma unroll
    for (int j = 0; j < VEC; ++j) {
      xs[j] = __shfl(own[j / 8], c + (j % 8) * 8, 64);
      p2 = p2 && make_div(xs[j]).inv != 0.0f;
    }
    if (live && r == 0) {
      float* xd = a.X + b * n + j0;
#pragma unroll
      for (int q = 0; q < VEC / 4; ++q)
        *reinterpret_cast<float4*>(xd + 4 * q) = make_float4(xs[4 * q], xs[4 * q + 1], xs[4 * q + 2], xs[4 * q + 3]);
    }
    const bool div = s.scale_rule && !__all(p2);
    if (div) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < VEC; ++j) v[i][j] = apply_div(v[i][j], make_div(xs[j]));
    } else if (s.scale_rule) {
#pragma unroll
      for (int j = 0; j < VEC; ++j) {
        const float inv = make_div(xs[j]).inv;        // every scale here is a normal power of two: exact
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i][j] = v[i][j] * inv;
      }
    }
    // nearest even: the hardware conversions give the codes (ocp_hw.h).  Under MX-Gemmini's scale every
    // finite V scales to |z| < 2, inside their range; a non-finite one (whose codes block.lut refuses) sets
    // the flag instead.
    if constexpr (MODE == MXQ_RNE) {
#pragma unroll
      for (int j = 0; j < VEC; ++j) bad |= !(am[j] < 0x7F800000u);
    }
    if (!live) continue;
    // row i's VEC codes: stored, and each counted in its column's unit (a code with no bin, from a non-finite
    // V, sets the flag and is counted in bin 0: the call then raises, and no branch per code is needed)
    auto emit = [&](int i, const uint32_t (&wd)[VEC / 4]) {
      uint8_t* dst = a.codes + (k0 + r * 4 + i) * n + j0;
      if constexpr (VEC == 8) *reinterpret_cast<uint2*>(dst) = make_uint2(wd[0], wd[1]);
      else *reinterpret_cast<uint32_t*>(dst) = wd[0];
#pragma unroll
      for (int q = 0; q < VEC / 4; ++q)
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const int bin = code_bin((wd[q] >> (8 * t)) & 0xFFu, a.cg);
          bad |= bin < 0;
          atomicAdd(&hist[((jt + 4 * q + t) >> a.group) * a.nv + (bin < 0 ? 0 : bin)], 1);
        }
    };
    if constexpr (MODE == MXQ_RNE) {
      float z[4 * VEC];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < VEC; ++j) z[i * VEC + j] = v[i][j];
      uint32_t c[VEC];                                 // row i in words i * VEC / 4 ..
      mxq_ocp_hw::codes<4 * VEC>(z, s.e, s.m, c);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if (rows != 32 && r * 4 + i >= rows) continue;
        uint32_t wd[VEC / 4];
#pragma unroll
        for (int q = 0; q < VEC / 4; ++q) wd[q] = c[i * (VEC / 4) + q];
        emit(i, wd);
      }
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if (rows != 32 && r * 4 + i >= rows) continue;
        uint32_t wd[VEC / 4];
#pragma unroll
        for (int q = 0; q < VEC / 4; ++q) {
          const float z[4] = {v[i][4 * q], v[i][4 * q + 1], v[i][4 * q + 2], v[i][4 * q + 3]};
          wd[q] = a.sink.template word<MXQ_ELEM_OCP, MODE, 4>(z, s);
        }
        emit(i, wd);
      }
    }
  }
  if (bad) atomicOr(a.err, 1);
  __syncthreads();
  // this tile's units into the split's slice: unit u of tile t is slot t * units + u (a unit that starts past
  // n has no columns and no slot that k-means reads)
  int* out = a.partial + (int64_t)blockIdx.y * a.split_stride + (int64_t)blockIdx.x * a.units * a.nv;
  for (int i = threadIdx.x; i < a.units * a.nv; i += blockDim.x) {
    const int u = i / a.nv;
    if ((int64_t)blockIdx.x * CW + ((int64_t)u << a.group) < n) out[i] = hist[i];
  }
}

// Launch k_lut_quant over a grid of ntiles x nsplit workgroups: tiles of 128 columns (VEC 8), or of 32
// (VEC 4) when cw is 32.
template <typename T>
int launch_lut_quant(const T* V, const LutQuantArgs& a, const mxq_block_spec& s, int cw, int64_t ntiles,
                     int64_t nsplit, hipStream_t st) {
  const dim3 grid((unsigned)ntiles, (unsigned)nsplit);
  const size_t lds = (size_t)a.units * a.nv * sizeof(int);
  auto go = [&](auto mode_c) {
    constexpr int MODE = decltype(mode_c)::value;
    if (cw == 128) k_lut_quant<T, MODE, 8, 128><<<grid, 1024, lds, st>>>(V, a, s);
    else k_lut_quant<T, MODE, 4, 32><<<grid, 1024, lds, st>>>(V, a, s);
  };
  switch (s.rounding) {
    case MXQ_RNE: go(std::integral_constant<int, MXQ_RNE>{}); break;
    case MXQ_TIES_AWAY: go(std::integral_constant<int, MXQ_TIES_AWAY>{}); break;
    default: go(std::integral_constant<int, MXQ_TRUNC>{}); break;
  }
  return mxq::check_launch("mxq_block_lut quantize");
}

}  // namespace mxq_lut

// One instantiation per input type (lut_operand_{f32,bf16,f16}.hip).
int mxq_lut_quant_f32(const void* V, const mxq_lut::LutQuantArgs& a, const mxq_block_spec& s, int cw,
                      int64_t ntiles, int64_t nsplit, hipStream_t st);
int mxq_lut_quant_bf16(const void* V, const mxq_lut::LutQuantArgs& a, const mxq_block_spec& s, int cw,
                       int64_t ntiles, int64_t nsplit, hipStream_t st);
int mxq_lut_quant_f16(const void* V, const mxq_lut::LutQuantArgs& a, const mxq_block_spec& s, int cw,
                      int64_t ntiles, int64_t nsplit, hipStream_t st);
