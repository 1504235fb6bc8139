// LDS tile staging and the per-step stage functions shared by the reducers (systolic.hip, trees.hip).
#pragma once

#include "mxq_common.h"
#include "mxq_numerics.h"

namespace mxq_red {

// RNE of y at m fraction bits by Veltkamp's split with C = 2^(23 - m) + 1: c = y * C, then c - (c - y).  Three
// full-rate float operations; the bit form, (u + 2^(22-m) - 1 + lsb) & mask, needs a bit-field extract and a
// three-way add, which gfx950 issues at half rate.  Equal to the bit form for every integer |y| < 2^24 at
// m = 1..9 (an exhaustive check), hence, the split commuting with powers of two, for every finite y whose
// y * C stays finite and normal: the systolic e4 sums (integers in lane units, below 2^(15 + m)), the
// systolic bf16 lane's sums (below 2^10 in magnitude, or the workgroup's results are discarded) and the adder
// tree's level sums.  A subnormal y on the bf16 grid (a multiple of 2^-133) is returned unchanged, as by the
// bit form.  Not contracted: an fma of y * C - y would leave c unrounded.
__device__ __forceinline__ float split_rne(float y, float C) {
#pragma clang fp contract(off)
  const float c = y * C;
  return c - (c - y);
}

// An operand matrix: row stride and problem stride in elements.
struct Operand {
  const float* p;
  int64_t ld;     // elements between rows
  int64_t batch;  // elements between problems
};

// Workgroup tile BM x BN outputs, K staged 32 rows at a time through LDS (two buffers).
constexpr int KT = 32;

template <int BM, int BN>
struct Smem {
  float a[2][KT][BM];
  float b[2][KT][BN];
};

// Loads rows [k0, k0 + KT) x cols [c0, c0 + W) of an R x L matrix with row stride ld into registers (zero
// outside the matrix).  vec_ok: ld and the base are multiples of 4 floats / 16 bytes.
template <int W, int NT>
struct TileLoader {
  static constexpr int PER = KT * W / NT;  // floats per thread
  float v[PER];
  __device__ __forceinline__ void load(const float* __restrict__ src, int64_t ld, int64_t R, int64_t L, int64_t k0,
                                       int64_t c0, bool vec_ok) {
    const int t = threadIdx.x;
    if (vec_ok) {
#pragma unroll
      for (int j = 0; j < PER / 4; ++j) {
        const int e = (t + j * NT) * 4;
        const int r = e / W, c = e % W;
        const int64_t gr = k0 + r, gc = c0 + c;
        float4 q = make_float4(0.f, 0.f, 0.f, 0.f);
        if (gr < R && gc + 3 < L) q = *reinterpret_cast<const float4*>(src + gr * ld + gc);
        else if (gr < R) {
          if (gc < L) q.x = src[gr * ld + gc];
          if (gc + 1 < L) q.y = src[gr * ld + gc + 1];
          if (gc + 2 < L) q.z = src[gr * ld + gc + 2];
        }
        v[j * 4 + 0] = q.x; v[j * 4 + 1] = q.y; v[j * 4 + 2] = q.z; v[j * 4 + 3] = q.w;
      }
    } else {
#pragma unroll
      for (int j = 0; j < PER; ++j) {
        const int e = t + j * NT;
        const int r = e / W, c = e % W;
        const int64_t gr = k0 + r, gc = c0 + c;
        v[j] = (gr < R && gc < L) ? src[gr * ld + gc] : 0.0f;
      }
    }
  }
  // The same rows when all of them and all W columns lie inside the matrix, 16-byte aligned: `row0` points at
  // (k0, c0), an address uniform over the workgroup, and each lane adds its own 32-bit element offset
  // r * ld + c (loop-invariant; the caller keeps 32 * ld below 2^31), so no bounds or 64-bit address math per
  // load.
  __device__ __forceinline__ void load_inner(const float* __restrict__ row0, uint32_t ld) {
    const int t = threadIdx.x;
#pragma unroll
    for (int j = 0; j < PER / 4; ++j) {
      const int e = (t + j * NT) * 4;
      const uint32_t r = (uint32_t)(e / W), c = (uint32_t)(e % W);
      const float4 q = *reinterpret_cast<const float4*>(row0 + (r * ld + c));
      v[j * 4 + 0] = q.x; v[j * 4 + 1] = q.y; v[j * 4 + 2] = q.z; v[j * 4 + 3] = q.w;
    }
  }
  __device__ __forceinline__ void store(float (*dst)[W], bool vec_ok) const {
    const int t = threadIdx.x;
    if (vec_ok) {
#pragma unroll
      for (int j = 0; j < PER / 4; ++j) {
        const int e = (t + j * NT) * 4;
        *reinterpret_cast<float4*>(&dst[e / W][e % W]) = make_float4(v[j * 4], v[j * 4 + 1], v[j * 4 + 2], v[j * 4 + 3]);
      }
    } else {
#pragma unroll
      for (int j = 0; j < PER; ++j) {
        const int e = t + j * NT;
        dst[e / W][e % W] = v[j];
      }
    }
  }
  // the largest |x| bit pattern among the staged values (patterns of non-negative floats order like values)
  __device__ __forceinline__ uint32_t max_bits() const {
    uint32_t mx = 0u;
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      const uint32_t u = f2u(v[j]) & 0x7FFFFFFFu;
      mx = u > mx ? u : mx;
    }
    return mx;
  }
};

__device__ __forceinline__ bool vec_ok(const Operand& o, const float* base) {
  return o.ld % 4 == 0 && reinterpret_cast<uintptr_t>(base) % 16 == 0;
}

__device__ __forceinline__ uint32_t umax(uint32_t a, uint32_t b) { return a > b ? a : b; }

// The Arithmetic's three stages for any supported codes (mxq/matmul/_arithmetic.py:64-134).
__device__ __forceinline__ float gen_product(float a, float b, const mxq_arith_spec& ar) {
  if (ar.kind == MXQ_ARITH_MXQUANT) return mxq_q(a * b, ar.prod_e, ar.prod_m);
  return mxg_product(a, b, ar.prod_m, ar.has_floor != 0, ar.flush_thr, ar.sat_limit, ar.sat_value);
}
__device__ __forceinline__ float gen_acc(float S, float p, int e, int m, const mxq_arith_spec& ar) {
  if (ar.kind == MXQ_ARITH_MXQUANT) return mxq_q(S + p, e, m);
  return mxg_acc_add(S, p, e, m);
}
__device__ __forceinline__ float gen_tile(float C, float tile, const mxq_arith_spec& ar) {
  if (ar.kind == MXQ_ARITH_MXQUANT) return C + tile;
  return mxg_tile_add(C, tile);
}

}  // namespace mxq_red
