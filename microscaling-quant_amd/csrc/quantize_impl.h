// Fused MX block quantization and dequantization for gfx950.
//
// A tensor is viewed as (outer, n, inner) with the block axis n in the middle.  Three layouts:
//   split    (block 32): eight lanes of a wavefront share one block column of VEC adjacent columns, four rows
//            each; their maxima meet through cross-lane exchanges; the block stays in registers.
//   contig32 (inner == 1, block 32, n % 32 == 0): eight lanes own one contiguous 128-byte block, four
//            elements each.
//   strided  (any other block size): one thread per block column, the block read twice.
// Kernels are specialised on the element rule and, for the OCP grid and the microxcaling step, on the
// rounding mode.
// Step 1 (the scale) runs once per block and column; step 2 (the element grid) once per element.  The
// division by the scale is a multiply by its reciprocal when the scale is a normal power of two (then both
// are the same correctly rounded value) and an IEEE division otherwise (the 1e-38 floor is not a power of two).
#pragma once
#include "mxq_common.h"
#include "mxq_numerics.h"

#include <stdlib.h>

namespace mxq_quant {


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

// Codes are written once and not read back by this kernel: streaming (non-temporal) stores.
typedef float f32x4 __attribute__((ext_vector_type(4)));
template <int VEC>
__device__ __forceinline__ void store_vec_nt(float* p, const float (&in)[VEC]) {
  if constexpr (VEC == 4) {
    f32x4 r = {in[0], in[1], in[2], in[3]};
    __builtin_nontemporal_store(r, reinterpret_cast<f32x4*>(p));
  } else {
#pragma unroll
    for (int j = 0; j < VEC; ++j) __builtin_nontemporal_store(in[j], p + j);
  }
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

// z = v / X for the VEC block columns of a lane: a multiply by the exact reciprocal when every scale of the
// wave is a normal power of two (the same correctly rounded value), the IEEE division otherwise.
template <int VEC>
__device__ __forceinline__ bool wave_needs_div(const Div (&d)[VEC]) {
  bool need = false;
#pragma unroll
  for (int j = 0; j < VEC; ++j) need |= (d[j].inv == 0.0f);
  return __any(need);
}

// Any block size (read twice: once for the amax, once for the elements), one thread per block column of
// VEC adjacent columns.
template <typename T, int ELEM, int MODE, int VEC>
__global__ void __launch_bounds__(256) k_quant_strided(const T* __restrict__ V, float* __restrict__ P,
                                                       float* __restrict__ X, int64_t outer, int64_t n,
                                                       int64_t inner, int64_t bs, int64_t nb, mxq_block_spec s) {
  const int64_t groups = inner / VEC;
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= outer * nb * groups) return;
  int64_t o, b, g;
  split_index(t, groups, nb, o, b, g);
  const int64_t k0 = b * bs;
  const int64_t rows = (n - k0 < bs) ? n - k0 : bs;
  const int64_t off = (o * n + k0) * inner + g * VEC;
  float amax[VEC];
#pragma unroll
  for (int j = 0; j < VEC; ++j) amax[j] = 0.0f;
  for (int64_t r = 0; r < rows; ++r) {
    float v[VEC];
    load_vec<T, VEC>(V + off + r * inner, v);
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
    load_vec<T, VEC>(V + off + r * inner, v);
#pragma unroll
    for (int j = 0; j < VEC; ++j) q[j] = elem_qm<ELEM, MODE>(s.scale_rule ? apply_div(v[j], d[j]) : v[j], s);
    store_vec_nt<VEC>(P + off + r * inner, q);
  }
  store_vec<VEC>(X + (o * nb + b) * inner + g * VEC, xs);
}

// Block size 32 with R lanes of one wavefront sharing a block column: lane l of a wave takes row part
// r = l / (64 / R) (rows [r * 32/R, (r+1) * 32/R) of the block) and column group cg_base + l % (64 / R); the R
// partial maxima meet through cross-lane exchanges.  Few values per lane keep many waves resident, which is
// what hides the HBM latency here (measured on MI355X: R = 8, VEC = 4 is the fastest layout on 8192 x 8192
// bf16 and on 4096 x 512 float32).
//   * The wave's index is uniform, so the (outer, block, column-group) split of it runs in scalar registers.
//   * A whole block (all but a tail) loads without per-row conditions; lanes past the last column group read
//     column group 0 (valid memory) and store nothing.
//   * The block maximum is the largest |v| bit pattern (non-negative floats order like their patterns, and
//     every NaN pattern lies above +Inf, so a NaN wins as torch.amax's does).
//   * The R lanes of a column group hold the same maxima after the exchanges; lane r < VEC computes the scale
//     of column r alone and the others read it (one scale rule evaluation per lane instead of VEC).
template <typename T, int ELEM, int MODE, int VEC, int R>
__global__ void __launch_bounds__(256) k_quant_split(const T* __restrict__ V, float* __restrict__ P,
                                                     float* __restrict__ X, int64_t outer, int64_t n, int64_t inner,
                                                     int64_t nb, int64_t waves_per_row, mxq_block_spec s) {
  constexpr int CPW = 64 / R;          // column groups per wave
  constexpr int ROWS = 32 / R;         // rows per lane
  static_assert(VEC <= R, "one scale-computing lane per column");
  const int64_t groups = inner / VEC;
  const int lane = threadIdx.x & 63;
  const int64_t wave = (int64_t)blockIdx.x * (256 / 64) + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (wave >= outer * nb * waves_per_row) return;    // whole waves only: the exchanges below see every lane
  const int64_t wr = wave / waves_per_row;           // (o, b) flattened
  const int64_t o = wr / nb, b = wr - o * nb;
  const int64_t k0 = b * 32;
  const int rows = (int)((n - k0 < 32) ? n - k0 : 32);
  const int c = lane % CPW, r = lane / CPW;
  const int64_t cg = (wave - wr * waves_per_row) * CPW + c;
  const bool live = cg < groups;
  const T* src = V + (o * n + k0 + r * ROWS) * inner + (live ? cg : 0) * VEC;

  float v[ROWS][VEC];
  uint32_t am[VEC];
#pragma unroll
  for (int j = 0; j < VEC; ++j) am[j] = 0u;
  if (rows == 32) {
#pragma unroll
    for (int i = 0; i < ROWS; ++i) load_vec<T, VEC>(src + (int64_t)i * inner, v[i]);
  } else {
#pragma unroll
    for (int i = 0; i < ROWS; ++i) {
      if (r * ROWS + i < rows) {
        load_vec<T, VEC>(src + (int64_t)i * inner, v[i]);
      } else {
#pragma unroll
        for (int j = 0; j < VEC; ++j) v[i][j] = 0.0f;
      }
    }
  }
#pragma unroll
  for (int i = 0; i < ROWS; ++i)
#pragma unroll
    for (int j = 0; j < VEC; ++j) am[j] = max(am[j], f2u(v[i][j]) & 0x7FFFFFFFu);
#pragma unroll
  for (int step = CPW; step < 64; step <<= 1)
#pragma unroll
    for (int j = 0; j < VEC; ++j) am[j] = max(am[j], (uint32_t)__shfl_xor((int)am[j], step, 64));
  // lane r < VEC: the scale of column r of its group; every lane then reads column j's from lane c + j * CPW
  uint32_t mine = am[0];
#pragma unroll
  for (int j = 1; j < VEC; ++j) mine = (r == j) ? am[j] : mine;
  const float own = block_scale(u2f(mine), s);
  float xs[VEC];
  Div d[VEC];
#pragma unroll
  for (int j = 0; j < VEC; ++j) {
    xs[j] = __shfl(own, c + j * CPW, 64);
    d[j] = make_div(xs[j]);
  }
  if (s.scale_rule && wave_needs_div<VEC>(d)) {
#pragma unroll
    for (int i = 0; i < ROWS; ++i)
#pragma unroll
      for (int j = 0; j < VEC; ++j) v[i][j] = apply_div(v[i][j], d[j]);
  } else if (s.scale_rule) {
#pragma unroll
    for (int i = 0; i < ROWS; ++i)
#pragma unroll
      for (int j = 0; j < VEC; ++j) v[i][j] = v[i][j] * d[j].inv;
  }
  if (!live) return;
  float* dst = P + (o * n + k0 + r * ROWS) * inner + cg * VEC;
#pragma unroll
  for (int i = 0; i < ROWS; ++i) {
    if (rows == 32 || r * ROWS + i < rows) {
      float q[VEC];
#pragma unroll
      for (int j = 0; j < VEC; ++j) q[j] = elem_qm<ELEM, MODE>(v[i][j], s);
      store_vec_nt<VEC>(dst + (int64_t)i * inner, q);
    }
  }
  if (r == 0) store_vec<VEC>(X + (o * nb + b) * inner + cg * VEC, xs);
}

// inner == 1, blocks of 32 contiguous elements, n % 32 == 0: eight lanes per block, four elements per lane.
template <typename T, int ELEM, int MODE>
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
  for (int j = 0; j < 4; ++j) q[j] = elem_qm<ELEM, MODE>(s.scale_rule ? apply_div(v[j], d) : v[j], s);
  store_vec_nt<4>(P + off, q);
  if ((t & 7) == 0) X[blk] = xs;
}

// V = M^T with M (inner x n) row-major in memory, blocks of 32 along n: every block is 32 contiguous elements
// of a row of M.  A workgroup quantizes a tile of 64 rows of M x 64 of n (two blocks per row): loads along M's
// rows (coalesced), eight lanes of four elements per block whose maxima meet through exchanges, and the codes
// pass through LDS to leave along P's rows (P is V-shaped: n x inner).  The same scale and element rules as
// the other layouts, per block; no copy of the transposed input is made.
constexpr int kTT = 64;

template <typename T, int ELEM, int MODE>
__global__ void __launch_bounds__(256) k_quant_t(const T* __restrict__ M, float* __restrict__ P,
                                                 float* __restrict__ X, int64_t n, int64_t inner, int64_t tiles_k,
                                                 int vec_in, int vec_out, mxq_block_spec s) {
  __shared__ float tile[kTT][kTT + 1];               // [position along n][row of M]
  const int64_t tc = blockIdx.x / tiles_k, tk = blockIdx.x - tc * tiles_k;
  const int64_t c0 = tc * kTT, k0 = tk * kTT;
  const bool full = c0 + kTT <= inner && k0 + kTT <= n;
  const int tid = threadIdx.x;
#pragma unroll
  for (int it = 0; it < 4; ++it) {
    const int id = it * 256 + tid;
    const int row = id >> 4, quad = id & 15;          // 8 consecutive lanes: one row, one block of 32
    const int64_t c = c0 + row, k = k0 + quad * 4;
    float v[4];
    if (full && vec_in) {
      load_vec<T, 4>(M + c * n + k, v);
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = (c < inner && k + e < n) ? to_f32(M[c * n + k + e]) : 0.0f;
    }
    uint32_t am = 0u;
#pragma unroll
    for (int e = 0; e < 4; ++e) am = max(am, f2u(v[e]) & 0x7FFFFFFFu);
    am = max(am, (uint32_t)__shfl_xor((int)am, 1, 8));
    am = max(am, (uint32_t)__shfl_xor((int)am, 2, 8));
    am = max(am, (uint32_t)__shfl_xor((int)am, 4, 8));
    const float xs = block_scale(u2f(am), s);
    const Div d = make_div(xs);
#pragma unroll
    for (int e = 0; e < 4; ++e) tile[quad * 4 + e][row] = elem_qm<ELEM, MODE>(s.scale_rule ? apply_div(v[e], d) : v[e], s);
    if ((quad & 7) == 0 && c < inner && k < n) X[(k >> 5) * inner + c] = xs;
  }
  __syncthreads();
#pragma unroll
  for (int it = 0; it < 4; ++it) {
    const int id = it * 256 + tid;
    const int key = id >> 4, cq = (id & 15) * 4;
    const int64_t k = k0 + key, c = c0 + cq;
    float q[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) q[e] = tile[key][cq + e];
    if (full && vec_out) {
      store_vec_nt<4>(P + k * inner + c, q);
    } else if (k < n) {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (c + e < inner) P[k * inner + c + e] = q[e];
    }
  }
}

template <typename T, int ELEM, int MODE>
int launch_quant_t(const T* M, float* P, float* X, int64_t n, int64_t inner, const mxq_block_spec& q,
                   hipStream_t st) {
  mxq::KernelTimer timer("block_quantize", st);
  const int64_t tiles_k = mxq::ceil_div(n, kTT), tiles = mxq::ceil_div(inner, kTT) * tiles_k;
  if (tiles > INT32_MAX) return mxq::invalid("mxq_block_quantize_t: tensor too large");
  const int vec_in = n % 4 == 0 && reinterpret_cast<uintptr_t>(M) % (4 * sizeof(T)) == 0;
  const int vec_out = inner % 4 == 0 && reinterpret_cast<uintptr_t>(P) % 16 == 0;
  k_quant_t<T, ELEM, MODE><<<dim3((unsigned)tiles), 256, 0, st>>>(M, P, X, n, inner, tiles_k, vec_in, vec_out, q);
  return mxq::check_launch("mxq_block_quantize_t");
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
    store_vec_nt<VEC>(out + off + r * inner, v);
  }
}

// ------------------------------------------------------------------------------------------ host side
inline int validate(const mxq_block_spec& s) {
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

// bs < 0: the transposed layout (outer 1, block 32, V read as M^T), k_quant_t.
template <typename T, int ELEM, int MODE>
int launch_quant(const T* V, float* P, float* X, int64_t outer, int64_t n, int64_t inner, int64_t bs,
                 const mxq_block_spec& q, hipStream_t st) {
  if (bs < 0) return launch_quant_t<T, ELEM, MODE>(V, P, X, n, inner, q, st);
  mxq::KernelTimer timer("block_quantize", st);
  const int64_t nb = mxq::ceil_div(n, bs);
  const uintptr_t av = reinterpret_cast<uintptr_t>(V), ap = reinterpret_cast<uintptr_t>(P),
                  ax = reinterpret_cast<uintptr_t>(X);
  if (inner == 1 && bs == 32 && n % 32 == 0 && av % (4 * sizeof(T)) == 0 && ap % 16 == 0) {
    const int64_t nblocks = outer * nb;
    k_quant_contig32<T, ELEM, MODE><<<mxq::grid_for(nblocks * 8, 256), 256, 0, st>>>(V, P, X, nblocks, q);
    return mxq::check_launch("mxq_block_quantize");
  }
  auto aligned = [&](int vec) {
    return inner % vec == 0 && av % (vec * sizeof(T)) == 0 && ap % (vec * 4) == 0 && ax % (vec * 4) == 0;
  };
  const int vec = aligned(4) ? 4 : (aligned(2) ? 2 : 1);
  if (bs == 32) {
    constexpr int R = 8;
    const int64_t wpr = mxq::ceil_div(inner / vec, 64 / R);
    const int64_t threads = outer * nb * wpr * 64;
    const dim3 grid = mxq::grid_for(threads, 256);
    if (vec == 4) k_quant_split<T, ELEM, MODE, 4, R><<<grid, 256, 0, st>>>(V, P, X, outer, n, inner, nb, wpr, q);
    else if (vec == 2) k_quant_split<T, ELEM, MODE, 2, R><<<grid, 256, 0, st>>>(V, P, X, outer, n, inner, nb, wpr, q);
    else k_quant_split<T, ELEM, MODE, 1, R><<<grid, 256, 0, st>>>(V, P, X, outer, n, inner, nb, wpr, q);
    return mxq::check_launch("mxq_block_quantize");
  }
  const int64_t threads = outer * nb * (inner / vec);
  const dim3 grid = mxq::grid_for(threads, 256);
  if (vec == 4) k_quant_strided<T, ELEM, MODE, 4><<<grid, 256, 0, st>>>(V, P, X, outer, n, inner, bs, nb, q);
  else if (vec == 2) k_quant_strided<T, ELEM, MODE, 2><<<grid, 256, 0, st>>>(V, P, X, outer, n, inner, bs, nb, q);
  else k_quant_strided<T, ELEM, MODE, 1><<<grid, 256, 0, st>>>(V, P, X, outer, n, inner, bs, nb, q);
  return mxq::check_launch("mxq_block_quantize");
}

template <typename T, int ELEM>
int launch_mode(const T* V, float* P, float* X, int64_t outer, int64_t n, int64_t inner, int64_t bs,
                const mxq_block_spec& q, hipStream_t st) {
  switch (q.rounding) {
    case MXQ_RNE: return launch_quant<T, ELEM, MXQ_RNE>(V, P, X, outer, n, inner, bs, q, st);
    case MXQ_TIES_AWAY: return launch_quant<T, ELEM, MXQ_TIES_AWAY>(V, P, X, outer, n, inner, bs, q, st);
    default: return launch_quant<T, ELEM, MXQ_TRUNC>(V, P, X, outer, n, inner, bs, q, st);
  }
}

template <typename T>
int dispatch_elem(const T* V, float* P, float* X, int64_t outer, int64_t n, int64_t inner, int64_t bs,
                  const mxq_block_spec& q, hipStream_t st) {
  switch (q.elem) {
    case MXQ_ELEM_QTORCH: return launch_quant<T, MXQ_ELEM_QTORCH, -1>(V, P, X, outer, n, inner, bs, q, st);
    case MXQ_ELEM_IEEE: return launch_quant<T, MXQ_ELEM_IEEE, -1>(V, P, X, outer, n, inner, bs, q, st);
    case MXQ_ELEM_OCP: return launch_mode<T, MXQ_ELEM_OCP>(V, P, X, outer, n, inner, bs, q, st);
    case MXQ_ELEM_MICROSOFT: return launch_mode<T, MXQ_ELEM_MICROSOFT>(V, P, X, outer, n, inner, bs, q, st);
    default: return launch_quant<T, MXQ_ELEM_NONE, -1>(V, P, X, outer, n, inner, bs, q, st);
  }
}

}  // namespace mxq_quant
