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
#include "ocp_hw.h"

#include <stdlib.h>
#include <type_traits>

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

// Where a kernel's codes and scales go; the sink also runs step 2 (the element rule) on the scaled values z.
//   FloatSink  float32 P and X, the reference's outputs (codes written with streaming stores).
//   ByteSink   one element-code byte per element and one E8M0 byte per scale (mx_encode, e8m0_encode); a value
//              neither format holds sets *err (a zero block's scale is free, its value being 0 under any).
// `at` is an element index of P (or X); VEC consecutive elements, VEC-aligned.
struct FloatSink {
  float* P;
  float* X;
  static constexpr int kBytes = 4;
  template <int ELEM, int MODE, int VEC>
  __device__ __forceinline__ void elems(int64_t at, const float (&z)[VEC], const mxq_block_spec& s) const {
    float q[VEC];
#pragma unroll
    for (int j = 0; j < VEC; ++j) q[j] = elem_qm<ELEM, MODE>(z[j], s);
    store_vec_nt<VEC>(P + at, q);
  }
  template <int VEC>
  __device__ __forceinline__ void scales(int64_t at, const float (&xs)[VEC], const bool (&)[VEC]) const {
    store_vec<VEC>(X + at, xs);
  }
  // The OCP grid rounded to nearest even by the hardware conversions (ocp_hw.h; the caller has checked the
  // range): the rows of a lane's strip of VEC (4 or 8) columns, rows [0, live) stored.
  template <int ROWS, int VEC>
  __device__ __forceinline__ void hw_rows(int64_t at, int64_t stride, const float (&v)[ROWS][VEC], int live,
                                          const mxq_block_spec& s) const {
    float z[ROWS * VEC];
#pragma unroll
    for (int i = 0; i < ROWS; ++i)
#pragma unroll
      for (int j = 0; j < VEC; ++j) z[VEC * i + j] = v[i][j];
    mxq_ocp_hw::values<ROWS * VEC>(z, s.e, s.m);
#pragma unroll
    for (int i = 0; i < ROWS; ++i) {
      if (i >= live) break;
#pragma unroll
      for (int q = 0; q < VEC / 4; ++q) {
        const float o[4] = {z[VEC * i + 4 * q], z[VEC * i + 4 * q + 1], z[VEC * i + 4 * q + 2], z[VEC * i + 4 * q + 3]};
        store_vec_nt<4>(P + at + (int64_t)i * stride + 4 * q, o);
      }
    }
  }
  __device__ __forceinline__ bool hw_format(const mxq_block_spec&) const { return true; }
  __device__ __forceinline__ uintptr_t p_addr() const { return reinterpret_cast<uintptr_t>(P); }
  __device__ __forceinline__ uintptr_t x_addr() const { return reinterpret_cast<uintptr_t>(X); }
};

template <int VEC>
__device__ __forceinline__ void store_bytes(uint8_t* p, uint32_t w) {
  if constexpr (VEC == 4) *reinterpret_cast<uint32_t*>(p) = w;
  else if constexpr (VEC == 2) *reinterpret_cast<uint16_t*>(p) = (uint16_t)w;
  else *p = (uint8_t)w;
}

// W words of code bytes (1, 2 or 4: 4, 8 or 16 bytes, aligned), one store.
// The byte sink's stores: plain, not streaming.  A wave writes 64 bytes of a code row and the next wave the rest of
// its 128-byte line; streaming stores of those halves wrote 1.28x the code and scale bytes (bf16 8192 x 8192: 88.4 MB for 69.2),
// plain ones exactly them, in the same time.  (The float sink's rows are whole lines; its streaming stores keep
// 268 MB of codes out of L2 and run faster than plain ones.)
template <int W>
__device__ __forceinline__ void store_words(uint8_t* p, const uint32_t (&w)[W]) {
  if constexpr (W == 1) {
    *reinterpret_cast<uint32_t*>(p) = w[0];
  } else if constexpr (W == 4) {
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    *reinterpret_cast<u32x4*>(p) = u32x4{w[0], w[1], w[2], w[3]};
  } else {
    static_assert(W == 2, "4, 8 or 16 bytes");
    typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
    *reinterpret_cast<u32x2*>(p) = u32x2{w[0], w[1]};
  }
}

// The element format's constants for the byte sink's short encoder.
struct CodeConsts {
  uint32_t nmin;      // bit pattern of 2^emin, the smallest normal
  uint32_t nshift;    // 23 - m
  uint32_t nsub;      // (127 - bias) << m: float32 exponent bias to the format's, in code position
  uint32_t lowmask;   // the float32 fraction bits below the format's m
  uint32_t maxbits;   // bit pattern of the largest finite value
  float sub_mul;      // 2^(m - emin): a subnormal value in units of the format's subnormal step
  int sign_at;        // e + m
};

__host__ __device__ inline CodeConsts code_consts(int e, int m) {
  CodeConsts k{};
  const int bias = (1 << (e - 1)) - 1, emin = 1 - bias;
  k.nmin = (uint32_t)(emin + 127) << 23;
  k.nshift = (uint32_t)(23 - m);
  k.nsub = (uint32_t)(127 - bias) << m;
  k.lowmask = (1u << (23 - m)) - 1u;
  int emax = (1 << e) - 1 - bias;                  // largest exponent field's exponent
  uint32_t mmax = (1u << m) - 1u;                   // largest mantissa there
  if (e == 5 && m == 2) emax -= 1;                  // E5M2: the top exponent field is Inf / NaN
  if (e == 4 && m == 3) mmax -= 1;                  // E4M3: S.1111.111 is NaN
  k.maxbits = ((uint32_t)(emax + 127) << 23) | (mmax << (23 - m));
  k.sub_mul = __builtin_bit_cast(float, (uint32_t)(m - emin + 127) << 23);
  k.sign_at = e + m;
  return k;
}

// The code of a value the element rule put on the format's grid: normal, (bits >> (23 - m)) less the exponent
// bias difference; subnormal (or zero), its multiple of the subnormal step.  `good` is false for anything
// else (beyond the largest finite value, a special, or off the grid: the qtorch grid's smallest values), which
// then takes mx_encode.
__device__ __forceinline__ uint32_t short_encode(float q, const CodeConsts& k, bool& good) {
  const uint32_t u = f2u(q), a = u & 0x7FFFFFFFu;
  const bool nrm = a >= k.nmin;
  const float t = u2f(a) * k.sub_mul;
  const uint32_t cs = __float2uint_rz(t);            // saturating convert: any t is defined
  const uint32_t mag = nrm ? (a >> k.nshift) - k.nsub : cs;
  good = a <= k.maxbits && (nrm ? (a & k.lowmask) == 0u : (float)cs == t);
  return mag | ((u >> 31) << k.sign_at);
}

struct ByteSink {
  uint8_t* P;
  uint8_t* X;
  int32_t* err;
  int e, m;
  CodeConsts k;
  uint32_t maxcode;    // the code of the largest finite value
  static constexpr int kBytes = 1;
  // mxgemmini's ocp grid without `via` yields the code from its own roundings (ocp_code_t); every other rule
  // rounds to float32 and the code is read off the value (short_encode).  Specials, and values the grid made
  // that the format lacks, take mx_encode.
  template <int ELEM, int MODE, int VEC>
  __device__ __forceinline__ void elems(int64_t at, const float (&z)[VEC], const mxq_block_spec& s) const {
    if constexpr (VEC == 8 || VEC == 16) {
      uint32_t w[VEC / 4];
#pragma unroll
      for (int q = 0; q < VEC / 4; ++q) {
        const float z4[4] = {z[4 * q], z[4 * q + 1], z[4 * q + 2], z[4 * q + 3]};
        w[q] = word<ELEM, MODE, 4>(z4, s);
      }
      store_words<VEC / 4>(P + at, w);
    } else {
      store_bytes<VEC>(P + at, word<ELEM, MODE, VEC>(z, s));
    }
  }
  // The codes of VEC (at most 4) scaled values, code j in byte j.
  template <int ELEM, int MODE, int VEC>
  __device__ __forceinline__ uint32_t word(const float (&z)[VEC], const mxq_block_spec& s) const {
    uint32_t w = 0u;
    bool all_good = true;
    if constexpr (ELEM == MXQ_ELEM_OCP && MODE >= 0) {
      if (s.via_e == 0) {
#pragma unroll
        for (int j = 0; j < VEC; ++j) {
          bool good;
          w |= ocp_code_t<MODE>(z[j], e, m, maxcode, &good) << (8 * j);
          all_good = all_good && good;
        }
        return all_good ? w : general_codes<ELEM, MODE, VEC>(z, s);
      }
    }
#pragma unroll
    for (int j = 0; j < VEC; ++j) {
      bool good;
      w |= short_encode(elem_qm<ELEM, MODE>(z[j], s), k, good) << (8 * j);
      all_good = all_good && good;
    }
    return all_good ? w : general_codes<ELEM, MODE, VEC>(z, s);
  }
  template <int ELEM, int MODE, int VEC>
  __device__ __forceinline__ uint32_t general_codes(const float (&z)[VEC], const mxq_block_spec& s) const {
    bool ok = true;
    uint32_t w = 0u;
#pragma unroll
    for (int j = 0; j < VEC; ++j) w |= mx_encode(elem_qm<ELEM, MODE>(z[j], s), e, m, &ok) << (8 * j);
    if (!ok) atomicOr(err, 1);
    return w;
  }
  // hw_rows of FloatSink with the codes themselves (the byte format is the element format: e, m == s.e, s.m).
  template <int ROWS, int VEC>
  __device__ __forceinline__ void hw_rows(int64_t at, int64_t stride, const float (&v)[ROWS][VEC], int live,
                                          const mxq_block_spec& s) const {
    float z[ROWS * VEC];
#pragma unroll
    for (int i = 0; i < ROWS; ++i)
#pragma unroll
      for (int j = 0; j < VEC; ++j) z[VEC * i + j] = v[i][j];
    // the conversions take at most 32 values: in chunks of rows
    constexpr int CH = ROWS * VEC <= 32 ? ROWS * VEC : 32;
    uint32_t w[ROWS * VEC / 4];
#pragma unroll
    for (int c0 = 0; c0 < ROWS * VEC; c0 += CH) {
      float zc[CH];
      uint32_t wc[CH / 4];
#pragma unroll
      for (int k = 0; k < CH; ++k) zc[k] = z[c0 + k];
      mxq_ocp_hw::codes<CH>(zc, s.e, s.m, wc);
#pragma unroll
      for (int k = 0; k < CH / 4; ++k) w[c0 / 4 + k] = wc[k];
    }
#pragma unroll
    for (int i = 0; i < ROWS; ++i) {
      if (i >= live) break;
      uint32_t row[VEC / 4];
#pragma unroll
      for (int q = 0; q < VEC / 4; ++q) row[q] = w[i * (VEC / 4) + q];
      store_words<VEC / 4>(P + at + (int64_t)i * stride, row);
    }
  }
  // the codes the conversions give are the byte format's when it is the grid's
  __device__ __forceinline__ bool hw_format(const mxq_block_spec& s) const { return e == s.e && m == s.m; }
  template <int VEC>
  __device__ __forceinline__ void scales(int64_t at, const float (&xs)[VEC], const bool (&zero)[VEC]) const {
    bool ok = true;
    uint32_t w[(VEC + 3) / 4] = {};
#pragma unroll
    for (int j = 0; j < VEC; ++j) w[j / 4] |= e8m0_encode(xs[j], zero[j], &ok) << (8 * (j % 4));
    if constexpr (VEC >= 8) store_words<VEC / 4>(X + at, w);
    else store_bytes<VEC>(X + at, w[0]);
    if (!ok) atomicOr(err, 2);
  }
  __device__ __forceinline__ uintptr_t p_addr() const { return reinterpret_cast<uintptr_t>(P); }
  __device__ __forceinline__ uintptr_t x_addr() const { return reinterpret_cast<uintptr_t>(X); }
};

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
template <typename T, int ELEM, int MODE, int VEC, typename SINK>
__global__ void __launch_bounds__(256) k_quant_strided(const T* __restrict__ V, const SINK out, int64_t outer,
                                                       int64_t n, int64_t inner, int64_t bs, int64_t nb,
                                                       mxq_block_spec s) {
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
    float v[VEC], z[VEC];
    load_vec<T, VEC>(V + off + r * inner, v);
#pragma unroll
    for (int j = 0; j < VEC; ++j) z[j] = s.scale_rule ? apply_div(v[j], d[j]) : v[j];
    out.template elems<ELEM, MODE, VEC>(off + r * inner, z, s);
  }
  bool zero[VEC];
#pragma unroll
  for (int j = 0; j < VEC; ++j) zero[j] = amax[j] == 0.0f;
  out.template scales<VEC>((o * nb + b) * inner + g * VEC, xs, zero);
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
//   * The R lanes of a column group hold the same maxima after the exchanges; lane r computes the scales of
//     columns r, r + R, ... alone and the others read them (ceil(VEC / R) scale rule evaluations per lane
//     instead of VEC).
template <typename T, int ELEM, int MODE, int VEC, int R, typename SINK>
__global__ void __launch_bounds__(256) k_quant_split(const T* __restrict__ V, const SINK out, int64_t outer,
                                                     int64_t n, int64_t inner, mxq::DivU31 nb_div,
                                                     mxq::DivU31 wpr_div, mxq_block_spec s) {
  constexpr int CPW = 64 / R;          // column groups per wave
  constexpr int ROWS = 32 / R;         // rows per lane
  constexpr int PER = (VEC + R - 1) / R;  // scales each lane evaluates
  const int64_t groups = inner / VEC;
  const int lane = threadIdx.x & 63;
  const int64_t nb = nb_div.d, waves_per_row = wpr_div.d;
  // the launch keeps the wave count below 2^31
  const uint32_t wave = blockIdx.x * (256 / 64) + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if ((int64_t)wave >= outer * nb * waves_per_row) return;   // whole waves only: the exchanges below see every lane
  const uint32_t wr = mxq::divu31(wave, wpr_div);      // (o, b) flattened
  const uint32_t o32 = mxq::divu31(wr, nb_div);
  const int64_t o = o32, b = wr - o32 * nb_div.d;
  const int64_t k0 = b * 32;
  const int rows = (int)((n - k0 < 32) ? n - k0 : 32);
  const int c = lane % CPW, r = lane / CPW;
  const int64_t cg = (int64_t)(wave - wr * wpr_div.d) * CPW + c;
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
  // lane r evaluates the scales of columns r, r + R, ... of its group (those below VEC); every lane then reads
  // column j's from lane c + (j % R) * CPW
  float own[PER];
#pragma unroll
  for (int q = 0; q < PER; ++q) {
    uint32_t mine = am[q * R];
#pragma unroll
    for (int jj = 1; jj < R; ++jj)
      if (q * R + jj < VEC) mine = (r == jj) ? am[q * R + jj] : mine;
    own[q] = block_scale(u2f(mine), s);
  }
  float xs[VEC];
  Div d[VEC];
#pragma unroll
  for (int j = 0; j < VEC; ++j) {
    xs[j] = __shfl(own[j / R], c + (j % R) * CPW, 64);
    d[j] = make_div(xs[j]);
  }
  const bool div = s.scale_rule && wave_needs_div<VEC>(d);
  if (div) {
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
  // the OCP grid at nearest even by the hardware conversions when every scaled value of the wave is finite
  // and within their range (a column's largest |z| is its maximum scaled, the division being monotone) and the
  // grid saturates where they do (max_norm the format's own)
  constexpr bool HW_OCP = ELEM == MXQ_ELEM_OCP && MODE == MXQ_RNE && VEC >= 4;
  constexpr bool HW_MS = ELEM == MXQ_ELEM_MICROSOFT && MODE == MXQ_RNE && VEC >= 4;
  bool hw = false;
  if constexpr (HW_OCP) {
    if (s.via_e == 0 && mxq_ocp_hw::has_hw_n<ROWS * VEC>(s.e, s.m) && out.hw_format(s) &&
        s.max_norm == mxq_ocp_hw::fmt_max(s.e, s.m)) {
      const float lim = mxq_ocp_hw::hw_limit(s.e, s.m);
      bool ok = true;
#pragma unroll
      for (int j = 0; j < VEC; ++j) {
        const float a = u2f(am[j]);
        const float zm = !s.scale_rule ? a : (div ? apply_div(a, d[j]) : a * d[j].inv);
        ok = ok && am[j] < 0x7F800000u && zm < lim;
      }
      hw = __all(ok);
    }
  }
  // microxcaling's "even" (mxq/microxcaling/elemwise.py:29-60) is the OCP grid at nearest even, saturating at
  // max_norm, with one exception: the float32 just below half the smallest subnormal step, which its float32
  // floor(|A| + 0.5) rounds up to that step.  So with every value and scaled value finite and none of that
  // magnitude, the values clamped to +-max_norm go to the hardware conversions.
  mxq_block_spec hs = s;                             // the element format as the conversions name it
  if constexpr (HW_MS) {
    hs.m = s.m - 2;                                   // microxcaling's mbits count the sign and hidden bits
    if (s.via_e == 0 && mxq_ocp_hw::has_hw_n<ROWS * VEC>(hs.e, hs.m) && out.hw_format(hs) &&
        s.max_norm == mxq_ocp_hw::fmt_max(hs.e, hs.m)) {
      const int emin = 2 - (1 << (hs.e - 1));
      const uint32_t odd = (uint32_t)(127 + emin - hs.m - 1) << 23;  // 2^(emin - m - 1), then one float below
      bool ok = true;
#pragma unroll
      for (int j = 0; j < VEC; ++j) {               // finite inputs and finite scaled values (a NaN scale fails)
        const float a = u2f(am[j]);
        const float zm = !s.scale_rule ? a : (div ? apply_div(a, d[j]) : a * d[j].inv);
        ok = ok && am[j] < 0x7F800000u && zm < INFINITY;
      }
#pragma unroll
      for (int i = 0; i < ROWS; ++i)
#pragma unroll
        for (int j = 0; j < VEC; ++j) ok = ok && (f2u(v[i][j]) & 0x7FFFFFFFu) != odd - 1u;
      hw = __all(ok);
      if (hw) {
#pragma unroll
        for (int i = 0; i < ROWS; ++i)
#pragma unroll
          for (int j = 0; j < VEC; ++j) v[i][j] = fminf(fmaxf(v[i][j], -s.max_norm), s.max_norm);
      }
    }
  }
  if (!live) return;
  const int64_t dst = (o * n + k0 + r * ROWS) * inner + cg * VEC;
  if constexpr (HW_OCP || HW_MS) {
    if (hw) out.template hw_rows<ROWS, VEC>(dst, inner, v, rows == 32 ? ROWS : rows - r * ROWS, hs);
  }
  if (!hw) {
    // the element grid in software, one row at a time from a second read of the row (the same loads and the
    // same scaling give the same values): the registers of this rare path are one row's, so the kernel's
    // count is the conversions' path's and more waves fit on a SIMD
#pragma unroll 1
    for (int i = 0; i < ROWS; ++i) {
      if (rows == 32 || r * ROWS + i < rows) {
        float z[VEC];
        load_vec<T, VEC>(src + (int64_t)i * inner, z);
        if (div) {
#pragma unroll
          for (int j = 0; j < VEC; ++j) z[j] = apply_div(z[j], d[j]);
        } else if (s.scale_rule) {
#pragma unroll
          for (int j = 0; j < VEC; ++j) z[j] = z[j] * d[j].inv;
        }
        out.template elems<ELEM, MODE, VEC>(dst + (int64_t)i * inner, z, s);
      }
    }
  }
  if (r == 0) {
    bool zero[VEC];
#pragma unroll
    for (int j = 0; j < VEC; ++j) zero[j] = am[j] == 0u;
    out.template scales<VEC>((o * nb + b) * inner + cg * VEC, xs, zero);
  }
}

// inner == 1, blocks of 32 contiguous elements, n % 32 == 0: eight lanes per block, four elements per lane.
template <typename T, int ELEM, int MODE, typename SINK>
__global__ void __launch_bounds__(256) k_quant_contig32(const T* __restrict__ V, const SINK out, int64_t nblocks,
                                                        mxq_block_spec s) {
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
  float z[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) z[j] = s.scale_rule ? apply_div(v[j], d) : v[j];
  out.template elems<ELEM, MODE, 4>(off, z, s);
  if ((t & 7) == 0) {
    const float x1[1] = {xs};
    const bool z1[1] = {a == 0.0f};
    out.template scales<1>(blk, x1, z1);
  }
}

// ------------------------------------------------------ code bytes of the OCP grid at nearest even, one pass
// k_pack_rne: the byte sink for the OCP element grid rounded to nearest even and saturating at the format's own
// largest value (block.mxgemmini's rounding_mode="rne" without `via`), blocks of 32 along the axis, eight
// adjacent columns a lane, R lanes of a wave per block column (32 / R rows each), as k_quant_split lays them out.
// Written for the instruction count of the common wave, whose inputs and scaled values are finite and whose
// block scales are normal powers of two:
//   * 16-bit inputs stay packed two to a register; the column maxima are packed 16-bit maxima (|x| patterns
//     order as the values do, a NaN above Inf, as in float32).
//   * one lane of each column's R evaluates the scale rule and hands the others its E8M0 byte, which is all
//     they need: the reciprocal of a normal power of two 2^k is 2^-k, read off the byte.
//   * z = fma(v, 1/X, +0): v / X correctly rounded, -0 made +0 (the grid's sign for an exact zero);
//     clamped to +-max (the grid saturates: rounding a clamped value gives the saturated one), then converted
//     by gfx950's scaled conversions at scale 1, which round to nearest even with true subnormals.
//   * FP6 through the FP8 conversions: E2M3 is E4M3's grid on z * 2^-6 and E3M2 is E5M2's on z * 2^-12 (the
//     same mantissa widths; the exponent offsets map one format's subnormal step and binades onto the other's),
//     whose code bytes, with the top exponent bits zero, move the sign from bit 7 to bit 5.  FP4 converts two
//     values into a byte, spread to one a byte.
// A wave with any other block (a non-finite value, a scale that is not a normal power of two) takes
// k_quant_split's software element path for all of its blocks.
namespace pkr {

template <typename T>
struct In;                                            // a lane's row of eight values: loads and maxima
template <>
struct In<float> {
  static constexpr int NW = 8, NA = 8;                // words per row, words of column maxima
  static constexpr uint32_t kFin = 0x7F800000u;       // |x| patterns below this are finite
  __device__ static void load(const float* p, uint32_t (&w)[NW]) {
    const uint4 a = *reinterpret_cast<const uint4*>(p), b = *reinterpret_cast<const uint4*>(p + 4);
    w[0] = a.x; w[1] = a.y; w[2] = a.z; w[3] = a.w; w[4] = b.x; w[5] = b.y; w[6] = b.z; w[7] = b.w;
  }
  __device__ static void amax(uint32_t (&am)[NA], const uint32_t (&w)[NW]) {
#pragma unroll
    for (int j = 0; j < NW; ++j) am[j] = max(am[j], w[j] & 0x7FFFFFFFu);
  }
  __device__ static uint32_t column(const uint32_t (&am)[NA], int j) { return am[j]; }
  __device__ static float f32(uint32_t a) { return u2f(a); }
  __device__ static float value(const uint32_t (&w)[NW], int j) { return u2f(w[j]); }
};
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t max_u16x2(uint32_t a, uint32_t b) {
  return __builtin_bit_cast(uint32_t, __builtin_elementwise_max(__builtin_bit_cast(u16x2, a),
                                                               __builtin_bit_cast(u16x2, b)));
}
struct In16 {
  static constexpr int NW = 4, NA = 4;
  template <typename T>
  __device__ static void load(const T* p, uint32_t (&w)[NW]) {
    const uint4 a = *reinterpret_cast<const uint4*>(p);
    w[0] = a.x; w[1] = a.y; w[2] = a.z; w[3] = a.w;
  }
  __device__ static void amax(uint32_t (&am)[NA], const uint32_t (&w)[NW]) {
#pragma unroll
    for (int j = 0; j < NW; ++j) am[j] = max_u16x2(am[j], w[j] & 0x7FFF7FFFu);
  }
  __device__ static uint32_t column(const uint32_t (&am)[NA], int j) { return (am[j >> 1] >> (16 * (j & 1))) & 0xFFFFu; }
};
template <>
struct In<bf16_t> : In16 {
  static constexpr uint32_t kFin = 0x7F80u;
  __device__ static float f32(uint32_t a) { return u2f(a << 16); }
  __device__ static float value(const uint32_t (&w)[NW], int j) {
    return (j & 1) ? u2f(w[j >> 1] & 0xFFFF0000u) : u2f(w[j >> 1] << 16);
  }
};
template <>
struct In<f16_t> : In16 {
  static constexpr uint32_t kFin = 0x7C00u;
  __device__ static float f32(uint32_t a) { return (float)__builtin_bit_cast(_Float16, (uint16_t)a); }
  __device__ static float value(const uint32_t (&w)[NW], int j) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(w[j >> 1] >> (16 * (j & 1))));
  }
};

// Per element format (e, m): the pre-scale exponent of the conversion used, the clamp, the four codes.
template <int E, int M>
struct Code {
  static_assert((E == 4 && M == 3) || (E == 5 && M == 2) || (E == 2 && M == 3) || (E == 3 && M == 2) ||
                (E == 2 && M == 1), "an OCP MX element format");
  static constexpr int SH = (E == 2 && M == 3) ? 6 : ((E == 3 && M == 2) ? 12 : 0);   // z * 2^-SH converted
  static constexpr float MAXV = (E == 4) ? 448.0f : (E == 5) ? 57344.0f : (M == 3) ? 7.5f : (E == 3) ? 28.0f : 6.0f;
  static constexpr float CLAMP = MAXV / (float)(1u << SH);
  __device__ static uint32_t four(float z0, float z1, float z2, float z3) {
    if constexpr (E == 2 && M == 1) {
      uint32_t r = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(0u, z0, z1, 1.0f, 0);     // byte 0: z1 z0 nibbles
      r = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(r, z2, z3, 1.0f, 2);              // byte 2: z3 z2
      return (r & 0x000F000Fu) | ((r & 0x00F000F0u) << 4);
    } else {
      mxq_ocp_hw::s2v r = {0, 0};
      if constexpr (M == 3) {                                                         // E4M3, E2M3
        r = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(r, z0, z1, 1.0f, false);
        r = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(r, z2, z3, 1.0f, true);
      } else {                                                                        // E5M2, E3M2
        r = __builtin_amdgcn_cvt_scalef32_pk_bf8_f32(r, z0, z1, 1.0f, false);
        r = __builtin_amdgcn_cvt_scalef32_pk_bf8_f32(r, z2, z3, 1.0f, true);
      }
      const uint32_t w = __builtin_bit_cast(uint32_t, r);
      if constexpr (SH != 0) return (w & 0x1F1F1F1Fu) | ((w >> 2) & 0x20202020u);   // sign: bit 7 -> bit 5
      else return w;
    }
  }
};

}  // namespace pkr

template <typename T, int E, int M, int R>
__global__ void __launch_bounds__(256) k_pack_rne(const T* __restrict__ V, const ByteSink out, int64_t outer, int64_t n,
                                                  int64_t inner, mxq::DivU31 nb_div, mxq::DivU31 wpr_div,
                                                  mxq_block_spec s) {
  using In = pkr::In<T>;
  using Cd = pkr::Code<E, M>;
  constexpr int VEC = 8, CPW = 64 / R, ROWS = 32 / R, PER = VEC / R;
  static_assert(R == 4 || R == 8, "4 or 8 lanes per block column");
  const int64_t groups = inner / VEC;
  const int lane = threadIdx.x & 63;
  const int64_t nb = nb_div.d;
  const uint32_t wave = blockIdx.x * (256 / 64) + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if ((int64_t)wave >= outer * nb * wpr_div.d) return;   // whole waves only: the exchanges below see every lane
  const uint32_t wr = mxq::divu31(wave, wpr_div);
  const uint32_t o32 = mxq::divu31(wr, nb_div);
  const int64_t o = o32, b = wr - o32 * nb_div.d;
  const int64_t k0 = b * 32;
  const int rows = (int)((n - k0 < 32) ? n - k0 : 32);
  const int c = lane % CPW, r = lane / CPW;
  const int64_t cg = (int64_t)(wave - wr * wpr_div.d) * CPW + c;
  const bool live = cg < groups;
  const T* src = V + (o * n + k0 + r * ROWS) * inner + (live ? cg : 0) * VEC;

  uint32_t w[ROWS][In::NW];
  uint32_t am[In::NA];
#pragma unroll
  for (int j = 0; j < In::NA; ++j) am[j] = 0u;
#pragma unroll
  for (int i = 0; i < ROWS; ++i) {
    if (rows == 32 || r * ROWS + i < rows) {
      In::load(src + (int64_t)i * inner, w[i]);
    } else {
#pragma unroll
      for (int j = 0; j < In::NW; ++j) w[i][j] = 0u;
    }
    In::amax(am, w[i]);
  }
#pragma unroll
  for (int step = CPW; step < 64; step <<= 1)
#pragma unroll
    for (int j = 0; j < In::NA; ++j) {
      const uint32_t other = (uint32_t)__shfl_xor((int)am[j], step, 64);
      if constexpr (In::NA == 8) am[j] = max(am[j], other);
      else am[j] = pkr::max_u16x2(am[j], other);
    }
  // lane r evaluates the scales of columns r, r + R, ...; a column's E8M0 byte when its maximum is finite and
  // its scale a normal power of two, else 0
  float own_x[PER];
  uint32_t own_b[PER];
#pragma unroll
  for (int q = 0; q < PER; ++q) {
    uint32_t mine = In::column(am, q * R);
#pragma unroll
    for (int jj = 1; jj < R; ++jj) mine = (r == jj) ? In::column(am, q * R + jj) : mine;
    own_x[q] = block_scale(In::f32(mine), s);
    const uint32_t u = f2u(own_x[q]), be = u >> 23;
    own_b[q] = (mine < In::kFin && (u & 0x807FFFFFu) == 0u && be >= 1u && be <= 254u) ? be : 0u;
  }
  uint32_t eb[VEC];
  bool fast = true;
#pragma unroll
  for (int j = 0; j < VEC; ++j) {
    eb[j] = (uint32_t)__shfl((int)own_b[j / R], c + (j % R) * CPW, 64);
    fast = fast && eb[j] != 0u;
  }
  const int64_t dst = (o * n + k0 + r * ROWS) * inner + cg * VEC;
  const int64_t xat = (o * nb + b) * inner + cg * VEC;
  if (__all(fast)) {
    if (!live) return;
    float inv[VEC];
#pragma unroll
    for (int j = 0; j < VEC; ++j) {
      const int ex = 254 - (int)eb[j] - Cd::SH;                     // 2^-(k + SH), normal or subnormal
      inv[j] = u2f(ex >= 1 ? (uint32_t)ex << 23 : 1u << (22 + ex));
    }
#pragma unroll
    for (int i = 0; i < ROWS; ++i) {
      float z[VEC];
#pragma unroll
      for (int j = 0; j < VEC; ++j)
        z[j] = __builtin_amdgcn_fmed3f(__builtin_fmaf(In::value(w[i], j), inv[j], 0.0f), -Cd::CLAMP, Cd::CLAMP);
      const uint32_t w0 = Cd::four(z[0], z[1], z[2], z[3]), w1 = Cd::four(z[4], z[5], z[6], z[7]);
      if (rows == 32 || r * ROWS + i < rows) store_words<2>(out.P + dst + (int64_t)i * inner, {w0, w1});
    }
    if (r == 0)
      store_words<2>(out.X + xat, {eb[0] | eb[1] << 8 | eb[2] << 16 | eb[3] << 24,
                                   eb[4] | eb[5] << 8 | eb[6] << 16 | eb[7] << 24});
    return;
  }
  // the software element path for the whole wave (k_quant_split's, on the same scales and divisions)
  float xs[VEC];
  Div d[VEC];
#pragma unroll
  for (int j = 0; j < VEC; ++j) {
    xs[j] = __shfl(own_x[j / R], c + (j % R) * CPW, 64);
    d[j] = make_div(xs[j]);
  }
  if (!live) return;
  // rows read again from memory (the same values), so that this rare path holds one row's registers
#pragma unroll 1
  for (int i = 0; i < ROWS; ++i) {
    if (rows == 32 || r * ROWS + i < rows) {
      uint32_t wi[In::NW];
      In::load(src + (int64_t)i * inner, wi);
#pragma unroll 1
      for (int h = 0; h < VEC; h += 4) {                 // four codes at a time: fewer registers again
        float z[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float v = In::value(wi, h + j);
          z[j] = s.scale_rule ? apply_div(v, d[h + j]) : v;
        }
        out.template elems<MXQ_ELEM_OCP, MXQ_RNE, 4>(dst + (int64_t)i * inner + h, z, s);
      }
    }
  }
  if (r == 0) {
    bool zero[VEC];
#pragma unroll
    for (int j = 0; j < VEC; ++j) zero[j] = In::column(am, j) == 0u;
    out.template scales<VEC>(xat, xs, zero);
  }
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

// out = P * expand(X) as one flat pass over the (outer, n, inner) view: a thread takes VEC adjacent elements of a
// row (one block, so one VEC-wide load of X), and every thread has work, whatever the block size and shape.
// I is uint32_t while the element count fits it (cheap index arithmetic), else int64_t.
template <int VEC, typename I>
__global__ void __launch_bounds__(256) k_dequant_flat(const float* __restrict__ P, const float* __restrict__ X,
                                                      float* __restrict__ out, I count, I inner_v, I n, I bs, I nb) {
  const I t = (I)blockIdx.x * 256u + (I)threadIdx.x;
  if (t >= count) return;
  const I row = t / inner_v;                      // (o, k) flattened
  const I iv = t - row * inner_v;
  const I o = row / n, k = row - o * n;
  float v[VEC], xs[VEC];
  load_vec<float, VEC>(P + (int64_t)t * VEC, v);
  load_vec<float, VEC>(X + ((int64_t)(o * nb + k / bs) * inner_v + iv) * VEC, xs);
#pragma unroll
  for (int j = 0; j < VEC; ++j) v[j] = v[j] * xs[j];
  store_vec_nt<VEC>(out + (int64_t)t * VEC, v);
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

// k_pack_rne for blocks of 32 along the axis, inner % 8 == 0, V 16-byte aligned, codes and scales 8-byte
// aligned: four lanes per block column (eight rows each) while that gives the chip at least 2048 waves,
// else eight (four rows each).
template <typename T>
int launch_pack_rne(const T* V, const ByteSink& out, int64_t outer, int64_t n, int64_t inner, int64_t nb,
                    const mxq_block_spec& q, hipStream_t st) {
  const int64_t groups = inner / 8;
  if (outer * nb * mxq::ceil_div(groups, 8) >= (int64_t(1) << 31))
    return mxq::invalid("block quantize: tensor too large (2^31 waves of 2048 elements)");
  auto go = [&](auto r_const) {
    constexpr int R = decltype(r_const)::value;
    const int64_t wpr = mxq::ceil_div(groups, 64 / R);
    const dim3 grid = mxq::grid_for(outer * nb * wpr * 64, 256);
    const mxq::DivU31 dnb = mxq::make_divu31((uint32_t)nb), dwpr = mxq::make_divu31((uint32_t)wpr);
    auto run = [&](auto kern) { kern<<<grid, 256, 0, st>>>(V, out, outer, n, inner, dnb, dwpr, q); };
    if (q.e == 4) run(k_pack_rne<T, 4, 3, R>);
    else if (q.e == 5) run(k_pack_rne<T, 5, 2, R>);
    else if (q.e == 3) run(k_pack_rne<T, 3, 2, R>);
    else if (q.m == 3) run(k_pack_rne<T, 2, 3, R>);
    else run(k_pack_rne<T, 2, 1, R>);
  };
  if (outer * nb * mxq::ceil_div(groups, 16) >= 2048) go(std::integral_constant<int, 4>{});
  else go(std::integral_constant<int, 8>{});
  return mxq::check_launch("mxq_block_quantize_packed");
}

// bs < 0: the transposed layout (outer 1, block 32, V read as M^T), k_quant_t (float32 outputs only).
template <typename T, int ELEM, int MODE, typename SINK>
int launch_quant(const T* V, const SINK& out, int64_t outer, int64_t n, int64_t inner, int64_t bs,
                 const mxq_block_spec& q, hipStream_t st) {
  if constexpr (SINK::kBytes == 4) {
    if (bs < 0) return launch_quant_t<T, ELEM, MODE>(V, out.P, out.X, n, inner, q, st);
  } else if (bs < 0) {
    return mxq::invalid("mxq_block_quantize_packed: no transposed layout");
  }
  mxq::KernelTimer timer("block_quantize", st);
  const int64_t nb = mxq::ceil_div(n, bs);
  const uintptr_t av = reinterpret_cast<uintptr_t>(V), ap = reinterpret_cast<uintptr_t>(out.P),
                  ax = reinterpret_cast<uintptr_t>(out.X);
  constexpr int OB = SINK::kBytes;
  if (inner == 1 && bs == 32 && n % 32 == 0 && av % (4 * sizeof(T)) == 0 && ap % (4 * OB) == 0) {
    const int64_t nblocks = outer * nb;
    k_quant_contig32<T, ELEM, MODE, SINK><<<mxq::grid_for(nblocks * 8, 256), 256, 0, st>>>(V, out, nblocks, q);
    return mxq::check_launch("mxq_block_quantize");
  }
  auto aligned = [&](int vec) {
    return inner % vec == 0 && av % (vec * sizeof(T)) == 0 && ap % (vec * OB) == 0 && ax % (vec * OB) == 0;
  };
  const int vec = aligned(4) ? 4 : (aligned(2) ? 2 : 1);
  if constexpr (SINK::kBytes == 1 && ELEM == MXQ_ELEM_OCP && MODE == MXQ_RNE) {
    if (bs == 32 && q.via_e == 0 && out.e == q.e && out.m == q.m && mxq_ocp_hw::has_hw(q.e, q.m) &&
        q.max_norm == mxq_ocp_hw::fmt_max(q.e, q.m) && aligned(8) && av % 16 == 0)
      return launch_pack_rne(V, out, outer, n, inner, nb, q, st);
  }
  if (bs == 32) {
    // code bytes: eight columns a lane when they align (8-byte stores: a wave's eight lanes write 64 contiguous
    // bytes of a row, the next wave the other half of the line; sixteen would keep 64 values a lane, which
    // this layout's registers do not hold)
    const int bvec = SINK::kBytes == 1 && aligned(8) ? 8 : 0;
    const int kvec = bvec ? bvec : vec;
    // R = 8 lanes per block column (4 rows each) while that gives the chip at least 8 waves per SIMD; smaller
    // tensors take R = 32 (one row per lane, four times the waves), which keeps more loads in flight (MI355X,
    // block.ocp on 4096 x 512 float32: 12.2 us at R = 8, 9.7 us at R = 32; bf16 8192 x 8192: R = 8 fastest)
    const int64_t waves8 = outer * nb * mxq::ceil_div(inner / kvec, 64 / 8);
    auto go = [&](auto r_const) {
      constexpr int R = decltype(r_const)::value;
      const int64_t wpr = mxq::ceil_div(inner / kvec, 64 / R);
      const dim3 grid = mxq::grid_for(outer * nb * wpr * 64, 256);
      const mxq::DivU31 dnb = mxq::make_divu31((uint32_t)nb), dwpr = mxq::make_divu31((uint32_t)wpr);
      if constexpr (SINK::kBytes == 1) {
        if (bvec == 8) {
          k_quant_split<T, ELEM, MODE, 8, R, SINK><<<grid, 256, 0, st>>>(V, out, outer, n, inner, dnb, dwpr, q);
          return;
        }
      }
      if (vec == 4) k_quant_split<T, ELEM, MODE, 4, R, SINK><<<grid, 256, 0, st>>>(V, out, outer, n, inner, dnb, dwpr, q);
      else if (vec == 2) k_quant_split<T, ELEM, MODE, 2, R, SINK><<<grid, 256, 0, st>>>(V, out, outer, n, inner, dnb, dwpr, q);
      else k_quant_split<T, ELEM, MODE, 1, R, SINK><<<grid, 256, 0, st>>>(V, out, outer, n, inner, dnb, dwpr, q);
    };
    // the kernel indexes waves in 32 bits
    if (outer * nb * mxq::ceil_div(inner / kvec, 64 / 32) >= (int64_t(1) << 31))
      return mxq::invalid("block quantize: tensor too large (2^31 waves of 2048 elements)");
    if (waves8 >= 8 * 1024) go(std::integral_constant<int, 8>{});
    else go(std::integral_constant<int, 32>{});
    return mxq::check_launch("mxq_block_quantize");
  }
  const int64_t threads = outer * nb * (inner / vec);
  const dim3 grid = mxq::grid_for(threads, 256);
  if (vec == 4) k_quant_strided<T, ELEM, MODE, 4, SINK><<<grid, 256, 0, st>>>(V, out, outer, n, inner, bs, nb, q);
  else if (vec == 2) k_quant_strided<T, ELEM, MODE, 2, SINK><<<grid, 256, 0, st>>>(V, out, outer, n, inner, bs, nb, q);
  else k_quant_strided<T, ELEM, MODE, 1, SINK><<<grid, 256, 0, st>>>(V, out, outer, n, inner, bs, nb, q);
  return mxq::check_launch("mxq_block_quantize");
}

template <typename T, int ELEM, typename SINK>
int launch_mode(const T* V, const SINK& out, int64_t outer, int64_t n, int64_t inner, int64_t bs,
                const mxq_block_spec& q, hipStream_t st) {
  switch (q.rounding) {
    case MXQ_RNE: return launch_quant<T, ELEM, MXQ_RNE>(V, out, outer, n, inner, bs, q, st);
    case MXQ_TIES_AWAY: return launch_quant<T, ELEM, MXQ_TIES_AWAY>(V, out, outer, n, inner, bs, q, st);
    default: return launch_quant<T, ELEM, MXQ_TRUNC>(V, out, outer, n, inner, bs, q, st);
  }
}

// Float32 outputs: every element rule.  Bytes: the rules whose grids are the OCP element formats' (mxgemmini's
// ocp grid, block.ocp's microxcaling step) and mxquant's qtorch grid (whose smallest values some formats lack:
// those set the error word).
template <typename T, typename SINK>
int dispatch_elem(const T* V, const SINK& out, int64_t outer, int64_t n, int64_t inner, int64_t bs,
                  const mxq_block_spec& q, hipStream_t st) {
  switch (q.elem) {
    case MXQ_ELEM_QTORCH: return launch_quant<T, MXQ_ELEM_QTORCH, -1>(V, out, outer, n, inner, bs, q, st);
    case MXQ_ELEM_OCP: return launch_mode<T, MXQ_ELEM_OCP>(V, out, outer, n, inner, bs, q, st);
    case MXQ_ELEM_MICROSOFT: return launch_mode<T, MXQ_ELEM_MICROSOFT>(V, out, outer, n, inner, bs, q, st);
    default: break;
  }
  if constexpr (SINK::kBytes == 4) {
    if (q.elem == MXQ_ELEM_IEEE) return launch_quant<T, MXQ_ELEM_IEEE, -1>(V, out, outer, n, inner, bs, q, st);
    return launch_quant<T, MXQ_ELEM_NONE, -1>(V, out, outer, n, inner, bs, q, st);
  } else {
    return mxq::invalid("mxq_block_quantize_packed: the element rule has no byte format");
  }
}

}  // namespace mxq_quant
