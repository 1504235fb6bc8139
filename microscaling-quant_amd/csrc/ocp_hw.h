// gfx950's conversions to and from the OCP element formats (V_CVT_SCALEF32_*, scale 1) as a fast form of the
// OCP element grid rounded to nearest even (ocp_code_t<MXQ_RNE> / ocp_grid_t<MXQ_RNE> in mxq_numerics.h).
//
// The conversions round to nearest even with true subnormals, and the FP6 and FP4 formats saturate, as the
// grid does.  They differ from it in three places: E4M3 rounds |z| >= 480 to NaN and E5M2 overflows to Inf
// instead of saturating, an exact -0 keeps its sign (the grid gives +0), and NaN and Inf are not the grid's
// pass-through.  So the callers use them only when every |z| of the wave is finite and below hw_ocp_limit,
// and add +0 first (-0 + 0 is +0; every other z is unchanged).  Measured equal on MI355X over 8.4 M float32
// values per format: every grid value, midpoint and their float32 neighbours, both signs, and random patterns
// with |z| < 8.
//
// FP6 packs 32 values into six words: V_CVT_SCALEF32_2XPK16 takes two vectors of 16 and interleaves them
// (field 2k from the first, 2k + 1 from the second), so the even elements go first and the odd second, and
// field k is element k.
#pragma once
#include <stdint.h>

namespace mxq_ocp_hw {

typedef float f16v __attribute__((ext_vector_type(16)));
typedef float f32v __attribute__((ext_vector_type(32)));
typedef unsigned u6v __attribute__((ext_vector_type(6)));
typedef short s2v __attribute__((ext_vector_type(2)));
typedef float f2v __attribute__((ext_vector_type(2)));

// The element formats with a conversion: E4M3, E5M2, E2M3, E3M2, E2M1.
__host__ __device__ inline bool has_hw(int e, int m) {
  return (e == 4 && m == 3) || (e == 5 && m == 2) || (e == 2 && m == 3) || (e == 3 && m == 2) || (e == 2 && m == 1);
}

// The formats whose conversion of N values a lane takes here: the FP6 forms convert 32 values at a time, whose
// register vectors are not worth it for fewer than 16 (a kernel converting fewer leaves FP6 to the grid).
template <int N>
__host__ __device__ inline bool has_hw_n(int e, int m) {
  return has_hw(e, m) && (N >= 16 || !((e == 2 && m == 3) || (e == 3 && m == 2)));
}

// The format's largest finite value, where the conversions saturate (E4M3 448, E5M2 57344, E2M3 7.5, E3M2 28,
// E2M1 6).  A grid clamped at another max_norm is not theirs, so the callers gate on max_norm equal to this.
__host__ __device__ inline float fmt_max(int e, int m) {
  if (e == 4 && m == 3) return 448.0f;
  if (e == 5 && m == 2) return 57344.0f;
  if (e == 2 && m == 3) return 7.5f;
  if (e == 3 && m == 2) return 28.0f;
  if (e == 2 && m == 1) return 6.0f;
  return 0.0f;
}

// |z| below this (and finite) converts as the grid rounds.
__host__ __device__ inline float hw_limit(int e, int m) {
  return (e == 4 && m == 3) ? 464.0f : ((e == 5 && m == 2) ? 57344.0f : 3.0e38f);
}

// The 32 fields of a six-word FP6 pack of N <= 32 values (even, odd split; zeros past N).
template <int N>
__device__ __forceinline__ void fp6_split(const float (&z)[N], f16v& even, f16v& odd) {
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    even[k] = 2 * k < N ? z[2 * k] + 0.0f : 0.0f;
    odd[k] = 2 * k + 1 < N ? z[2 * k + 1] + 0.0f : 0.0f;
  }
}

// The wide FP6 conversions, written so that their destination never shares a register with a source: the
// compiler's own allocation of __builtin_amdgcn_cvt_scalef32_2xpk16_{fp6,bf6}_f32 can place the six result
// words inside the sixteen source words (seen on gfx950 as corrupted fields wherever they overlapped); the
// early-clobber outputs ("=&v") rule that out.  Two wait states follow each, as after the compiler's own
// transcendental-class results, before anything reads them.
__device__ __forceinline__ u6v pack16x2(const f16v& even, const f16v& odd, bool e2m3) {
  u6v r;
  if (e2m3) asm("v_cvt_scalef32_2xpk16_fp6_f32 %0, %1, %2, 1.0\n\ts_nop 1" : "=&v"(r) : "v"(even), "v"(odd));
  else asm("v_cvt_scalef32_2xpk16_bf6_f32 %0, %1, %2, 1.0\n\ts_nop 1" : "=&v"(r) : "v"(even), "v"(odd));
  return r;
}
__device__ __forceinline__ f32v unpack32(const u6v& p, bool e2m3) {
  f32v r;
  if (e2m3) asm("v_cvt_scalef32_pk32_f32_fp6 %0, %1, 1.0\n\ts_nop 1" : "=&v"(r) : "v"(p));
  else asm("v_cvt_scalef32_pk32_f32_bf6 %0, %1, 1.0\n\ts_nop 1" : "=&v"(r) : "v"(p));
  return r;
}

__device__ __forceinline__ uint32_t field6(const u6v& p, int k) {
  const int bit = 6 * k, w = bit >> 5, off = bit & 31;
  uint32_t v = p[w] >> off;
  if (off > 26) v |= p[w + 1] << (32 - off);
  return v & 63u;
}

// The element codes of N values (N % 4 == 0, N <= 32), code j in byte j % 4 of w[j / 4]; FP6 for N >= 16 only
// (has_hw_n).
template <int N>
__device__ __forceinline__ void codes(const float (&z)[N], int e, int m, uint32_t (&w)[N / 4]) {
  static_assert(N % 4 == 0 && N <= 32, "N values in whole words");
  if (e == 4 || e == 5) {
#pragma unroll
    for (int q = 0; q < N / 4; ++q) {
      s2v r = {0, 0};
      if (e == 4) {
        r = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(r, z[4 * q] + 0.0f, z[4 * q + 1] + 0.0f, 1.0f, false);
        r = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(r, z[4 * q + 2] + 0.0f, z[4 * q + 3] + 0.0f, 1.0f, true);
      } else {
        r = __builtin_amdgcn_cvt_scalef32_pk_bf8_f32(r, z[4 * q] + 0.0f, z[4 * q + 1] + 0.0f, 1.0f, false);
        r = __builtin_amdgcn_cvt_scalef32_pk_bf8_f32(r, z[4 * q + 2] + 0.0f, z[4 * q + 3] + 0.0f, 1.0f, true);
      }
      w[q] = __builtin_bit_cast(uint32_t, r);
    }
  } else if (m == 1) {
#pragma unroll
    for (int q = 0; q < N / 4; ++q) {
      const uint32_t r =
          __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(0u, z[4 * q] + 0.0f, z[4 * q + 1] + 0.0f, 1.0f, 0) |
          (__builtin_amdgcn_cvt_scalef32_pk_fp4_f32(0u, z[4 * q + 2] + 0.0f, z[4 * q + 3] + 0.0f, 1.0f, 0) << 8);
      // nibbles n0 n1 | n2 n3 in the low two bytes -> one code a byte
      w[q] = (r & 0xFu) | ((r & 0xF0u) << 4) | ((r & 0xF00u) << 8) | ((r & 0xF000u) << 12);
    }
  } else if constexpr (N >= 16) {
    f16v even, odd;
    fp6_split<N>(z, even, odd);
    const u6v p = pack16x2(even, odd, e == 2);
#pragma unroll
    for (int q = 0; q < N / 4; ++q)
      w[q] = field6(p, 4 * q) | (field6(p, 4 * q + 1) << 8) | (field6(p, 4 * q + 2) << 16) | (field6(p, 4 * q + 3) << 24);
  }
}

// The grid values of N values (N even, N <= 32), in place: converted and converted back; FP6 for N >= 16 only
// (has_hw_n).
template <int N>
__device__ __forceinline__ void values(float (&z)[N], int e, int m) {
  static_assert(N % 2 == 0 && N <= 32, "N values in pairs");
  if (e == 4 || e == 5 || m == 1) {
#pragma unroll
    for (int q = 0; q < N / 2; ++q) {
      f2v r;
      if (e == 4) {
        const s2v c = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(s2v{0, 0}, z[2 * q] + 0.0f, z[2 * q + 1] + 0.0f, 1.0f, false);
        r = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(__builtin_bit_cast(uint32_t, c), 1.0f, false);
      } else if (e == 5) {
        const s2v c = __builtin_amdgcn_cvt_scalef32_pk_bf8_f32(s2v{0, 0}, z[2 * q] + 0.0f, z[2 * q + 1] + 0.0f, 1.0f, false);
        r = __builtin_amdgcn_cvt_scalef32_pk_f32_bf8(__builtin_bit_cast(uint32_t, c), 1.0f, false);
      } else {
        const uint32_t c = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(0u, z[2 * q] + 0.0f, z[2 * q + 1] + 0.0f, 1.0f, 0);
        r = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(c, 1.0f, 0);
      }
      z[2 * q] = r.x;
      z[2 * q + 1] = r.y;
    }
  } else if constexpr (N >= 16) {
    f16v even, odd;
    fp6_split<N>(z, even, odd);
    const f32v r = unpack32(pack16x2(even, odd, e == 2), e == 2);
#pragma unroll
    for (int k = 0; k < N; ++k) z[k] = r[k];
  }
}

}  // namespace mxq_ocp_hw
