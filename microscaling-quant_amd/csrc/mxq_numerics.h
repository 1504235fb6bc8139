// Bit-exact float primitives of the MX datapath, for gfx950 device code and (through a host build of this
// same header) for host-side tests.  Every function states the reference function it reproduces.
//
// Conventions
//   * Rounding modes follow mxq.rounding.MODES order: 0 ties_away, 1 rne, 2 truncate
//     (microxcaling names: nearest, even, floor).
//   * Grids follow mxq.element_quant.float_em.GRIDS order: 0 qtorch, 1 ieee, 2 ocp.
//   * Nothing here relies on FMA contraction or flush-to-zero: the library is compiled with
//     -ffp-contract=off and float32 denormals preserved, and every float operation below is an IEEE
//     operation whose rounding is the one the reference's torch CPU kernels perform.
#pragma once

#include <stdint.h>

#if defined(__HIPCC__) || defined(__HIP__)
#include <hip/hip_runtime.h>
#define MXQ_HD __host__ __device__ __forceinline__
#define MXQ_DEV __device__ __forceinline__
#else
#include <math.h>
#include <string.h>
#define MXQ_HD static inline
#define MXQ_DEV static inline
#endif

#include "log2_edges.inc"
#include "../../include/mxq_hip.h"

enum { MXQ_TIES_AWAY = 0, MXQ_RNE = 1, MXQ_TRUNC = 2 };
// microxcaling's "dither" (floor(|A| + u) with a uniform u per element): its element step only
enum { MXQ_DITHER = 3 };
enum { MXQ_GRID_QTORCH = 0, MXQ_GRID_IEEE = 1, MXQ_GRID_OCP = 2 };

#if defined(__HIP_DEVICE_COMPILE__)
static __constant__ uint32_t mxq_log2_edge_dev[277] = {MXQ_LOG2_EDGE_LIST};
#define MXQ_LOG2_EDGE(i) mxq_log2_edge_dev[(i)]
#else
static const uint32_t mxq_log2_edge_host[277] = {MXQ_LOG2_EDGE_LIST};
#define MXQ_LOG2_EDGE(i) mxq_log2_edge_host[(i)]
#endif

// ---------------------------------------------------------------------------------------------- bits
MXQ_HD uint32_t f2u(float f) { return __builtin_bit_cast(uint32_t, f); }
MXQ_HD float u2f(uint32_t u) { return __builtin_bit_cast(float, u); }
MXQ_HD uint64_t d2u(double d) { return __builtin_bit_cast(uint64_t, d); }
MXQ_HD double u2d(uint64_t u) { return __builtin_bit_cast(double, u); }
MXQ_HD int clz32(uint32_t x) { return __builtin_clz(x); }        // x != 0
MXQ_HD int clz64(uint64_t x) { return __builtin_clzll(x); }      // x != 0
MXQ_HD bool is_nan_f(float x) { return (f2u(x) & 0x7FFFFFFFu) > 0x7F800000u; }
MXQ_HD bool is_finite_f(float x) { return (f2u(x) & 0x7F800000u) != 0x7F800000u; }
MXQ_HD bool is_nan_d(double x) { return (d2u(x) & 0x7FFFFFFFFFFFFFFFull) > 0x7FF0000000000000ull; }
MXQ_HD float copysign_f(float mag, float sgn) { return u2f((f2u(mag) & 0x7FFFFFFFu) | (f2u(sgn) & 0x80000000u)); }
MXQ_HD double copysign_d(double mag, double sgn) {
  return u2d((d2u(mag) & 0x7FFFFFFFFFFFFFFFull) | (d2u(sgn) & 0x8000000000000000ull));
}
MXQ_HD float f_inf() { return u2f(0x7F800000u); }
// NaN payloads are not part of the datapath's spec: a NaN produced by arithmetic is replaced by the canonical
// quiet NaN 0x7FC00000 before any rounding that reads a NaN's bits (the qtorch grid carries a large payload
// into the exponent and sign; x86 and CUDA propagate different payloads, so the reference itself differs there).
MXQ_HD float canon_nan(float x) { return ((__builtin_bit_cast(uint32_t, x) & 0x7FFFFFFFu) > 0x7F800000u) ? __builtin_bit_cast(float, 0x7FC00000u) : x; }
MXQ_HD float f_nan() { return u2f(0x7FC00000u); }
MXQ_HD double d_inf() { return u2d(0x7FF0000000000000ull); }
// 2^k as float32 for k in [-149, 127] (exact, subnormal included); 0 below, Inf above.
MXQ_HD float pow2f(int k) {
  if (k > 127) return f_inf();
  if (k >= -126) return u2f((uint32_t)(k + 127) << 23);
  if (k >= -149) return u2f(1u << (k + 149));
  return 0.0f;
}
// 2^k as float64 for k in [-1074, 1023].
MXQ_HD double pow2d(int k) {
  if (k > 1023) return d_inf();
  if (k >= -1022) return u2d((uint64_t)(k + 1023) << 52);
  if (k >= -1074) return u2d(1ull << (k + 1074));
  return 0.0;
}
// Multiply by 2^k exactly: mathematically the value v * 2^k, rounded once (used only where exact).
MXQ_HD float scale_pow2f(float v, int k) {
  // split so that no intermediate under- or overflows when the final value is representable
  while (k > 127) { v = v * pow2f(127); k -= 127; }
  while (k < -126) { v = v * pow2f(-126); k += 126; }
  return v * pow2f(k);
}

// ------------------------------------------------------------------------------------- rounding.round_bits
// mxq/rounding/__init__.py:34-55 with rne.py:6-8, ties_away.py:5-6, truncate.py:5-6: keep `keep` fraction bits
// of a float32 bit pattern (keep in [0, 22]); a carry runs into the exponent; arithmetic wraps at 2^32.
MXQ_HD uint32_t round_bits32(uint32_t bits, int keep, int mode) {
  const int drop = 23 - keep;
  const uint32_t mask = (1u << drop) - 1u, half = 1u << (drop - 1);
  if (mode == MXQ_TIES_AWAY) return (bits + half) & ~mask;
  if (mode == MXQ_RNE) return (bits + (half - 1u) + ((bits >> drop) & 1u)) & ~mask;
  return bits & ~mask;
}

// The same with the mode fixed at compile time.
template <int MODE>
MXQ_HD uint32_t round_bits32_t(uint32_t bits, int keep) {
  const int drop = 23 - keep;
  const uint32_t mask = (1u << drop) - 1u, half = 1u << (drop - 1);
  if constexpr (MODE == MXQ_TIES_AWAY) return (bits + half) & ~mask;
  else if constexpr (MODE == MXQ_RNE) return (bits + (half - 1u) + ((bits >> drop) & 1u)) & ~mask;
  else return bits & ~mask;
}

// mxq/rounding/__init__.py:64-85 `bf16`: bit RNE at 7 fraction bits, NaN passes unchanged.
MXQ_HD float bf16_rne(float x) {
  if (is_nan_f(x)) return x;
  return u2f(round_bits32(f2u(x), 7, MXQ_RNE));
}

// --------------------------------------------------------------------------------------- floor(log2 x)
// floor(torch.log2(x)) for a positive finite float32 x: the exponent of x, plus one where the correctly
// rounded log2 reaches the next integer (table generated by gen_log2_edges.py).
MXQ_HD int floor_log2_pos(float x) {
  const uint32_t u = f2u(x);
  const int E = (u >= 0x00800000u) ? (int)(u >> 23) - 127 : (31 - clz32(u)) - 149;
  return E + (u >= MXQ_LOG2_EDGE(E + 149) ? 1 : 0);
}

// 2^floor(log2(a)) in float32 as torch computes pow(2, floor(log2(a))): NaN for NaN or a < 0,
// Inf for +Inf, 0 for +-0 (log2 -> -inf).
MXQ_HD float pow2_floor_log2(float a) {
  if (is_nan_f(a) || a < 0.0f) return f_nan();
  if (a == 0.0f) return 0.0f;
  if (!is_finite_f(a)) return f_inf();
  return pow2f(floor_log2_pos(a));
}

// ------------------------------------------------------------------------------ integer rounding helpers
// round(sig / 2^sh) for sig < 2^24, sh >= 1, in the reference's round_int semantics evaluated in float32:
// ties_away = floor(fl32(k + 0.5)) (mxq/rounding/ties_away.py:9-10), rne = torch.round (rne.py:11-12),
// truncate = trunc.  fl32(k + 0.5) differs from k + 0.5 only for k = 0.5 - 2^-25, where it rounds to 1.0.
MXQ_HD uint32_t shift_round32(uint32_t sig, int sh, int mode) {
  if (sh >= 26) return 0u;
  if (sh == 25) return (mode == MXQ_TIES_AWAY && sig == 0xFFFFFFu) ? 1u : 0u;
  const uint32_t q = sig >> sh, rem = sig & ((1u << sh) - 1u), half = 1u << (sh - 1);
  if (mode == MXQ_TIES_AWAY) return q + (rem >= half ? 1u : 0u);
  if (mode == MXQ_RNE) return q + ((rem > half || (rem == half && (q & 1u))) ? 1u : 0u);
  return q;
}
// The same for a 53-bit significand evaluated in float64 (artifact at k = 0.5 - 2^-54).
MXQ_HD uint64_t shift_round64(uint64_t sig, int sh, int mode) {
  if (sh >= 55) return 0ull;
  if (sh == 54) return (mode == MXQ_TIES_AWAY && sig == 0x1FFFFFFFFFFFFFull) ? 1ull : 0ull;
  const uint64_t q = sig >> sh, rem = sig & ((1ull << sh) - 1ull), half = 1ull << (sh - 1);
  if (mode == MXQ_TIES_AWAY) return q + (rem >= half ? 1ull : 0ull);
  if (mode == MXQ_RNE) return q + ((rem > half || (rem == half && (q & 1ull))) ? 1ull : 0ull);
  return q;
}

MXQ_HD int f_bias(int e) { return (1 << (e - 1)) - 1; }

// Decompose a finite nonzero float32 magnitude into sig * 2^lsb_exp with the unbiased exponent E of its
// leading bit (subnormals normalised, as torch.frexp does).
MXQ_HD void decompose32(uint32_t a, uint32_t& sig, int& E, int& lsb_exp) {
  const int be = (int)(a >> 23);
  if (be) { sig = (a & 0x7FFFFFu) | 0x800000u; E = be - 127; lsb_exp = be - 150; }
  else { sig = a; lsb_exp = -149; E = (31 - clz32(a)) - 149; }
}
MXQ_HD void decompose64(uint64_t a, uint64_t& sig, int& E, int& lsb_exp) {
  const int be = (int)(a >> 52);
  if (be) { sig = (a & 0xFFFFFFFFFFFFFull) | 0x10000000000000ull; E = be - 1023; lsb_exp = be - 1075; }
  else { sig = a; lsb_exp = -1074; E = (63 - clz64(a)) - 1074; }
}

// k * 2^q as float32, or +Inf when it reaches 2^(emax + 1).  k < 2^25, and the value, when below the overflow
// bound, lies on a float(e <= 8, m <= 23) grid, so it is a float32.
MXQ_HD float compose_grid(uint32_t k, int q, int emax) {
  if (k == 0u) return 0.0f;
  const int top = (31 - clz32(k)) + q;
  if (top >= emax + 1) return f_inf();
  return scale_pow2f((float)k, q);
}
MXQ_HD float compose_grid64(uint64_t k, int q, int emax) {
  if (k == 0ull) return 0.0f;
  const int top = (63 - clz64(k)) + q;
  if (top >= emax + 1) return f_inf();
  return (float)((double)k * pow2d(q));
}

// ------------------------------------------------------------------------------------- float_em grids
// mxq/element_quant/float_em.py:53-73 `_qtorch`: round the float32 bits at m, then clip the exponent to
// [127 - L, 127 + L]; above saturates to +-max, below goes to +-2^-L when above 2^(-L-1), else +0.
MXQ_HD float qtorch_round(float z, int e, int m, int mode) {
  const uint32_t bits = f2u(z);
  uint32_t q = round_bits32(bits, m, mode);
  const uint32_t L = (uint32_t)f_bias(e), min_store = 127u - L, max_store = 127u + L;
  const uint32_t exp_store = (q >> 23) & 0xFFu, sign = bits & 0x80000000u;
  if (exp_store > max_store) {
    q = sign | (max_store << 23) | (0x007FFFFFu & ~((1u << (23 - m)) - 1u));
  } else if (exp_store < min_store) {
    const uint32_t q_mag = q & 0x7FFFFFFFu, middle = (min_store - 1u) << 23;
    q = (q_mag > middle) ? (sign | (min_store << 23)) : 0u;
  }
  return u2f(q);
}

// mxq/element_quant/float_em.py:76-99 `_ieee` on a float32 input: step 2^(max(E, emin) - m), k = round(|x|/step),
// overflow at 2^(emax+1) -> Inf, NaN/Inf/+-0 pass, underflow -> +0 (e < 8) or signed zero (e = 8, float64 path).
MXQ_HD float ieee_round32(float x, int e, int m, int mode) {
  const uint32_t u = f2u(x), a = u & 0x7FFFFFFFu;
  if (a == 0u || a >= 0x7F800000u) return x;
  uint32_t sig; int E, lsb;
  decompose32(a, sig, E, lsb);
  const int b = f_bias(e), emin = 1 - b, emax = b;
  const int q = (E > emin ? E : emin) - m;
  const int sh = q - lsb;
  // e = 8 evaluates in float64, where k + 0.5 is exact: no ties_away artifact (mode stays, sh path same)
  uint32_t k;
  if (sh <= 0) k = sig << (-sh);     // m = 23 on the float32 grid: exact
  else if (e == 8 && sh == 25) k = 0u;
  else k = shift_round32(sig, sh, mode);
  const float val = compose_grid(k, q, emax);
  if (val == 0.0f) return (e < 8) ? 0.0f : copysign_f(0.0f, x);
  return copysign_f(val, x);
}

// `_ieee` on a float64 input (exact_add's float64 path and float64 tensors): the same rule in float64.
MXQ_HD float ieee_round64(double x, int e, int m, int mode) {
  const uint64_t u = d2u(x), a = u & 0x7FFFFFFFFFFFFFFFull;
  if (a == 0ull || a >= 0x7FF0000000000000ull) return (float)x;
  uint64_t sig; int E, lsb;
  decompose64(a, sig, E, lsb);
  const int b = f_bias(e), emin = 1 - b, emax = b;
  const int q = (E > emin ? E : emin) - m;
  const int sh = q - lsb;
  uint64_t k = (sh <= 0) ? (sig << (-sh)) : shift_round64(sig, sh, mode);
  const float val = compose_grid64(k, q, emax);
  const float sx = (u >> 63) ? -1.0f : 1.0f;
  if (val == 0.0f) return (e < 8) ? 0.0f : copysign_f(0.0f, sx);
  return copysign_f(val, sx);
}

// mxq/element_quant/float_em.py:102-123 `_ocp` on a float32 input: ieee's step, clamp at max_norm, exact +-0 -> +0,
// a negative value that rounds to zero -> -0, Inf/NaN pass.
MXQ_HD float ocp_round32(float x, int e, int m, int mode, float max_norm) {
  const uint32_t u = f2u(x), a = u & 0x7FFFFFFFu;
  if (a == 0u) return 0.0f;
  if (a >= 0x7F800000u) return x;
  uint32_t sig; int E, lsb;
  decompose32(a, sig, E, lsb);
  const int emin = 1 - f_bias(e);
  const int q = (E > emin ? E : emin) - m;
  const uint32_t k = shift_round32(sig, q - lsb, mode);
  float val = compose_grid(k, q, 1000);      // the ocp formats never overflow float32 before the clamp
  if (val > max_norm) val = max_norm;
  return copysign_f(val, x);
}
MXQ_HD float ocp_round64(double x, int e, int m, int mode, float max_norm) {
  const uint64_t u = d2u(x), a = u & 0x7FFFFFFFFFFFFFFFull;
  if (a == 0ull) return 0.0f;
  if (a >= 0x7FF0000000000000ull) return (float)x;
  uint64_t sig; int E, lsb;
  decompose64(a, sig, E, lsb);
  const int emin = 1 - f_bias(e);
  const int q = (E > emin ? E : emin) - m;
  const uint64_t k = shift_round64(sig, q - lsb, mode);
  float val = compose_grid64(k, q, 1000);
  if (val > max_norm) val = max_norm;
  return copysign_f(val, (u >> 63) ? -1.0f : 1.0f);
}

// mxq/element_quant/float_em.py:39-50 `quantize` for a float32 input with validated (e, m, mode, grid).
MXQ_HD float float_em_quantize32(float z, int e, int m, int mode, int grid, float max_norm) {
  if (e == 8 && m == 23) return z;
  if (grid == MXQ_GRID_QTORCH) return qtorch_round(z, e, m, mode);
  if (grid == MXQ_GRID_IEEE) return ieee_round32(z, e, m, mode);
  return ocp_round32(z, e, m, mode, max_norm);
}
// ... and for a float64 input: qtorch converts to float32 first; ieee/ocp round from float64.
MXQ_HD float float_em_quantize64(double z, int e, int m, int mode, int grid, float max_norm) {
  if (e == 8 && m == 23) return ieee_round64(z, 8, 23, mode);
  if (grid == MXQ_GRID_QTORCH) return qtorch_round((float)z, e, m, mode);
  if (grid == MXQ_GRID_IEEE) return ieee_round64(z, e, m, mode);
  return ocp_round64(z, e, m, mode, max_norm);
}

// ---------------------------------------------------------------------------- microxcaling element step
// mxq/microxcaling/elemwise.py:63-151 `_quantize_elemwise_core` with `_round_mantissa` (:29-60), for a float32 A,
// float exponent format (exp_bits > 0), allow_denorm=True.  The float32 operations are the reference's, in its
// order: private_exp = floor(log2(|A| + (A == 0))) clipped at min_exp; out = A / 2^pe * 2^(bits-2); round;
// out / 2^(bits-2) * 2^pe; saturate (clamp) or overflow to Inf; +-Inf inputs restored.
template <int MODE>
MXQ_HD float ms_round_mantissa_t(float A, float u = 0.0f) {
  const float absA = fabsf(A);
  const float sgn = (A > 0.0f) ? 1.0f : ((A < 0.0f) ? -1.0f : 0.0f);   // torch.sign (0 for NaN and +-0)
  if constexpr (MODE == MXQ_TRUNC) {
    return sgn * floorf(absA);
  } else if constexpr (MODE == MXQ_DITHER) {
    return sgn * floorf(absA + u);                   // u: the element's draw of torch.rand_like, in [0, 1)
  } else if constexpr (MODE == MXQ_TIES_AWAY) {
    return sgn * floorf(absA + 0.5f);
  } else {
    // "even": (absA - 0.5) % 2 == 0 subtracts one.  torch.remainder(t, 2) is 0 exactly when t is an even
    // integer, i.e. when t / 2 (exact: t is a multiple of 2^-25 here) is an integer.
    const float t = absA - 0.5f;
    const float h = t * 0.5f;
    const float maskA = (floorf(h) == h) ? 1.0f : 0.0f;
    return sgn * (floorf(absA + 0.5f) - maskA);
  }
}

template <int MODE>
MXQ_HD float microsoft_quantize_t(float A, int ebits, int mbits, float max_norm, bool saturate, float u = 0.0f) {
  const uint32_t ua = f2u(A), aa = ua & 0x7FFFFFFFu;
  if (aa >= 0x7F800000u) return A;                       // NaN stays NaN; +-Inf is restored at the end
  const int min_exp = -(1 << (ebits - 1)) + 2;
  int pe = (aa == 0u) ? 0 : floor_log2_pos(u2f(aa));
  if (pe < min_exp) pe = min_exp;
  // A / 2^pe and x / 2^(bits-2) as products with the exact reciprocal powers of two: the same correctly
  // rounded values as the reference's divisions while 2^pe is finite (pe <= 127).  pe = 128 (the log2
  // round-up band below FLT_MAX) makes 2^pe = Inf and the reference's A / Inf = 0 then 0 * Inf = NaN.
  const float p2 = pow2f(pe);                            // 2 ** private_exp, exact or Inf
  float out = (pe <= 127) ? A * pow2f(-pe) : A / p2;
  out = out * (float)(1 << (mbits - 2));
  out = ms_round_mantissa_t<MODE>(out, u);
  out = out * pow2f(2 - mbits);
  out = out * p2;
  if (saturate) {
    if (is_nan_f(out)) return out;
    if (out > max_norm) out = max_norm;
    if (out < -max_norm) out = -max_norm;
  } else if (fabsf(out) > max_norm) {
    out = (out > 0.0f) ? f_inf() : -f_inf();
  }
  return out;
}

MXQ_HD float ms_round_mantissa(float A, int mode) {
  if (mode == MXQ_TRUNC) return ms_round_mantissa_t<MXQ_TRUNC>(A);
  if (mode == MXQ_TIES_AWAY) return ms_round_mantissa_t<MXQ_TIES_AWAY>(A);
  return ms_round_mantissa_t<MXQ_RNE>(A);
}

MXQ_HD float microsoft_quantize(float A, int ebits, int mbits, float max_norm, int mode, bool saturate) {
  if (mode == MXQ_TRUNC) return microsoft_quantize_t<MXQ_TRUNC>(A, ebits, mbits, max_norm, saturate);
  if (mode == MXQ_TIES_AWAY) return microsoft_quantize_t<MXQ_TIES_AWAY>(A, ebits, mbits, max_norm, saturate);
  return microsoft_quantize_t<MXQ_RNE>(A, ebits, mbits, max_norm, saturate);
}

// ---------------------------------------------------------------------------------------- scale factors
// mxq/scale_factor.py:40-44 `mxquant`: 2^floor(log2(max(amax, floor))), then clamp(min=floor). floor is the
// float32 value of the Python float (1e-38 is a float32 subnormal).
MXQ_HD float scale_mxquant(float amax, float floor_) {
  float a = amax;
  if (!is_nan_f(a) && a < floor_) a = floor_;
  float sc = pow2_floor_log2(a);
  if (!is_nan_f(sc) && sc < floor_) sc = floor_;
  return sc;
}

// mxq/scale_factor.py:47-59 `ocp`: shared = floor(log2(amax + 2^-126 [amax == 0])) - emax, NaN above the E8M0 max,
// clamped at -(2^(scale_bits-1) - 1); X = 2^shared.
MXQ_HD float scale_ocp(float amax, int emax, int scale_bits) {
  const float a = (amax == 0.0f) ? pow2f(-126) : amax;
  if (is_nan_f(a) || a < 0.0f) return f_nan();
  if (!is_finite_f(a)) return f_nan();                  // +Inf - emax > scale_emax
  const int scale_emax = (1 << (scale_bits - 1)) - 1;
  int s = floor_log2_pos(a) - emax;
  if (s > scale_emax) return f_nan();
  if (s < -scale_emax) s = -scale_emax;
  return pow2f(s);
}

// mxq/scale_factor.py:68-81 `ocp_no_clip`: ocp's X, doubled where microsoft(amax / X) without saturation is Inf.
// Mode MXQ_DITHER rounds with u, the block's draw.
MXQ_HD float scale_ocp_no_clip(float amax, int emax, int scale_bits, int ebits, int mbits, float max_norm, int mode,
                               float u = 0.0f) {
  const float X = scale_ocp(amax, emax, scale_bits);
  const float r = mode == MXQ_DITHER ? microsoft_quantize_t<MXQ_DITHER>(amax / X, ebits, mbits, max_norm, false, u)
                                     : microsoft_quantize(amax / X, ebits, mbits, max_norm, mode, false);
  const bool inf = (f2u(r) & 0x7FFFFFFFu) == 0x7F800000u;
  return inf ? X * 2.0f : X;
}

// ------------------------------------------------------------------------------------------------ arith
// mxq/arith.py:106-117 `truncate_significand`: keep m fraction bits of |x|'s significand (subnormals normalised),
// toward zero; zeros, Inf and NaN pass.
MXQ_HD float truncate_significand(float x, int m) {
  const uint32_t u = f2u(x), a = u & 0x7FFFFFFFu;
  if (a == 0u || a >= 0x7F800000u) return x;
  const int lead = (a >= 0x00800000u) ? 23 : 31 - clz32(a);      // bit of the leading 1 in the pattern
  const int drop = lead - m;
  if (drop <= 0) return x;
  return u2f(u & ~((1u << drop) - 1u));
}

// mxq/arith.py:120-124 `flush_product`: |x| < thr -> +0 (thr = float32(2^floor_exp)).
MXQ_HD float flush_product(float x, float thr) { return (fabsf(x) < thr) ? 0.0f : x; }

// mxq/arith.py:127-137 `saturate`: sign(x) * (|x| > limit ? value : |x|), with torch.sign (0 for +-0 and NaN).
MXQ_HD float saturate(float x, float limit, float value) {
  const float ax = fabsf(x);
  const float s = (x > 0.0f) ? 1.0f : ((x < 0.0f) ? -1.0f : 0.0f);
  return s * ((ax > limit) ? value : ax);
}

// mxq/arith.py:21-30
MXQ_HD bool fits_float32(int e, int m) { return (1 << e) - 1 + m <= 24; }

// mxq/arith.py:33-38 Knuth's TwoSum in float32.
MXQ_HD void two_sum(float a, float b, float& s, float& t) {
  s = a + b;
  const float bb = s - a;
  t = (a - (s - bb)) + (b - bb);
}

// mxq/arith.py:41-65 `_round_pair`: s + t (exact, |t| <= ulp(s)/2) rounded to float(e <= 7, m <= 22), RNE, with t
// deciding an exact midpoint of s; overflow -> Inf; NaN/Inf/+-0 pass; underflow -> +0.
MXQ_HD float round_pair(float s, float t, int e, int m) {
  const uint32_t u = f2u(s), a = u & 0x7FFFFFFFu;
  if (a == 0u || a >= 0x7F800000u) return s;
  uint32_t sig; int E, lsb;
  decompose32(a, sig, E, lsb);
  const int b = f_bias(e), emin = 1 - b, emax = b;
  const int q = (E > emin ? E : emin) - m;
  const int sh = q - lsb;                           // >= 1
  uint32_t k;
  if (sh >= 26) {
    k = 0u;
  } else {
    const uint32_t kf = sig >> sh, rem = sig & ((1u << sh) - 1u), half = 1u << (sh - 1);
    const bool tie = (sh <= 24) && (rem == half);
    if (tie && t != 0.0f) {
      const bool up = ((s > 0.0f) ? t : -t) > 0.0f;
      k = up ? kf + 1u : kf;
    } else {
      k = shift_round32(sig, sh, MXQ_RNE);
    }
  }
  const float val = compose_grid(k, q, emax);
  if (val == 0.0f) return 0.0f;
  return copysign_f(val, s);
}

// mxq/arith.py:68-103 `exact_add`: a + b exactly, rounded once to float(e, m); a zero addend returns the other.
// The three paths are the reference's, chosen on (e, m, mode, grid) alone.
MXQ_HD float exact_add(float a, float b, int e, int m, int mode, int grid, float max_norm) {
  if (mode == MXQ_RNE && grid == MXQ_GRID_IEEE && fits_float32(e, m)) {
    if (a == 0.0f) return b;
    if (b == 0.0f) return a;
    return ieee_round32(a + b, e, m, MXQ_RNE);
  }
  if (mode == MXQ_RNE && grid == MXQ_GRID_IEEE && e <= 7) {
    if (a == 0.0f) return b;
    if (b == 0.0f) return a;
    float s, t;
    two_sum(a, b, s, t);
    return round_pair(s, t, e, m);
  }
  if (a == 0.0f) return b;
  if (b == 0.0f) return a;
  return float_em_quantize64((double)a + (double)b, e, m, mode, grid, max_norm);
}

// ------------------------------------------------------------------------------ Arithmetic stages
// mxq/matmul/_arithmetic.py:105-108 `_unsigned_zero`
MXQ_HD float unsigned_zero(float x) { return (x == 0.0f) ? 0.0f : x; }

// mxq/matmul/_arithmetic.py:125-127 MXGEMMINI lane: rne to float(e, m) (bf16 by bits for (8, 7)), then +0.
MXQ_HD float mxg_lane(float x, int e, int m) {
  float r;
  if (e == 8 && m == 7) r = bf16_rne(x);
  else if (e == 8 && m == 23) r = x;
  else r = ieee_round32(x, e, m, MXQ_RNE);
  return unsigned_zero(r);
}

// exact_add of two lane values of a bf16 (8, 7) or float32 (8, 23) lane.  Both operands already sit on the
// lane's grid, so the float32 sum rounded to the lane is the exact sum rounded once: for (8, 23) the float32 add
// is that rounding; for bf16 a float32 add then RNE to 8 significant bits is a double rounding that cannot
// differ from one (24 >= 2 * 8 + 1), bf16 subnormal sums are exact in float32, and overflow goes to Inf either
// way.  Zeros short-circuit as exact_add's do.
MXQ_HD float wide_lane_add(float a, float b, int m) {
  if (a == 0.0f) return b;
  if (b == 0.0f) return a;
  const float s = a + b;
  return m == 7 ? bf16_rne(s) : s;
}

// MXGEMMINI acc_add (mxq/matmul/_arithmetic.py:132) and tile_add (:133).
MXQ_HD float mxg_acc_add(float S, float p, int e, int m) {
  if (e == 8 && (m == 7 || m == 23)) return wide_lane_add(mxg_lane(S, e, m), mxg_lane(p, e, m), m);
  return exact_add(mxg_lane(S, e, m), mxg_lane(p, e, m), e, m, MXQ_RNE, MXQ_GRID_IEEE, 0.0f);
}
MXQ_HD float mxg_tile_add(float C, float tile) {
  return wide_lane_add(mxg_lane(C, 8, 7), mxg_lane(tile, 8, 7), 7);
}
// MXGEMMINI product (mxq/matmul/_arithmetic.py:131): saturate(flush(truncate(a * b, prod_m))).
MXQ_HD float mxg_product(float a, float b, int prod_m, bool do_flush, float flush_thr, float limit, float value) {
  float t = truncate_significand(a * b, prod_m);
  if (do_flush) t = flush_product(t, flush_thr);
  return saturate(t, limit, value);
}

// MXQUANT (mxq/matmul/_arithmetic.py:64-73): qtorch ties_away on the product and on the fp32 lane sum.
MXQ_HD float mxq_q(float x, int e, int m) {
  if (e == 8 && m == 23) return x;
  return qtorch_round(canon_nan(x), e, m, MXQ_TIES_AWAY);
}

// ------------------------------------------------------------------------------ block quantization steps
// torch.amax: NaN propagates.
MXQ_HD float amax_combine(float a, float b) { return (is_nan_f(a) || a > b) ? a : b; }

MXQ_HD float block_scale(float amax, const mxq_block_spec& s) {
  if (s.scale_rule == MXQ_SCALE_MXQUANT) return scale_mxquant(amax, s.scale_floor);
  if (s.scale_rule == MXQ_SCALE_OCP) return scale_ocp(amax, s.scale_emax, s.scale_bits);
  if (s.scale_rule == MXQ_SCALE_OCP_NO_CLIP)
    return scale_ocp_no_clip(amax, s.scale_emax, s.scale_bits, s.e, s.m, s.max_norm, s.rounding);
  return 1.0f;
}

// z = v / X.  `inv` is 1/X when X is a normal power of two (exact), else 0 to request the division.
struct Div {
  float X, inv;
};
// inv: the reciprocal of a positive normal power of two 2^(be - 127), exact, from its bits: 2^(127 - be), normal
// for be <= 253 and the subnormal 2^-127 for be = 254 (what 1.0f / X gives, without the division's sequence);
// 0 for any other X.
MXQ_HD Div make_div(float X) {
  const uint32_t u = f2u(X), be = (u >> 23) & 0xFFu;
  const bool p2 = (u & 0x807FFFFFu) == 0u && be >= 1u && be <= 254u;
  const uint32_t ib = be <= 253u ? (254u - be) << 23 : 0x00400000u;
  return Div{X, p2 ? u2f(ib) : 0.0f};
}
MXQ_HD float apply_div(float v, const Div& d) { return d.inv != 0.0f ? v * d.inv : v / d.X; }

// The OCP element grid (float_em.py:102-123) for e <= 5, m <= 3 on a float32 z, both paths computed and one
// selected.  At or above the format's min normal: the significand rounded at m fraction bits on the bit
// pattern (the carry runs into the exponent).  Below it: k = round(|z| / step) evaluated in float32 exactly as
// round_int does (ties_away adds 0.5 in float32), times the step.  Then the max_norm clamp and the sign;
// an exact +-0 gives +0, Inf and NaN pass.
template <int MODE>
MXQ_HD float ocp_grid_t(float z, int e, int m, float max_norm) {
  const uint32_t u = f2u(z), a = u & 0x7FFFFFFFu;
  const int emin = 2 - (1 << (e - 1));
  const uint32_t rn = round_bits32_t<MODE>(a, m);
  const float k = u2f(a) * pow2f(m - emin);
  float r;
  if constexpr (MODE == MXQ_RNE) r = rintf(k);
  else if constexpr (MODE == MXQ_TIES_AWAY) r = floorf(k + 0.5f);
  else r = truncf(k);
  const float rs = r * pow2f(emin - m);
  float mag = (a >= ((uint32_t)(emin + 127) << 23)) ? u2f(rn) : rs;
  mag = (mag > max_norm) ? max_norm : mag;
  const float out = (a == 0u) ? 0.0f : copysign_f(mag, z);
  return (a >= 0x7F800000u) ? z : out;
}

// ocp_grid_t's result as its element code (mx_encode's layout), from the same two roundings: the rounded
// significand bits (normal: bits >> (23 - m), less the float32-to-format exponent bias difference) or the
// rounded multiple of the subnormal step (whose 2^m is the code of the smallest normal), clamped at the
// largest finite code `maxcode` as the grid clamps at max_norm.  An exact +-0 is +0, a value rounded to 0 keeps
// its sign.  *good is cleared for Inf and NaN, which the grid passes through and mx_encode takes.
template <int MODE>
MXQ_HD uint32_t ocp_code_t(float z, int e, int m, uint32_t maxcode, bool* good) {
  const uint32_t u = f2u(z), a = u & 0x7FFFFFFFu;
  const int emin = 2 - (1 << (e - 1));
  const uint32_t rn = round_bits32_t<MODE>(a, m);
  const float k = u2f(a) * pow2f(m - emin);
  float r;
  if constexpr (MODE == MXQ_RNE) r = rintf(k);
  else if constexpr (MODE == MXQ_TIES_AWAY) r = floorf(k + 0.5f);
  else r = truncf(k);
  const uint32_t nsub = (uint32_t)(128 - (1 << (e - 1))) << m;
  const uint32_t cn = (rn >> (23 - m)) - nsub;
  uint32_t mag = (a >= ((uint32_t)(emin + 127) << 23)) ? cn : (uint32_t)(int)r;
  mag = mag < maxcode ? mag : maxcode;
  *good = a < 0x7F800000u;
  return (a == 0u) ? 0u : (mag | ((u >> 31) << (e + m)));
}

MXQ_HD float ocp_grid_fast(float z, int e, int m, int mode, float max_norm) {
  if (mode == MXQ_RNE) return ocp_grid_t<MXQ_RNE>(z, e, m, max_norm);
  if (mode == MXQ_TIES_AWAY) return ocp_grid_t<MXQ_TIES_AWAY>(z, e, m, max_norm);
  return ocp_grid_t<MXQ_TRUNC>(z, e, m, max_norm);
}

// Step 2 of a block spec.  MODE >= 0 fixes the rounding mode at compile time; MODE < 0 reads s.rounding.
template <int ELEM, int MODE>
MXQ_HD float elem_qm(float z, const mxq_block_spec& s) {
  if constexpr (ELEM == MXQ_ELEM_QTORCH) {
    // a NaN made by the division is taken as the canonical quiet NaN before the bit rounding
    return (s.e == 8 && s.m == 23) ? z : qtorch_round(canon_nan(z), s.e, s.m, s.rounding);
  } else if constexpr (ELEM == MXQ_ELEM_IEEE) {
    return float_em_quantize32(z, s.e, s.m, s.rounding, MXQ_GRID_IEEE, 0.0f);
  } else if constexpr (ELEM == MXQ_ELEM_OCP) {
    if (s.via_e) z = float_em_quantize32(z, s.via_e, s.via_m, s.rounding, MXQ_GRID_IEEE, 0.0f);
    if constexpr (MODE < 0) return ocp_grid_fast(z, s.e, s.m, s.rounding, s.max_norm);
    else return ocp_grid_t<MODE>(z, s.e, s.m, s.max_norm);
  } else if constexpr (ELEM == MXQ_ELEM_MICROSOFT) {
    if constexpr (MODE < 0) return microsoft_quantize(z, s.e, s.m, s.max_norm, s.rounding, true);
    else return microsoft_quantize_t<MODE>(z, s.e, s.m, s.max_norm, true);
  } else {
    return z;
  }
}

template <int ELEM>
MXQ_HD float elem_q(float z, const mxq_block_spec& s) { return elem_qm<ELEM, -1>(z, s); }


// ----------------------------------------------------------------------------------- packed byte codes
// Element codes in the OCP MX layout (OCP Microscaling Formats v1.0): sign | e exponent bits | m mantissa bits,
// bias 2^(e-1) - 1, low bits of a byte.  For every finite value of the format this is the numbering of the
// reference's element codes (mxq/lut/formats.py:87-99).  Specials: E5M2 keeps IEEE Inf (exponent all ones,
// mantissa 0) and NaN (0x7F); E4M3's only special is NaN, S.1111.111 (so 480, its code in MX-Gemmini's
// decoders, is not a value here); FP6 and FP4 have none.
//
// The code of a float32 value q; *ok is cleared when q is not exactly a value of the format (off its grid,
// beyond its range, or a special it lacks).  -0 keeps its sign bit.
MXQ_HD uint32_t mx_encode(float q, int e, int m, bool* ok) {
  const uint32_t u = f2u(q), a = u & 0x7FFFFFFFu;
  const uint32_t sbit = (u >> 31) << (e + m);
  const bool e4m3 = e == 4 && m == 3, e5m2 = e == 5 && m == 2;
  if (a == 0u) return sbit;
  if (a >= 0x7F800000u) {                                         // Inf or NaN
    if (e5m2) return sbit | (a == 0x7F800000u ? 0x7Cu : 0x7Fu);
    if (e4m3 && a > 0x7F800000u) return sbit | 0x7Fu;
    *ok = false;
    return 0u;
  }
  const int bias = (1 << (e - 1)) - 1, emin = 1 - bias;
  const int E = (int)(a >> 23) - 127;                              // -127 for a float32 subnormal
  const uint32_t sig = (a & 0x7FFFFFu) | (E > -127 ? 0x800000u : 0u);   // 24-bit significand of a normal
  uint32_t code;
  if (E >= emin) {
    if (a & ((1u << (23 - m)) - 1u)) *ok = false;                  // more than m fraction bits
    const int be = E + bias;
    code = ((uint32_t)be << m) | ((a >> (23 - m)) & ((1u << m) - 1u));
    const int emax_field = (1 << e) - 1;
    if (be > emax_field || (e5m2 && be == emax_field) || (e4m3 && code == 0x7Fu)) *ok = false;
  } else {
    // subnormal: q = mant * 2^(emin - m), 1 <= mant < 2^m, so 2^(emin - m) <= |q| < 2^emin
    const int sh = 23 - (E - (emin - m));                          // sig >> sh = mant
    if (E <= -127 || E < emin - m || sh > 23 || (sig & ((1u << sh) - 1u))) {
      *ok = false;
      return 0u;
    }
    code = sig >> sh;
  }
  return sbit | (code & ((1u << (e + m)) - 1u));
}

// The float32 value of a code (the inverse of mx_encode on its values).
MXQ_HD float mx_decode(uint32_t code, int e, int m) {
  const uint32_t s = (code >> (e + m)) & 1u, ex = (code >> m) & ((1u << e) - 1u), man = code & ((1u << m) - 1u);
  const int bias = (1 << (e - 1)) - 1;
  float v;
  if (e == 5 && m == 2 && ex == 31u) v = man ? f_nan() : f_inf();
  else if (e == 4 && m == 3 && ex == 15u && man == 7u) v = f_nan();
  else if (ex == 0u) v = (float)man * pow2f(1 - bias - m);
  else v = u2f(((uint32_t)((int)ex - bias + 127) << 23) | (man << (23 - m)));
  return s ? -v : v;
}

// E8M0 scale byte of a block scale x: 2^(k) for k in [-127, 127] is k + 127, NaN is 0xFF.  A block whose codes
// are all zero (zero_block) has the value 0 under any scale: a scale E8M0 lacks (the 1e-38 floor of a zero
// block) becomes 0, i.e. 2^-127.  *ok is cleared for any other scale E8M0 lacks.
MXQ_HD uint32_t e8m0_encode(float x, bool zero_block, bool* ok) {
  const uint32_t u = f2u(x);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return 0xFFu;
  const uint32_t ex = u >> 23;                                     // sign 0 for a positive scale
  if ((u & 0x7FFFFFu) == 0u && ex >= 1u && ex <= 254u) return ex;  // 2^-126 .. 2^127
  if (u == 0x00400000u) return 0u;                                 // 2^-127, a float32 subnormal
  if (!zero_block) *ok = false;
  return 0u;
}

MXQ_HD float e8m0_decode(uint32_t b) { return b == 0xFFu ? f_nan() : pow2f((int)b - 127); }
