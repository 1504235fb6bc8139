// The comparison product on the gfx950 matrix cores: C = A^T B from MX codes and block scales with
// V_MFMA_SCALE_F32_32X32X64_F8F6F4, the matrix-core counterpart of fp64_accum (mxq/_fp64_accum.py:24-29).  Not
// bit-exact with anything: the instruction sums each group of 8 consecutive k in a fixed-point window 13 bits
// below the group's largest exponent sum (products truncated toward zero), then combines the groups and the
// float32 accumulator with about float32 precision.  The bound that follows is stated with mfma_accum.
//
//   k_mx_pack   codes (K x n float32, exact values of an FP8/FP6/FP4 element format) and power-of-two scales
//               (ceil(K/32) x n) -> the instruction's operand type (kind: 0 FP8 E4M3, 1 BF8 E5M2, 2 FP6 E2M3,
//               3 BF6 E3M2, 4 FP4 E2M1; a code of a narrower format also fits E4M3) and one E8M0 byte per scale, in
//               the instruction's lane order: for 32-column tile t and 64-deep K step s, lane l = 32h + r (column
//               32t + r) holds 32 codes in BPL = 32 w / 8 bytes (w = 8, 6 or 4) at byte ((t * nk + s) * 64 + l) *
//               BPL (nk = K64 / 64, K padded to a multiple of 64 with zeros), code j in bits [w j, w j + w): for FP8,
//               codes [16h, 16h + 16) of block 2s then the same of block 2s + 1; for FP6 and FP4, the 32 codes of
//               block 2s + h in order (each lane layout established on the device with single-product outputs).
//               The lane's scale, block 2s + h's, is byte (t * nk + s) * 64 + l of the scale array.  Columns past n (up to the tile) are zero codes with
//               scale 1.  So one wave's operand for one step is 64 BPL bytes read contiguously.  A code the
//               type cannot hold exactly, or a scale that is not a power of two in [2^-127, 2^127] over a block
//               with a nonzero code, sets the error word.
//   k_mx_mfma   32 x 32 tiles of C, 64 K per instruction, lane layout as above (established on the device with
//               exact integer data); lane l's 16 results are C[8(i/4) + 4h + i%4][l % 32], i = 0..15.  Each
//               output is the sum, in a fixed order, of four float32 chains over every fourth K step.
#include "mxq_common.h"
#include "mxq_numerics.h"
#include "ocp_hw.h"

namespace {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));
using mxq_ocp_hw::f2v;
using mxq_ocp_hw::s2v;

// The MFMA operand type codes (the instruction's cbsz / blgp values).
constexpr int kE4M3 = 0, kE5M2 = 1, kE2M3 = 2, kE3M2 = 3, kE2M1 = 4;

__host__ __device__ constexpr int code_bits(int kind) { return kind <= kE5M2 ? 8 : (kind <= kE3M2 ? 6 : 4); }
__host__ __device__ constexpr int lane_bytes(int kind) { return 4 * code_bits(kind); }   // 32 codes

// E8M0 byte of a power-of-two scale in [2^-127, 2^127]; false otherwise.
__device__ __forceinline__ bool e8m0_byte(float x, uint32_t& out) {
  const uint32_t u = f2u(x);
  if (u == 0x00400000u) {                                  // 2^-127, a float32 subnormal
    out = 0u;
    return true;
  }
  if ((u & 0x807FFFFFu) != 0u || u == 0u || u >= 0x7F800000u) return false;
  out = (u >> 23);                                         // biased exponent = e + 127, 1..254
  return true;
}

// Writes one (column c < n32, 32-row block g < K64/32) block: its 32 codes as the instruction's fields (code j
// at bit W j of words[], FP8: half j / 16 in words [h HW, ..)) and its scale byte, where the lane-ordered layout
// above puts them.
template <int W>
__device__ __forceinline__ void put_block(const uint32_t (&words)[W], uint32_t sbyte, int64_t c, int64_t g,
                                          int64_t nk, uint8_t* __restrict__ codes, uint8_t* __restrict__ scales) {
  constexpr int HW = 16 * W / 32;                          // words per half block (16 codes of W bits)
  constexpr int BPL = 4 * W;                               // bytes per lane and K step
  const int64_t tile = c / 32, r = c % 32, step = g / 2, half = g % 2;
  const int64_t chunk = (tile * nk + step) * 64;           // lane 0 of this (tile, step)
  if constexpr (W == 8) {
    // codes [0, 16) of the block go to lane r (h = 0), [16, 32) to lane 32 + r (h = 1); block 2s + half fills
    // bytes [16 half, 16 half + 16) of each lane's 32
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      uint32_t* dst = reinterpret_cast<uint32_t*>(codes + (chunk + 32 * h + r) * BPL + half * (BPL / 2));
#pragma unroll
      for (int w = 0; w < HW; ++w) dst[w] = words[h * HW + w];
    }
  } else {
    // the whole block to lane 32 half + r
    uint32_t* dst = reinterpret_cast<uint32_t*>(codes + (chunk + 32 * half + r) * BPL);
#pragma unroll
    for (int w = 0; w < 2 * HW; ++w) dst[w] = words[w];
  }
  scales[chunk + half * 32 + r] = (uint8_t)sbyte;          // lane 32 * half + r reads block 2s + half
}

// One thread per (column c < n32, 32-row block g < K64/32): the block's 32 codes and one scale byte.
// Consecutive threads take consecutive columns.  The codes come from gfx950's conversions (V_CVT_SCALEF32_PK_*,
// scale 1), whose fields are already in the lane order (FP8 byte j, FP6 field j at bit 6 j, FP4 nibble j at
// bit 4 j), and a value is a code of the type exactly when it is finite and converts back to itself, bit for
// bit: an exact value converts to its own code (-0 keeping its sign, as the OCP code of -0 does), and anything
// else to a different value (rounded, saturated, or E4M3's NaN and E5M2's Inf past their ranges).
template <int W>
__global__ void __launch_bounds__(256) k_mx_pack(const float* __restrict__ P, const float* __restrict__ X,
                                                 int64_t K, int64_t n, int64_t n32, int64_t K64, int kind,
                                                 uint8_t* __restrict__ codes, uint8_t* __restrict__ scales,
                                                 int* __restrict__ err) {
  const int64_t nb64 = K64 / 32, nk = K64 / 64;
  const uint32_t t = blockIdx.x * blockDim.x + threadIdx.x;   // the launch keeps n32 * nb64 below 2^31
  if ((int64_t)t >= n32 * nb64) return;
  const uint32_t gq = t / (uint32_t)n32;
  const int64_t g = gq, c = t - gq * (uint32_t)n32;
  const bool live = c < n;
  float x[32];
  bool nonzero = false, finite = true;
#pragma unroll
  for (int j = 0; j < 32; ++j) {
    const int64_t k = g * 32 + j;
    x[j] = live && k < K ? P[k * n + c] : 0.0f;
    nonzero |= (f2u(x[j]) & 0x7FFFFFFFu) != 0u;
    finite &= (f2u(x[j]) & 0x7FFFFFFFu) < 0x7F800000u;
  }
  uint32_t words[W];                                       // code j at bit W j (FP8: half j / 16 in words [h HW, ..))
  bool same = true;                                        // every value came back from its code
  if constexpr (W == 8) {
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      s2v r = {0, 0};
      f2v lo, hi;
      if (kind == kE4M3) {
        r = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(r, x[4 * q], x[4 * q + 1], 1.0f, false);
        r = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(r, x[4 * q + 2], x[4 * q + 3], 1.0f, true);
        lo = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(__builtin_bit_cast(uint32_t, r), 1.0f, false);
        hi = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(__builtin_bit_cast(uint32_t, r), 1.0f, true);
      } else {
        r = __builtin_amdgcn_cvt_scalef32_pk_bf8_f32(r, x[4 * q], x[4 * q + 1], 1.0f, false);
        r = __builtin_amdgcn_cvt_scalef32_pk_bf8_f32(r, x[4 * q + 2], x[4 * q + 3], 1.0f, true);
        lo = __builtin_amdgcn_cvt_scalef32_pk_f32_bf8(__builtin_bit_cast(uint32_t, r), 1.0f, false);
        hi = __builtin_amdgcn_cvt_scalef32_pk_f32_bf8(__builtin_bit_cast(uint32_t, r), 1.0f, true);
      }
      words[q] = __builtin_bit_cast(uint32_t, r);
      same &= f2u(lo.x) == f2u(x[4 * q]) && f2u(lo.y) == f2u(x[4 * q + 1]) && f2u(hi.x) == f2u(x[4 * q + 2]) &&
              f2u(hi.y) == f2u(x[4 * q + 3]);
    }
  } else if constexpr (W == 6) {
    mxq_ocp_hw::f16v even, odd;
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      even[k] = x[2 * k];
      odd[k] = x[2 * k + 1];
    }
    const mxq_ocp_hw::u6v pk = mxq_ocp_hw::pack16x2(even, odd, kind == kE2M3);
    const mxq_ocp_hw::f32v back = mxq_ocp_hw::unpack32(pk, kind == kE2M3);
#pragma unroll
    for (int w = 0; w < 6; ++w) words[w] = pk[w];
#pragma unroll
    for (int j = 0; j < 32; ++j) same &= f2u(back[j]) == f2u(x[j]);
  } else {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      uint32_t w = 0u;
      w = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(w, x[8 * q], x[8 * q + 1], 1.0f, 0);
      w = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(w, x[8 * q + 2], x[8 * q + 3], 1.0f, 1);
      w = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(w, x[8 * q + 4], x[8 * q + 5], 1.0f, 2);
      w = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(w, x[8 * q + 6], x[8 * q + 7], 1.0f, 3);
      words[q] = w;
      const f2v b0 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, 1.0f, 0);
      const f2v b1 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, 1.0f, 1);
      const f2v b2 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, 1.0f, 2);
      const f2v b3 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, 1.0f, 3);
      same &= f2u(b0.x) == f2u(x[8 * q]) && f2u(b0.y) == f2u(x[8 * q + 1]) && f2u(b1.x) == f2u(x[8 * q + 2]) &&
              f2u(b1.y) == f2u(x[8 * q + 3]) && f2u(b2.x) == f2u(x[8 * q + 4]) && f2u(b2.y) == f2u(x[8 * q + 5]) &&
              f2u(b3.x) == f2u(x[8 * q + 6]) && f2u(b3.y) == f2u(x[8 * q + 7]);
    }
  }
  bool bad = !(finite && same);
  uint32_t sbyte = 127u;
  if (live && g * 32 < K) {
    if (!e8m0_byte(X[g * n + c], sbyte)) {
      sbyte = 127u;
      if (nonzero) bad = true;                             // a non-power-of-two scale only over zero codes
    }
  }
  put_block<W>(words, sbyte, c, g, nk, codes, scales);
  if (bad) atomicOr(err, 1);
}

// k_mx_pack's layout from the byte wire format (mxq.packed: K x n code bytes, the code in the low w bits with
// the OCP MX numbering, and ceil(K/32) x n E8M0 bytes), one thread per (column, block): the fields are the codes
// themselves, so no conversion.  A byte that is no finite code of the type (E4M3 S.1111.111, E5M2's exponent
// field all ones, FP6 and FP4 bits above w) or a scale of 0xFF (NaN) over a block with a nonzero code sets
// the error word; the matrix cores then see what the low bits say.
template <int W>
__global__ void __launch_bounds__(256) k_mx_pack_bytes(const uint8_t* __restrict__ P, const uint8_t* __restrict__ X,
                                                       int64_t K, int64_t n, int64_t n32, int64_t K64, int kind,
                                                       uint8_t* __restrict__ codes, uint8_t* __restrict__ scales,
                                                       int* __restrict__ err) {
  const int64_t nb64 = K64 / 32, nk = K64 / 64;
  const uint32_t t = blockIdx.x * blockDim.x + threadIdx.x;   // the launch keeps n32 * nb64 below 2^31
  if ((int64_t)t >= n32 * nb64) return;
  const uint32_t gq = t / (uint32_t)n32;
  const int64_t g = gq, c = t - gq * (uint32_t)n32;
  const bool live = c < n;
  const uint32_t fmask = (1u << W) - 1u;                   // the field (FP8: the whole byte)
  const uint32_t mag = W == 8 ? 0x7Fu : (fmask >> 1);      // the field without its sign bit
  uint32_t words[W] = {};
  bool nonzero = false, bad = false;
#pragma unroll
  for (int j = 0; j < 32; ++j) {
    const int64_t k = g * 32 + j;
    const uint32_t b = live && k < K ? P[k * n + c] : 0u;
    nonzero |= (b & mag) != 0u;
    if constexpr (W == 8) bad |= kind == kE4M3 ? (b & 0x7Fu) == 0x7Fu : (b & 0x7Cu) == 0x7Cu;
    else bad |= b > fmask;
    const int bit = W * j;                                 // field j at bit W j of the 32 codes' W words
    words[bit / 32] |= (b & fmask) << (bit % 32);
    if (bit % 32 + W > 32) words[bit / 32 + 1] |= (b & fmask) >> (32 - bit % 32);
  }
  uint32_t sbyte = 127u;
  if (live && g * 32 < K) {
    sbyte = X[g * n + c];
    if (sbyte == 0xFFu) {
      if (nonzero) bad = true;                             // a NaN scale only over zero codes
      sbyte = 127u;
    }
  }
  put_block<W>(words, sbyte, c, g, nk, codes, scales);
  if (bad) atomicOr(err, 1);
}

// k_mx_pack_bytes for four adjacent columns of one block a thread, n % 4 == 0 and the byte arrays 4-byte
// aligned: the block's 32 rows load as one word each (the four columns' bytes; eight consecutive threads read
// 32 contiguous bytes of a row), a byte transpose of each 4 x 4 square by permutes gives each column's codes
// four rows to a word, and each column's lane bytes leave in 16- or 8-byte stores.  Same checks, fields and
// layout as k_mx_pack_bytes.
__device__ __forceinline__ void transpose4x4(uint32_t& a, uint32_t& b, uint32_t& c, uint32_t& d) {
  // rows a, b, c, d of four bytes (byte q = column q) -> columns: a = column 0's four rows, ...
  const uint32_t ab_lo = __builtin_amdgcn_perm(b, a, 0x05010400u);   // a0 b0 a1 b1
  const uint32_t ab_hi = __builtin_amdgcn_perm(b, a, 0x07030602u);   // a2 b2 a3 b3
  const uint32_t cd_lo = __builtin_amdgcn_perm(d, c, 0x05010400u);   // c0 d0 c1 d1
  const uint32_t cd_hi = __builtin_amdgcn_perm(d, c, 0x07030602u);   // c2 d2 c3 d3
  a = __builtin_amdgcn_perm(cd_lo, ab_lo, 0x05040100u);             // a0 b0 c0 d0
  b = __builtin_amdgcn_perm(cd_lo, ab_lo, 0x07060302u);             // a1 b1 c1 d1
  c = __builtin_amdgcn_perm(cd_hi, ab_hi, 0x05040100u);             // a2 b2 c2 d2
  d = __builtin_amdgcn_perm(cd_hi, ab_hi, 0x07060302u);             // a3 b3 c3 d3
}

template <int W>
__global__ void __launch_bounds__(256) k_mx_pack_bytes4(const uint8_t* __restrict__ P, const uint8_t* __restrict__ X,
                                                        int64_t K, int64_t n, int64_t n32, int64_t K64, int kind,
                                                        uint8_t* __restrict__ codes, uint8_t* __restrict__ scales,
                                                        int* __restrict__ err) {
  constexpr int BPL = 4 * W;
  const int64_t nk = K64 / 64, nq = n32 / 4;
  const uint32_t t = blockIdx.x * blockDim.x + threadIdx.x;   // the launch keeps nq * K64 / 32 below 2^31
  if ((int64_t)t >= nq * (K64 / 32)) return;
  const uint32_t gq = t / (uint32_t)nq;
  const int64_t g = gq, c0 = (int64_t)(t - gq * (uint32_t)nq) * 4;
  const bool live = c0 < n;                                // n % 4 == 0: the quad is whole or past n
  const int64_t tile = c0 / 32, r0 = c0 % 32, step = g / 2, half = g % 2;
  const int64_t chunk = (tile * nk + step) * 64;
  uint32_t w[32];                                          // row k's four bytes, then column-major (below)
  bool bad = false;
#pragma unroll
  for (int k = 0; k < 32; ++k) {
    const int64_t row = g * 32 + k;
    w[k] = live && row < K ? *reinterpret_cast<const uint32_t*>(P + row * n + c0) : 0u;
    if constexpr (W == 8) {
      const uint32_t y = kind == kE4M3 ? (w[k] & 0x7F7F7F7Fu) + 0x01010101u : (w[k] & 0x7C7C7C7Cu) + 0x04040404u;
      bad |= (y & 0x80808080u) != 0u;                      // E4M3 S.1111.111, E5M2 S.11111.xx
    } else {
      bad |= (w[k] & (W == 6 ? 0xC0C0C0C0u : 0xF0F0F0F0u)) != 0u;
    }
  }
  uint32_t sw = live && g * 32 < K ? *reinterpret_cast<const uint32_t*>(X + g * n + c0) : 0x7F7F7F7Fu;
  // after the transposes, w[4 i + q] holds column q's rows 4 i .. 4 i + 3
#pragma unroll
  for (int i = 0; i < 8; ++i) transpose4x4(w[4 * i], w[4 * i + 1], w[4 * i + 2], w[4 * i + 3]);
  const uint32_t mag = W == 8 ? 0x7F7F7F7Fu : (W == 6 ? 0x1F1F1F1Fu : 0x07070707u);
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    bool nonzero = false;
#pragma unroll
    for (int i = 0; i < 8; ++i) nonzero |= (w[4 * i + q] & mag) != 0u;
    if (((sw >> (8 * q)) & 0xFFu) == 0xFFu) {
      bad |= nonzero;                                      // a NaN scale only over zero codes
      sw = (sw & ~(0xFFu << (8 * q))) | (127u << (8 * q));
    }
    if constexpr (W == 8) {
      // codes [0, 16) to lane r (h = 0), [16, 32) to lane 32 + r, at bytes [16 half, 16 half + 16)
#pragma unroll
      for (int h = 0; h < 2; ++h)
        *reinterpret_cast<u32x4*>(codes + (chunk + 32 * h + r0 + q) * BPL + half * (BPL / 2)) =
            u32x4{w[4 * (4 * h) + q], w[4 * (4 * h + 1) + q], w[4 * (4 * h + 2) + q], w[4 * (4 * h + 3) + q]};
    } else {
      // the whole block to lane 32 half + r, code j at bit W j
      uint32_t f[W] = {};
#pragma unroll
      for (int j = 0; j < 32; ++j) {
        const uint32_t b = (w[4 * (j / 4) + q] >> (8 * (j % 4))) & 0xFFu;
        const int bit = W * j;
        f[bit / 32] |= b << (bit % 32);
        if (bit % 32 + W > 32) f[bit / 32 + 1] |= b >> (32 - bit % 32);
      }
      uint8_t* dst = codes + (chunk + 32 * half + r0 + q) * BPL;
      if constexpr (W == 4) {
        *reinterpret_cast<u32x4*>(dst) = u32x4{f[0], f[1], f[2], f[3]};
      } else {
#pragma unroll
        for (int j = 0; j < 3; ++j) reinterpret_cast<u32x2*>(dst)[j] = u32x2{f[2 * j], f[2 * j + 1]};
      }
    }
  }
  *reinterpret_cast<uint32_t*>(scales + chunk + half * 32 + r0) = sw;
  if (bad) atomicOr(err, 1);
}

// The product.  A workgroup of four waves owns a (32 TM) x (32 TN) block of C (TM x TN instruction tiles) and
// splits K four ways: wave w runs K steps w, w + 4, w + 8, ... over the whole block, TM x TN instructions per
// step, so every operand byte is loaded once per workgroup and feeds TN (A) or TM (B) instructions.  No wave
// shares operands with another, so they go from global memory straight to the wave's registers (one
// contiguous 64 BPL-byte chunk per 32-column tile and step), kDepth own steps ahead of the instructions.  At
// the end the four partial blocks meet in LDS and each output is ((p0 + p1) + p2) + p3, p_w the float32 chain
// of wave w's steps in K order.  The K split and the order of the sums do not depend on TM or TN, so neither do
// the results.  Tiles past the packed operand (M or N not reaching the block's last tile) re-read its last
// tile: valid bytes whose results are never stored.
template <int TM, int TN>
struct MxRegs {
  v8i a[TM], b[TN];
  int sa[TM], sb[TN];
};

// (tile, step) chunk c: this lane's BPL bytes of codes (the unused high registers of the operand are zero)
template <int BPL>
__device__ __forceinline__ v8i load_codes(const uint8_t* codes, int64_t chunk, int lane) {
  const uint8_t* q = codes + (chunk * 64 + lane) * BPL;
  if constexpr (BPL == 32) {
    const v4i* p = reinterpret_cast<const v4i*>(q);
    const v4i lo = p[0], hi = p[1];
    return v8i{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  } else if constexpr (BPL == 24) {
    typedef int v2i __attribute__((ext_vector_type(2)));
    const v2i* p = reinterpret_cast<const v2i*>(q);        // 8-byte aligned: 24 (chunk * 64 + lane)
    const v2i x = p[0], y = p[1], z = p[2];
    return v8i{x[0], x[1], y[0], y[1], z[0], z[1], 0, 0};
  } else {
    const v4i v = *reinterpret_cast<const v4i*>(q);
    return v8i{v[0], v[1], v[2], v[3], 0, 0, 0, 0};
  }
}

// Own steps in flight per wave: four when their operands take at most 200 VGPRs, else three (the TM TN
// accumulators live in the 256 AGPRs).
template <int BA, int BB, int TM, int TN>
struct MxDepth {
  static constexpr int kRegs = (TM * BA + TN * BB) / 4 + TM + TN;     // operand VGPRs of one step
  static constexpr int kDepth = kRegs * 4 <= 200 ? 4 : 3;
  static constexpr int kPhase = TM * TN <= 8 ? TM * TN : 8;          // tiles per wave and reduction phase
  static constexpr int kReduce = 4 * kPhase * 16 * 64 * 4;           // the four waves' partial tiles, bytes
  static_assert((TM * TN) % kPhase == 0 && kPhase % 4 == 0, "reduction phases");
};

template <int KA, int KB, int TM, int TN>
__device__ __forceinline__ void mfma_step(v16f (&acc)[TM][TN], const MxRegs<TM, TN>& g) {
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
      acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(g.a[i], g.b[j], acc[i][j], KA, KB, 0, g.sa[i], 0,
                                                                  g.sb[j]);
}

template <int KA, int KB, int TM, int TN>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
k_mx_mfma(const uint8_t* __restrict__ A, const uint8_t* __restrict__ SA, const uint8_t* __restrict__ B,
          const uint8_t* __restrict__ SB, float* __restrict__ C, int64_t K64, int64_t M, int64_t N) {
  // (registers for one wave per SIMD: the 128 x 128 and 64 x 128 blocks' reduction takes 128 KiB of LDS, one
  // workgroup per CU, and the operands in flight take what the accumulators leave)
  constexpr int BA = lane_bytes(KA), BB = lane_bytes(KB);
  using D = MxDepth<BA, BB, TM, TN>;
  constexpr int kDepth = D::kDepth;
  __shared__ __align__(16) float red[D::kReduce / 4];
  // the wave index as a scalar, so the own-step count and its branches are the wave's, not per lane
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int64_t nk = K64 / 64, tiles_m = (M + 31) / 32, tiles_n = (N + 31) / 32;
  const int64_t m0 = (int64_t)blockIdx.y * (32 * TM), n0 = (int64_t)blockIdx.x * (32 * TN);
  int64_t ta[TM], tb[TN];
#pragma unroll
  for (int i = 0; i < TM; ++i) ta[i] = min(m0 / 32 + i, tiles_m - 1) * nk;
#pragma unroll
  for (int j = 0; j < TN; ++j) tb[j] = min(n0 / 32 + j, tiles_n - 1) * nk;
  // own step j is K step 4 j + wave; loads past the last K step re-read it (never used)
  auto load = [&](MxRegs<TM, TN>& g, int64_t j) {
    int64_t s = 4 * j + wave;
    s = s < nk ? s : nk - 1;
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      g.a[i] = load_codes<BA>(A, ta[i] + s, lane);
      g.sa[i] = SA[(ta[i] + s) * 64 + lane];
    }
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      g.b[j] = load_codes<BB>(B, tb[j] + s, lane);
      g.sb[j] = SB[(tb[j] + s) * 64 + lane];
    }
  };
  const int64_t own = nk > wave ? (nk - wave + 3) / 4 : 0;
  v16f acc[TM][TN] = {};
  MxRegs<TM, TN> slot[kDepth];
#pragma unroll
  for (int d = 0; d < kDepth; ++d) load(slot[d], d);
  int64_t j = 0;
  for (; j + kDepth <= own; j += kDepth) {
#pragma unroll
    for (int d = 0; d < kDepth; ++d) {
      mfma_step<KA, KB>(acc, slot[d]);
      load(slot[d], j + d + kDepth);
    }
  }
#pragma unroll
  for (int d = 0; d < kDepth - 1; ++d)   // the last own - j < kDepth steps
    if (j + d < own) mfma_step<KA, KB>(acc, slot[d]);
  // the partial blocks meet in LDS kPhase tiles at a time: wave w's tile t (of the phase), elements
  // [4 e, 4 e + 4) of every lane, 16 bytes at ((w kPhase + t) 4 + e) 256 + 4 l floats; then wave v sums and
  // stores the phase's tiles v, v + 4, ...: lane l = 32 h + r, element 4 e + k of tile (i, jj) is
  // C[m0 + 32 i + 8 e + 4 h + k][n0 + 32 jj + r]
  constexpr int P = D::kPhase;
  const int r = lane & 31, h = lane >> 5;
#pragma unroll
  for (int ph = 0; ph < TM * TN / P; ++ph) {
    if (ph > 0) __syncthreads();   // the previous phase's sums have read their tiles
#pragma unroll
    for (int t = 0; t < P; ++t)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int i = (ph * P + t) / TN, jj = (ph * P + t) % TN;
        *reinterpret_cast<float4*>(red + (((wave * P + t) * 4 + e) * 64 + lane) * 4) =
            make_float4(acc[i][jj][4 * e], acc[i][jj][4 * e + 1], acc[i][jj][4 * e + 2], acc[i][jj][4 * e + 3]);
      }
    __syncthreads();
#pragma unroll
    for (int t = wave; t < P; t += 4) {
      const int i = (ph * P + t) / TN, jj = (ph * P + t) % TN;
      const int64_t n = n0 + 32 * jj + r;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float4 v = *reinterpret_cast<const float4*>(red + ((t * 4 + e) * 64 + lane) * 4);
#pragma unroll
        for (int w = 1; w < 4; ++w) {
          const float4 u = *reinterpret_cast<const float4*>(red + (((w * P + t) * 4 + e) * 64 + lane) * 4);
          v.x += u.x; v.y += u.y; v.z += u.z; v.w += u.w;
        }
        const int64_t m = m0 + 32 * i + 8 * e + 4 * h;
        if (n < N) {
          if (m < M) C[m * N + n] = v.x;
          if (m + 1 < M) C[(m + 1) * N + n] = v.y;
          if (m + 2 < M) C[(m + 2) * N + n] = v.z;
          if (m + 3 < M) C[(m + 3) * N + n] = v.w;
        }
      }
    }
  }
}

template <int TM, int TN, int KA>
void launch_mfma_b(int b_kind, dim3 grid, hipStream_t st, const uint8_t* A, const uint8_t* SA, const uint8_t* B,
                   const uint8_t* SB, float* C, int64_t K64, int64_t M, int64_t N) {
  switch (b_kind) {
    case kE4M3: k_mx_mfma<KA, kE4M3, TM, TN><<<grid, 256, 0, st>>>(A, SA, B, SB, C, K64, M, N); break;
    case kE5M2: k_mx_mfma<KA, kE5M2, TM, TN><<<grid, 256, 0, st>>>(A, SA, B, SB, C, K64, M, N); break;
    case kE2M3: k_mx_mfma<KA, kE2M3, TM, TN><<<grid, 256, 0, st>>>(A, SA, B, SB, C, K64, M, N); break;
    case kE3M2: k_mx_mfma<KA, kE3M2, TM, TN><<<grid, 256, 0, st>>>(A, SA, B, SB, C, K64, M, N); break;
    default: k_mx_mfma<KA, kE2M1, TM, TN><<<grid, 256, 0, st>>>(A, SA, B, SB, C, K64, M, N); break;
  }
}

template <int TM, int TN>
void launch_mfma(int a_kind, int b_kind, hipStream_t st, const uint8_t* A, const uint8_t* SA, const uint8_t* B,
                 const uint8_t* SB, float* C, int64_t K64, int64_t M, int64_t N) {
  const dim3 grid((unsigned)mxq::ceil_div(N, 32 * TN), (unsigned)mxq::ceil_div(M, 32 * TM));
  switch (a_kind) {
    case kE4M3: launch_mfma_b<TM, TN, kE4M3>(b_kind, grid, st, A, SA, B, SB, C, K64, M, N); break;
    case kE5M2: launch_mfma_b<TM, TN, kE5M2>(b_kind, grid, st, A, SA, B, SB, C, K64, M, N); break;
    case kE2M3: launch_mfma_b<TM, TN, kE2M3>(b_kind, grid, st, A, SA, B, SB, C, K64, M, N); break;
    case kE3M2: launch_mfma_b<TM, TN, kE3M2>(b_kind, grid, st, A, SA, B, SB, C, K64, M, N); break;
    default: launch_mfma_b<TM, TN, kE2M1>(b_kind, grid, st, A, SA, B, SB, C, K64, M, N); break;
  }
}

}  // namespace

extern "C" int mxq_mx_pack(const float* P, const float* X, int64_t K, int64_t n, int32_t kind, uint8_t* codes,
                           uint8_t* scales, int32_t* err, mxq_stream_t stream) {
  if (K < 0 || n < 0 || kind < kE4M3 || kind > kE2M1) return mxq::invalid("mxq_mx_pack: bad arguments");
  const int64_t K64 = mxq::ceil_div(K, 64) * 64;
  if (n == 0 || K64 == 0) return MXQ_OK;
  if (!P || !X || !codes || !scales || !err) return mxq::invalid("mxq_mx_pack: NULL pointer");
  if (reinterpret_cast<uintptr_t>(codes) % 16) return mxq::invalid("mxq_mx_pack: codes must be 16-byte aligned");
  const int64_t n32 = mxq::ceil_div(n, 32) * 32;
  const int64_t threads = n32 * (K64 / 32);
  if (threads >= (int64_t(1) << 31)) return mxq::invalid("mxq_mx_pack: operand too large (2^31 blocks of 32)");
  const dim3 grid = mxq::grid_for(threads, 256);
  hipStream_t st = mxq::as_stream(stream);
  if (code_bits(kind) == 8) k_mx_pack<8><<<grid, 256, 0, st>>>(P, X, K, n, n32, K64, kind, codes, scales, err);
  else if (code_bits(kind) == 6) k_mx_pack<6><<<grid, 256, 0, st>>>(P, X, K, n, n32, K64, kind, codes, scales, err);
  else k_mx_pack<4><<<grid, 256, 0, st>>>(P, X, K, n, n32, K64, kind, codes, scales, err);
  return mxq::check_launch("mxq_mx_pack");
}

extern "C" int mxq_mx_pack_bytes(const uint8_t* P, const uint8_t* X, int64_t K, int64_t n, int32_t kind,
                                 uint8_t* codes, uint8_t* scales, int32_t* err, mxq_stream_t stream) {
  if (K < 0 || n < 0 || kind < kE4M3 || kind > kE2M1) return mxq::invalid("mxq_mx_pack_bytes: bad arguments");
  const int64_t K64 = mxq::ceil_div(K, 64) * 64;
  if (n == 0 || K64 == 0) return MXQ_OK;
  if (!P || !X || !codes || !scales || !err) return mxq::invalid("mxq_mx_pack_bytes: NULL pointer");
  if (reinterpret_cast<uintptr_t>(codes) % 16) return mxq::invalid("mxq_mx_pack_bytes: codes must be 16-byte aligned");
  const int64_t n32 = mxq::ceil_div(n, 32) * 32;
  const int64_t threads = n32 * (K64 / 32);
  if (threads >= (int64_t(1) << 31)) return mxq::invalid("mxq_mx_pack_bytes: operand too large (2^31 blocks of 32)");
  const dim3 grid = mxq::grid_for(threads, 256);
  hipStream_t st = mxq::as_stream(stream);
  mxq::KernelTimer timer("mx_pack_bytes", st);
  if (n % 4 == 0 && (reinterpret_cast<uintptr_t>(P) | reinterpret_cast<uintptr_t>(X)) % 4 == 0) {
    const dim3 g4 = mxq::grid_for(n32 / 4 * (K64 / 32), 256);
    if (code_bits(kind) == 8) k_mx_pack_bytes4<8><<<g4, 256, 0, st>>>(P, X, K, n, n32, K64, kind, codes, scales, err);
    else if (code_bits(kind) == 6) k_mx_pack_bytes4<6><<<g4, 256, 0, st>>>(P, X, K, n, n32, K64, kind, codes, scales, err);
    else k_mx_pack_bytes4<4><<<g4, 256, 0, st>>>(P, X, K, n, n32, K64, kind, codes, scales, err);
    return mxq::check_launch("mxq_mx_pack_bytes");
  }
  if (code_bits(kind) == 8) k_mx_pack_bytes<8><<<grid, 256, 0, st>>>(P, X, K, n, n32, K64, kind, codes, scales, err);
  else if (code_bits(kind) == 6) k_mx_pack_bytes<6><<<grid, 256, 0, st>>>(P, X, K, n, n32, K64, kind, codes, scales, err);
  else k_mx_pack_bytes<4><<<grid, 256, 0, st>>>(P, X, K, n, n32, K64, kind, codes, scales, err);
  return mxq::check_launch("mxq_mx_pack_bytes");
}

extern "C" int mxq_mx_mfma(const uint8_t* A, const uint8_t* SA, int32_t a_kind, const uint8_t* B, const uint8_t* SB,
                           int32_t b_kind, float* C, int64_t K64, int64_t M, int64_t N, mxq_stream_t stream) {
  // K64 == 0 is refused: the kernel's prologue reads its first K step before the loop tests the count
  if (K64 <= 0 || K64 % 64 || M < 0 || N < 0) return mxq::invalid("mxq_mx_mfma: bad shape (K64 must be a positive multiple of 64)");
  if (a_kind < kE4M3 || a_kind > kE2M1 || b_kind < kE4M3 || b_kind > kE2M1)
    return mxq::invalid("mxq_mx_mfma: bad operand kind");
  if (M == 0 || N == 0) return MXQ_OK;
  if (!A || !SA || !B || !SB || !C) return mxq::invalid("mxq_mx_mfma: NULL pointer");
  if (reinterpret_cast<uintptr_t>(A) % 16 || reinterpret_cast<uintptr_t>(B) % 16)
    return mxq::invalid("mxq_mx_mfma: codes must be 16-byte aligned");
  // the largest block of 128 x 128, 64 x 128 or 64 x 64 outputs that still gives every CU a workgroup (an
  // operand byte feeds as many instructions as the block is wide or tall)
  const int64_t b44 = mxq::ceil_div(M, 128) * mxq::ceil_div(N, 128), b24 = mxq::ceil_div(M, 64) * mxq::ceil_div(N, 128);
  if (mxq::ceil_div(M, 64) > 65535) return mxq::invalid("mxq_mx_mfma: M too large");
  hipStream_t st = mxq::as_stream(stream);
  mxq::KernelTimer timer("mx_mfma", st);
  if (b44 >= 256) launch_mfma<4, 4>(a_kind, b_kind, st, A, SA, B, SB, C, K64, M, N);
  else if (b24 >= 256) launch_mfma<2, 4>(a_kind, b_kind, st, A, SA, B, SB, C, K64, M, N);
  else launch_mfma<2, 2>(a_kind, b_kind, st, A, SA, B, SB, C, K64, M, N);
  return mxq::check_launch("mxq_mx_mfma");
}
