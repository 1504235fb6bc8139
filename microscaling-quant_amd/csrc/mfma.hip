// The comparison product on the gfx950 matrix cores: C = A^T B from MX codes and block scales with
// V_MFMA_SCALE_F32_32X32X64_F8F6F4, the matrix-core counterpart of fp64_accum (mxq/_fp64_accum.py:24-29).  Not
// bit-exact with anything: the instruction sums each group of 8 consecutive k in a fixed-point window 13 bits
// below the group's largest exponent sum (products truncated toward zero), then combines the groups and the
// float32 accumulator with about float32 precision.  The bound that follows is stated with mfma_accum.
//
//   k_mx_pack   codes (K x n float32, exact values of an FP8/FP6/FP4 element format) and power-of-two scales
//               (ceil(K/32) x n) -> one byte per code in OCP FP8 (E4M3 holds every E4M3, E3M2, E2M3 and E2M1
//               value; E5M2 codes stay E5M2) and one E8M0 byte per scale, in the instruction's lane order: for
//               32-column tile t and 64-deep K step s, lane l = 32h + r (column 32t + r) holds 32 bytes, the codes
//               [16h, 16h + 16) of block 2s then the same of block 2s + 1, at byte ((t * nk + s) * 64 + l) * 32
//               (nk = K64 / 64, K padded to a multiple of 64 with zeros); its scale, block 2s + h's, is byte
//               (t * nk + s) * 64 + l of the scale array.  Columns past n (up to the tile) are zero codes with
//               scale 1.  So one wave's operand for one step is 2 KiB read contiguously.  A code the byte cannot
//               hold exactly, or a scale that is not a power of two in [2^-127, 2^127] over a block with a
//               nonzero code, sets the error word.
//   k_mx_mfma   32 x 32 tiles of C, 64 K per instruction, lane layout as above (established on the device with
//               exact integer data); lane l's 16 results are C[8(i/4) + 4h + i%4][l % 32], i = 0..15.
#include "mxq_common.h"
#include "mxq_numerics.h"

namespace {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));

constexpr int kE4M3 = 0, kE5M2 = 1;   // the MFMA operand type codes used here

// OCP FP8 byte of an exact value: E4M3 (bias 7, no infinities, max 448) or E5M2 (bias 15, max 57344).
// Returns false when x is not exactly representable.
__device__ __forceinline__ bool fp8_byte(float x, int kind, uint32_t& out) {
  const uint32_t u = f2u(x);
  const uint32_t sign = (u >> 31) << 7;
  const uint32_t a = u & 0x7FFFFFFFu;
  if (a == 0u) {
    out = sign;
    return true;
  }
  if (a >= 0x7F800000u) return false;                      // Inf / NaN codes are outside the comparison path
  const int man_bits = kind == kE4M3 ? 3 : 2;
  const int bias = kind == kE4M3 ? 7 : 15;
  const int emin = 1 - bias;                               // smallest normal exponent
  const int e = (int)(a >> 23) - 127;                      // float32 exponent (subnormal float32 never fits)
  if (e < emin - man_bits) return false;                   // below the format's smallest subnormal
  const uint32_t sig = (a & 0x007FFFFFu) | 0x00800000u;    // 24-bit significand (a is a normal float32 here)
  if (e >= emin) {
    const int drop = 23 - man_bits;
    if (sig & ((1u << drop) - 1u)) return false;           // more significand bits than the format has
    const uint32_t man = (sig >> drop) & ((1u << man_bits) - 1u);
    const int field = e + bias;
    if (kind == kE4M3 ? (field > 15 || (field == 15 && man == 7u)) : field > 30) return false;
    out = sign | ((uint32_t)field << man_bits) | man;
    return true;
  }
  // subnormal in the format: value = man * 2^(emin - man_bits)
  const int shift = 23 - (e - (emin - man_bits));          // sig >> shift = man
  if (shift > 31 || (sig & ((1u << shift) - 1u))) return false;
  out = sign | (sig >> shift);
  return true;
}

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

// One thread per (column c < n32, 32-row block g < K64/32): 32 bytes of codes and one scale byte, written
// where the lane-ordered layout above puts them.  Consecutive threads take consecutive columns.
__global__ void __launch_bounds__(256) k_mx_pack(const float* __restrict__ P, const float* __restrict__ X,
                                                 int64_t K, int64_t n, int64_t n32, int64_t K64, int kind,
                                                 uint8_t* __restrict__ codes, uint8_t* __restrict__ scales,
                                                 int* __restrict__ err) {
  const int64_t nb64 = K64 / 32, nk = K64 / 64;
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= n32 * nb64) return;
  const int64_t g = t / n32, c = t - (t / n32) * n32;
  const bool live = c < n;
  uint32_t words[8];
  bool nonzero = false, bad = false;
#pragma unroll
  for (int w = 0; w < 8; ++w) {
    uint32_t word = 0u;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t k = g * 32 + w * 4 + j;
      uint32_t byte = 0u;
      if (live && k < K) {
        const float x = P[k * n + c];
        nonzero |= (f2u(x) & 0x7FFFFFFFu) != 0u;
        bad |= !fp8_byte(x, kind, byte);
      }
      word |= (byte & 0xFFu) << (8 * j);
    }
    words[w] = word;
  }
  uint32_t sbyte = 127u;
  if (live && g * 32 < K) {
    if (!e8m0_byte(X[g * n + c], sbyte)) {
      sbyte = 127u;
      if (nonzero) bad = true;                             // a non-power-of-two scale only over zero codes
    }
  }
  const int64_t tile = c / 32, r = c % 32, step = g / 2, half = g % 2;
  const int64_t chunk = (tile * nk + step) * 64;           // lane 0 of this (tile, step)
  // elements [0, 16) of the block go to lane r (h = 0), [16, 32) to lane 32 + r (h = 1); block 2s + half fills
  // bytes [16 * half, 16 * half + 16) of each lane's 32
  *reinterpret_cast<v4i*>(codes + (chunk + r) * 32 + half * 16) =
      v4i{(int)words[0], (int)words[1], (int)words[2], (int)words[3]};
  *reinterpret_cast<v4i*>(codes + (chunk + 32 + r) * 32 + half * 16) =
      v4i{(int)words[4], (int)words[5], (int)words[6], (int)words[7]};
  scales[chunk + half * 32 + r] = (uint8_t)sbyte;          // lane 32 * half + r reads block 2s + half
  if (bad) atomicOr(err, 1);
}

// One wave per (32 TA) x 64 block of C (TA x 2 instructions per K step, so each B load feeds TA of them and
// each A load two); four waves per workgroup in a 2 x 2 arrangement ((64 TA) x 128).  TA = 2 where that still
// gives the chip 1024 waves, else TA = 1: on C2's 512 x 4096 the 64 x 64 blocks leave half the SIMDs idle.
// Tiles past the packed operand (M or N not reaching this wave's last tile) re-read the last tile: valid
// bytes whose results are never stored.  Operands are loaded kDepth K steps ahead of the instructions that
// use them.  A block's K order is the same for either TA, so the results are too.
template <int TA>
struct MxStep {
  v8i a[TA], b[2];
  int sa[TA], sb[2];
};

constexpr int kDepth = 4;

// (tile, step) chunk c: this lane's 32 bytes and scale byte
__device__ __forceinline__ v8i load_codes(const uint8_t* codes, int64_t chunk, int lane) {
  const v4i* p = reinterpret_cast<const v4i*>(codes + (chunk * 64 + lane) * 32);
  const v4i lo = p[0], hi = p[1];
  return v8i{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}

template <int TA>
__device__ __forceinline__ void load_step(MxStep<TA>& st, const uint8_t* A, const uint8_t* SA, const uint8_t* B,
                                          const uint8_t* SB, const int64_t (&ta)[TA], const int64_t (&tb)[2],
                                          int64_t nk, int64_t s, int lane) {
#pragma unroll
  for (int t = 0; t < TA; ++t) {
    st.a[t] = load_codes(A, ta[t] * nk + s, lane);
    st.sa[t] = SA[(ta[t] * nk + s) * 64 + lane];
  }
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    st.b[t] = load_codes(B, tb[t] * nk + s, lane);
    st.sb[t] = SB[(tb[t] * nk + s) * 64 + lane];
  }
}

template <int KA, int KB, int TA>
__global__ void __launch_bounds__(256) k_mx_mfma(const uint8_t* __restrict__ A, const uint8_t* __restrict__ SA,
                                                 const uint8_t* __restrict__ B, const uint8_t* __restrict__ SB,
                                                 float* __restrict__ C, int64_t K64, int64_t M, int64_t N) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int r = lane & 31, h = lane >> 5;
  const int64_t m0 = (int64_t)blockIdx.y * (64 * TA) + (wave >> 1) * (32 * TA);
  const int64_t n0 = (int64_t)blockIdx.x * 128 + (wave & 1) * 64;
  const int64_t nk = K64 / 64, tiles_m = (M + 31) / 32, tiles_n = (N + 31) / 32;
  int64_t ta[TA], tb[2];
#pragma unroll
  for (int t = 0; t < TA; ++t) ta[t] = min(m0 / 32 + t, tiles_m - 1);
#pragma unroll
  for (int t = 0; t < 2; ++t) tb[t] = min(n0 / 32 + t, tiles_n - 1);
  v16f acc[TA][2] = {};
  // kDepth K steps in flight: step s of each round issues its instructions, then refills its slot with the
  // step kDepth ahead (past the end it re-reads the last step, whose values are never used).
  MxStep<TA> slot[kDepth];
#pragma unroll
  for (int s = 0; s < kDepth; ++s) load_step(slot[s], A, SA, B, SB, ta, tb, nk, min((int64_t)s, nk - 1), lane);
  for (int64_t k = 0; k < nk; k += kDepth) {
#pragma unroll
    for (int s = 0; s < kDepth; ++s) {
      if (k + s < nk) {
#pragma unroll
        for (int i = 0; i < TA; ++i)
#pragma unroll
          for (int j = 0; j < 2; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(slot[s].a[i], slot[s].b[j], acc[i][j], KA, KB,
                                                                        0, slot[s].sa[i], 0, slot[s].sb[j]);
      }
      load_step(slot[s], A, SA, B, SB, ta, tb, nk, min(k + s + kDepth, nk - 1), lane);
    }
  }
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int64_t n = n0 + 32 * j + r;
    if (n >= N) continue;
#pragma unroll
    for (int i = 0; i < TA; ++i)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int64_t m = m0 + 32 * i + 8 * (e / 4) + 4 * h + (e % 4);
        if (m < M) C[m * N + n] = acc[i][j][e];
      }
  }
}

template <int TA>
void launch_mfma(int a_kind, int b_kind, dim3 grid, hipStream_t st, const uint8_t* A, const uint8_t* SA,
                 const uint8_t* B, const uint8_t* SB, float* C, int64_t K64, int64_t M, int64_t N) {
  if (a_kind == kE4M3 && b_kind == kE4M3) k_mx_mfma<kE4M3, kE4M3, TA><<<grid, 256, 0, st>>>(A, SA, B, SB, C, K64, M, N);
  else if (a_kind == kE4M3) k_mx_mfma<kE4M3, kE5M2, TA><<<grid, 256, 0, st>>>(A, SA, B, SB, C, K64, M, N);
  else if (b_kind == kE4M3) k_mx_mfma<kE5M2, kE4M3, TA><<<grid, 256, 0, st>>>(A, SA, B, SB, C, K64, M, N);
  else k_mx_mfma<kE5M2, kE5M2, TA><<<grid, 256, 0, st>>>(A, SA, B, SB, C, K64, M, N);
}

}  // namespace

extern "C" int mxq_mx_pack(const float* P, const float* X, int64_t K, int64_t n, int32_t kind, uint8_t* codes,
                           uint8_t* scales, int32_t* err, mxq_stream_t stream) {
  if (K < 0 || n < 0 || (kind != kE4M3 && kind != kE5M2)) return mxq::invalid("mxq_mx_pack: bad arguments");
  const int64_t K64 = mxq::ceil_div(K, 64) * 64;
  if (n == 0 || K64 == 0) return MXQ_OK;
  if (!P || !X || !codes || !scales || !err) return mxq::invalid("mxq_mx_pack: NULL pointer");
  if (reinterpret_cast<uintptr_t>(codes) % 16) return mxq::invalid("mxq_mx_pack: codes must be 16-byte aligned");
  const int64_t n32 = mxq::ceil_div(n, 32) * 32;
  const int64_t threads = n32 * (K64 / 32);
  k_mx_pack<<<mxq::grid_for(threads, 256), 256, 0, mxq::as_stream(stream)>>>(P, X, K, n, n32, K64, kind, codes,
                                                                               scales, err);
  return mxq::check_launch("mxq_mx_pack");
}

extern "C" int mxq_mx_mfma(const uint8_t* A, const uint8_t* SA, int32_t a_kind, const uint8_t* B, const uint8_t* SB,
                           int32_t b_kind, float* C, int64_t K64, int64_t M, int64_t N, mxq_stream_t stream) {
  // K64 == 0 is refused: the kernel's prologue reads its first K step before the loop tests the count
  if (K64 <= 0 || K64 % 64 || M < 0 || N < 0) return mxq::invalid("mxq_mx_mfma: bad shape (K64 must be a positive multiple of 64)");
  if ((a_kind != kE4M3 && a_kind != kE5M2) || (b_kind != kE4M3 && b_kind != kE5M2))
    return mxq::invalid("mxq_mx_mfma: bad operand kind");
  if (M == 0 || N == 0) return MXQ_OK;
  if (!A || !SA || !B || !SB || !C) return mxq::invalid("mxq_mx_mfma: NULL pointer");
  if (reinterpret_cast<uintptr_t>(A) % 16 || reinterpret_cast<uintptr_t>(B) % 16)
    return mxq::invalid("mxq_mx_mfma: codes must be 16-byte aligned");
  // 64 x 64 blocks per wave while they give at least 1024 waves, else 32 x 64
  const bool two = mxq::ceil_div(N, 128) * mxq::ceil_div(M, 128) * 4 >= 1024;
  if (mxq::ceil_div(M, two ? 128 : 64) > 65535) return mxq::invalid("mxq_mx_mfma: M too large");
  const dim3 grid((unsigned)mxq::ceil_div(N, 128), (unsigned)mxq::ceil_div(M, two ? 128 : 64));
  hipStream_t st = mxq::as_stream(stream);
  mxq::KernelTimer timer("mx_mfma", st);
  if (two) launch_mfma<2>(a_kind, b_kind, grid, st, A, SA, B, SB, C, K64, M, N);
  else launch_mfma<1>(a_kind, b_kind, grid, st, A, SA, B, SB, C, K64, M, N);
  return mxq::check_launch("mxq_mx_mfma");
}
