// The systolic PE column on gfx950: Y = A^T B from MX codes and scales, every output element its own strictly
// sequential chain in the reference's order (mxq/matmul/_systolic.py:23-62):
//   for each block of K: scale map X_A[g] (x) X_B[g]
//     for each reduction of `size` k: S = 0; S = acc_add(S, product(a_k, b_k), lane k % size)
//       C = tile_add(C, S * scale)
// Parallelism is over M x N only; nothing is split along K, so no summation order changes.  The work is
// VALU (integer and float32 bit manipulation), not MFMA: the matrix cores' accumulation would not round
// where the datapath does.
//
// Three kernels:
//   k_stats         max |x| bit pattern of A, B, X_A and X_B (atomic max on the patterns of |x|: patterns of
//                   non-negative floats order like their values; >= 0x7F800000 means Inf or NaN present)
//   k_systolic_fast MXGEMMINI with size in {4, 8, 16, 32}, lanes (4, m <= 9) of non-decreasing m, optionally a
//                   last (8, 7) lane, prod_m <= every e4 lane's m, when the stats show finite codes and scales,
//                   max|a| < 2^100 and max|a| * max|b| <= 8.  A's rows are staged into LDS times 2^(6 + m) of
//                   their lane, so an e4 lane works in units of its subnormal step 2^-(6+m):
//                      p = rint(trunc(a' * b))      float32 multiply, mask the dropped significand bits,
//                                                   round to an integer = lane(p) (the flush below
//                                                   2^prod_floor is under half a step, so it is subsumed)
//                      S = rne_m(S + p)             the sum is an exact integer below 2^24; bit RNE at m
//                                                   fraction bits is the lane rounding (identity below 2^m)
//                   7 VALU operations per emulated MAC; the sum is rescaled by 2 when m steps up.  The bf16
//                   lane and the tile add are one float32 add of two values of at most 8 significant bits
//                   followed by bit RNE to bf16, which equals the reference's exact add with one rounding
//                   (double rounding through 24 bits is harmless for 8-bit operands: 24 >= 2*8 + 1).
//   k_systolic_gen  every other case: the full per-step rule for any codes, any lanes (e <= 8), MXGEMMINI or
//                   MXQUANT, NaN/Inf/saturation/overflow included.
// Both compute kernels run; each reads the stats and returns at once unless the case is its own.
#include <cmath>

#include "mxq_common.h"
#include "mxq_numerics.h"

namespace {

constexpr int kMaxLanes = 64;
constexpr uint32_t kFastAMaxBits = 0x71800000u;   // 2^100: A's rows are staged times up to 2^15

struct SysArgs {
  const float* A;   // K x M
  const float* XA;  // nb x M
  const float* B;   // K x N
  const float* XB;  // nb x N
  float* C;         // M x N
  const uint32_t* stats;  // [max |A| bits, max |B| bits]
  int64_t K, M, N;
  int size, block_size;
  mxq_arith_spec ar;
  int8_t lane_e[kMaxLanes];
  int8_t lane_m[kMaxLanes];
  float fast_prod_max;    // the fast kernel's bound on max|a| * max|b| (see fast_prod_bound)
};

// ---------------------------------------------------------------------------------------------- stats
// stats[j] = max |x| bit pattern over A, B, X_A, X_B (j = 0..3): patterns of non-negative floats order like
// their values, and >= 0x7F800000 means Inf or NaN is present.
struct StatSrc {
  const float* p[4];
  int64_t n[4];
};

__global__ void k_zero4(uint32_t* s) {
  if (threadIdx.x < 4) s[threadIdx.x] = 0u;
}

__global__ void __launch_bounds__(256) k_stats(const StatSrc src, uint32_t* out) {
  __shared__ uint32_t red[4];
  const int which = blockIdx.y;
  const float* __restrict__ x = src.p[which];
  const int64_t n = src.n[which];
  uint32_t mx = 0u;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t n4 = (reinterpret_cast<uintptr_t>(x) % 16 == 0) ? n / 4 : 0;
  const float4* x4 = reinterpret_cast<const float4*>(x);
  for (int64_t i = gid; i < n4; i += stride) {
    const float4 v = x4[i];
    const uint32_t a = f2u(v.x) & 0x7FFFFFFFu, b = f2u(v.y) & 0x7FFFFFFFu, c = f2u(v.z) & 0x7FFFFFFFu,
                   d = f2u(v.w) & 0x7FFFFFFFu;
    const uint32_t ab = a > b ? a : b, cd = c > d ? c : d;
    const uint32_t m4 = ab > cd ? ab : cd;
    mx = m4 > mx ? m4 : mx;
  }
  for (int64_t i = n4 * 4 + gid; i < n; i += stride) {
    const uint32_t u = f2u(x[i]) & 0x7FFFFFFFu;
    mx = u > mx ? u : mx;
  }
  for (int off = 32; off > 0; off >>= 1) {
    const uint32_t o = (uint32_t)__shfl_xor((int)mx, off, 64);
    mx = o > mx ? o : mx;
  }
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mx;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t m = red[0];
    for (int w = 1; w < (int)(blockDim.x >> 6); ++w) m = red[w] > m ? red[w] : m;
    if (m) atomicMax(out + which, m);
  }
}

// The fast kernel's case: finite codes and scales, max|a| < 2^100, max|a| * max|b| <= the lane bound.
__device__ __forceinline__ bool fast_ok(const uint32_t* stats, float prod_max) {
  const uint32_t ua = stats[0], ub = stats[1];
  if (ua >= kFastAMaxBits || ub >= 0x7F800000u || stats[2] >= 0x7F800000u || stats[3] >= 0x7F800000u) return false;
  return u2f(ua) * u2f(ub) <= prod_max;
}

// ------------------------------------------------------------------------------------- tile staging
// Workgroup tile BM x BN outputs, K staged 32 rows at a time through LDS (two buffers).
constexpr int KT = 32;

template <int BM, int BN>
struct Smem {
  float a[2][KT][BM];
  float b[2][KT][BN];
};

// Load rows [k0, k0 + KT) x cols [c0, c0 + W) of a row-major R x L matrix into registers (zero outside).
template <int W, int NT>
struct TileLoader {
  static constexpr int PER = KT * W / NT;  // floats per thread
  float v[PER];
  __device__ __forceinline__ void load(const float* __restrict__ src, int64_t R, int64_t L, int64_t k0, int64_t c0,
                                       bool vec_ok) {
    const int t = threadIdx.x;
    if (vec_ok) {
      // PER / 4 float4 loads per thread: row = (t * 4 + j * NT * 4) / W
#pragma unroll
      for (int j = 0; j < PER / 4; ++j) {
        const int e = (t + j * NT) * 4;
        const int r = e / W, c = e % W;
        const int64_t gr = k0 + r, gc = c0 + c;
        float4 q = make_float4(0.f, 0.f, 0.f, 0.f);
        if (gr < R && gc + 3 < L) q = *reinterpret_cast<const float4*>(src + gr * L + gc);
        else if (gr < R) {
          if (gc < L) q.x = src[gr * L + gc];
          if (gc + 1 < L) q.y = src[gr * L + gc + 1];
          if (gc + 2 < L) q.z = src[gr * L + gc + 2];
        }
        v[j * 4 + 0] = q.x; v[j * 4 + 1] = q.y; v[j * 4 + 2] = q.z; v[j * 4 + 3] = q.w;
      }
    } else {
#pragma unroll
      for (int j = 0; j < PER; ++j) {
        const int e = t + j * NT;
        const int r = e / W, c = e % W;
        const int64_t gr = k0 + r, gc = c0 + c;
        v[j] = (gr < R && gc < L) ? src[gr * L + gc] : 0.0f;
      }
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
};

// ---------------------------------------------------------------------------------- fast datapath
// Per-lane constants of the fast kernel, built on the host from the schedule (see make_fast_lanes).
struct FastLanes {
  int32_t a_exp[32];     // A's rows of lane i are staged times 2^a_exp[i]: 6 + m_i (e4 lanes), 0 (bf16 lane)
  float rescale[32];     // before e4 lane i the scaled sum is multiplied by 2^(m_i - m_{i-1}) (1: unchanged)
  uint32_t half_m1[32];  // bit RNE at m_i fraction bits: add half - 1 + lsb, then mask
  uint32_t lmask[32];
  uint32_t dsh[32];      // 23 - m_i: position of the kept lsb
  float out_scale;       // scaled sum -> sum after the last e4 lane: 2^-(6 + m_last)
  uint32_t pmask;        // product truncation to prod_m fraction bits
  float flush_thr;       // bf16 lane: |product| below this becomes zero
};

// RNE of a float32 bit pattern at 7 fraction bits (bf16).  Finite values, infinities and the quiet NaNs the
// ALU makes (0x7FC00000, 0xFFC00000) map as bf16_rne does; a NaN whose low 16 bits would carry is never
// present here (codes and scales are finite, every NaN is produced by the ALU).
__device__ __forceinline__ float bf16_bits(float x) {
  const uint32_t u = f2u(x);
  return u2f((u + 0x7FFFu + ((u >> 16) & 1u)) & 0xFFFF0000u);
}

// Loads A's stage rows like TileLoader and scales each row by 2^a_exp[lane of the row] on the way to LDS.
// A thread always stages the same rows of a stage (stages start at multiples of 32 and SIZE | 32), so the
// exponents are fixed per thread.
template <int W, int NT, int SIZE>
struct ScaledRows {
  static constexpr int PER = KT * W / NT;
  int ex[PER];
  __device__ __forceinline__ void init(const FastLanes& fl, bool vec_ok) {
    const int t = threadIdx.x;
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      const int e = vec_ok ? (t + (j / 4) * NT) * 4 + (j % 4) : t + j * NT;
      ex[j] = fl.a_exp[(e / W) % SIZE];
    }
  }
  __device__ __forceinline__ void apply(float (&v)[PER]) const {
#pragma unroll
    for (int j = 0; j < PER; ++j) v[j] = ldexpf(v[j], ex[j]);
  }
};

template <int SIZE, bool BF16_LAST>
__global__ void __launch_bounds__(256) k_systolic_fast(const SysArgs args, const FastLanes fl) {
  constexpr int BM = 64, BN = 64, TM = 4, TN = 4, NT = 256;
  if (!fast_ok(args.stats, args.fast_prod_max)) return;
  __shared__ __align__(16) Smem<BM, BN> sm;
  const int tn = threadIdx.x % (BN / TN), tm = threadIdx.x / (BN / TN);
  const int64_t m0 = (int64_t)blockIdx.y * BM, n0 = (int64_t)blockIdx.x * BN;
  const bool va = (args.M % 4 == 0) && (reinterpret_cast<uintptr_t>(args.A) % 16 == 0);
  const bool vb = (args.N % 4 == 0) && (reinterpret_cast<uintptr_t>(args.B) % 16 == 0);
  const int bs = args.block_size;
  const int64_t K = args.K;

  float C[TM][TN];
#pragma unroll
  for (int x = 0; x < TM; ++x)
#pragma unroll
    for (int y = 0; y < TN; ++y) C[x][y] = 0.0f;

  TileLoader<BM, NT> la;
  TileLoader<BN, NT> lb;
  ScaledRows<BM, NT, SIZE> rows;
  rows.init(fl, va);
  int buf = 0;
  la.load(args.A, K, args.M, 0, m0, va);
  lb.load(args.B, K, args.N, 0, n0, vb);
  rows.apply(la.v);
  la.store(sm.a[0], va);
  lb.store(sm.b[0], vb);
  __syncthreads();

  float scale[TM][TN];
  int in_block = 0;      // k of the current reduction within its block
  int64_t g = 0;         // its block
  for (int64_t k0 = 0; k0 < K; k0 += KT) {
    const bool more = k0 + KT < K;
    if (more) {
      la.load(args.A, K, args.M, k0 + KT, m0, va);
      lb.load(args.B, K, args.N, k0 + KT, n0, vb);
    }
    const int kend = (int)((K - k0 < KT) ? (K - k0) : KT);
    // rows past K are zero in LDS: their products are +0 and leave every lane's sum unchanged, so a short
    // last reduction runs as a whole one
    for (int r0 = 0; r0 < kend; r0 += SIZE) {
      if (in_block == 0) {
        float xa[TM], xb[TN];
#pragma unroll
        for (int x = 0; x < TM; ++x) {
          const int64_t mm = m0 + tm * TM + x;
          xa[x] = mm < args.M ? args.XA[g * args.M + mm] : 0.0f;
        }
#pragma unroll
        for (int y = 0; y < TN; ++y) {
          const int64_t nn = n0 + tn * TN + y;
          xb[y] = nn < args.N ? args.XB[g * args.N + nn] : 0.0f;
        }
#pragma unroll
        for (int x = 0; x < TM; ++x)
#pragma unroll
          for (int y = 0; y < TN; ++y) scale[x][y] = xa[x] * xb[y];
      }
      float S[TM][TN];
#pragma unroll
      for (int x = 0; x < TM; ++x)
#pragma unroll
        for (int y = 0; y < TN; ++y) S[x][y] = 0.0f;
#pragma unroll
      for (int i = 0; i < SIZE; ++i) {
        const float4 a4 = *reinterpret_cast<const float4*>(&sm.a[buf][r0 + i][tm * TM]);
        const float4 b4 = *reinterpret_cast<const float4*>(&sm.b[buf][r0 + i][tn * TN]);
        const float a[TM] = {a4.x, a4.y, a4.z, a4.w};
        const float b[TN] = {b4.x, b4.y, b4.z, b4.w};
        if (BF16_LAST && i == SIZE - 1) {
          // bf16 lane: S (an e4 value, at most 8 significant bits) plus the truncated, flushed product
          // (prod_m + 1 <= 8 bits), one float32 add and bit RNE to bf16: rounding an exact sum of two 8-bit
          // precision values first to 24 bits and then to 8 equals rounding it once to 8 (24 >= 2*8 + 1).
#pragma unroll
          for (int x = 0; x < TM; ++x)
#pragma unroll
            for (int y = 0; y < TN; ++y) {
              float t = u2f(f2u(a[x] * b[y]) & fl.pmask);
              t = fabsf(t) < fl.flush_thr ? 0.0f : t;
              S[x][y] = bf16_bits(S[x][y] * fl.out_scale + t);
            }
        } else {
          if (i > 0 && fl.rescale[i] != 1.0f) {
#pragma unroll
            for (int x = 0; x < TM; ++x)
#pragma unroll
              for (int y = 0; y < TN; ++y) S[x][y] *= fl.rescale[i];
          }
          // e4 lane, in units of the lane's subnormal step 2^-(6+m): the truncated product rounded to an
          // integer is lane(p); the sum is exact below 2^24; bit RNE at m fraction bits is the lane rounding
          // (an identity under 2^m, the lane's subnormal range)
          const uint32_t half = fl.half_m1[i], mask = fl.lmask[i], d = fl.dsh[i];
#pragma unroll
          for (int x = 0; x < TM; ++x)
#pragma unroll
            for (int y = 0; y < TN; ++y) {
              const float p = __builtin_rintf(u2f(f2u(a[x] * b[y]) & fl.pmask));
              const uint32_t u = f2u(S[x][y] + p);
              S[x][y] = u2f((u + half + ((u >> d) & 1u)) & mask);
            }
        }
      }
      if (!BF16_LAST) {
#pragma unroll
        for (int x = 0; x < TM; ++x)
#pragma unroll
          for (int y = 0; y < TN; ++y) S[x][y] *= fl.out_scale;
      }
      // tile_add: C (a bf16 value, never -0) plus bf16(S * scale), one rounding to bf16 (same argument)
#pragma unroll
      for (int x = 0; x < TM; ++x)
#pragma unroll
        for (int y = 0; y < TN; ++y) C[x][y] = bf16_bits(C[x][y] + bf16_bits(S[x][y] * scale[x][y]));
      in_block += SIZE;
      if (in_block == bs) {
        in_block = 0;
        ++g;
      }
    }
    if (more) {
      rows.apply(la.v);
      la.store(sm.a[buf ^ 1], va);
      lb.store(sm.b[buf ^ 1], vb);
    }
    __syncthreads();
    buf ^= 1;
  }
#pragma unroll
  for (int x = 0; x < TM; ++x) {
    const int64_t mm = m0 + tm * TM + x;
    if (mm >= args.M) continue;
#pragma unroll
    for (int y = 0; y < TN; ++y) {
      const int64_t nn = n0 + tn * TN + y;
      if (nn < args.N) args.C[mm * args.N + nn] = C[x][y];
    }
  }
}

// ------------------------------------------------------------------------------- general datapath
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

template <int BM, int BN, int TM, int TN>
__global__ void __launch_bounds__((BM / TM) * (BN / TN)) k_systolic_gen(const SysArgs args, int force) {
  constexpr int NT = (BM / TM) * (BN / TN);
  if (!force && fast_ok(args.stats, args.fast_prod_max)) return;
  __shared__ Smem<BM, BN> sm;
  const int tn = threadIdx.x % (BN / TN), tm = threadIdx.x / (BN / TN);
  const int64_t m0 = (int64_t)blockIdx.y * BM, n0 = (int64_t)blockIdx.x * BN;
  const bool va = (args.M % 4 == 0) && (reinterpret_cast<uintptr_t>(args.A) % 16 == 0);
  const bool vb = (args.N % 4 == 0) && (reinterpret_cast<uintptr_t>(args.B) % 16 == 0);
  const int size = args.size, bs = args.block_size;
  float C[TM][TN];
#pragma unroll
  for (int x = 0; x < TM; ++x)
#pragma unroll
    for (int y = 0; y < TN; ++y) C[x][y] = 0.0f;
  TileLoader<BM, NT> la;
  TileLoader<BN, NT> lb;
  const int64_t K = args.K;
  int buf = 0;
  la.load(args.A, K, args.M, 0, m0, va);
  lb.load(args.B, K, args.N, 0, n0, vb);
  la.store(sm.a[0], va);
  lb.store(sm.b[0], vb);
  __syncthreads();
  float scale[TM][TN];
  for (int64_t k0 = 0; k0 < K; k0 += KT) {
    const bool more = k0 + KT < K;
    if (more) {
      la.load(args.A, K, args.M, k0 + KT, m0, va);
      lb.load(args.B, K, args.N, k0 + KT, n0, vb);
    }
    const int kend = (int)((K - k0 < KT) ? (K - k0) : KT);
    for (int r0 = 0; r0 < kend; r0 += size) {
      const int64_t kb = k0 + r0;
      if (kb % bs == 0) {
        const int64_t g = kb / bs;
#pragma unroll
        for (int x = 0; x < TM; ++x) {
          const int64_t mm = m0 + tm * TM + x;
          const float xa = mm < args.M ? args.XA[g * args.M + mm] : 0.0f;
#pragma unroll
          for (int y = 0; y < TN; ++y) {
            const int64_t nn = n0 + tn * TN + y;
            const float xb = nn < args.N ? args.XB[g * args.N + nn] : 0.0f;
            scale[x][y] = xa * xb;
          }
        }
      }
      const int64_t blk_end = (kb / bs + 1) * bs;
      int cnt = size;
      if (kb + cnt > blk_end) cnt = (int)(blk_end - kb);
      if (kb + cnt > K) cnt = (int)(K - kb);
      float S[TM][TN];
#pragma unroll
      for (int x = 0; x < TM; ++x)
#pragma unroll
        for (int y = 0; y < TN; ++y) S[x][y] = 0.0f;
      for (int i = 0; i < cnt; ++i) {
        const int kk = r0 + i;
        const int e = args.lane_e[i], m = args.lane_m[i];
#pragma unroll
        for (int x = 0; x < TM; ++x) {
          const float a = sm.a[buf][kk][tm * TM + x];
#pragma unroll
          for (int y = 0; y < TN; ++y) {
            const float b = sm.b[buf][kk][tn * TN + y];
            S[x][y] = gen_acc(S[x][y], gen_product(a, b, args.ar), e, m, args.ar);
          }
        }
      }
#pragma unroll
      for (int x = 0; x < TM; ++x)
#pragma unroll
        for (int y = 0; y < TN; ++y) C[x][y] = gen_tile(C[x][y], S[x][y] * scale[x][y], args.ar);
    }
    if (more) {
      la.store(sm.a[buf ^ 1], va);
      lb.store(sm.b[buf ^ 1], vb);
    }
    __syncthreads();
    buf ^= 1;
  }
#pragma unroll
  for (int x = 0; x < TM; ++x) {
    const int64_t mm = m0 + tm * TM + x;
    if (mm >= args.M) continue;
#pragma unroll
    for (int y = 0; y < TN; ++y) {
      const int64_t nn = n0 + tn * TN + y;
      if (nn < args.N) args.C[mm * args.N + nn] = C[x][y];
    }
  }
}

// A bound on |product| under which no e4 lane can overflow: with n e4 lanes of at least m_min fraction bits,
// a rounding in the normal range grows a value by a factor of at most 1 + u, u = 2^-(m_min+1), and one in the
// lane's subnormal range by at most 2^-7 absolute, so |S_k| <= P n (1 + u)^(n+1) + n 2^-7; the lanes stay
// finite while that is below 2^8 - 2^(6 - m_min) (the midpoint to 2^8 at m_min bits).
float fast_prod_bound(const int32_t* e, const int32_t* m, int size) {
  int n = 0, mmin = 99;
  for (int i = 0; i < size; ++i) {
    if (e[i] != 4) continue;
    ++n;
    mmin = m[i] < mmin ? m[i] : mmin;
  }
  if (n == 0) return 0.0f;
  const double u = std::ldexp(1.0, -(mmin + 1));
  const double bound = (256.0 - std::ldexp(1.0, 6 - mmin) - n / 128.0) / (n * std::pow(1.0 + u, n + 1));
  return (float)std::floor(bound);   // an integer, safely below the real bound
}

bool lanes_fast(const int32_t* e, const int32_t* m, int size, const mxq_arith_spec& ar) {
  if (ar.kind != MXQ_ARITH_MXGEMMINI || ar.prod_m > 7 || ar.prod_m < 0) return false;
  if (size != 4 && size != 8 && size != 16 && size != 32) return false;
  int prev = -1, mmax = 0, mmin = 99;
  for (int i = 0; i < size; ++i) {
    if (e[i] == 8 && m[i] == 7 && i == size - 1) continue;
    if (e[i] != 4 || m[i] < 1 || m[i] > 9 || m[i] < prev) return false;
    prev = m[i];
    mmax = m[i] > mmax ? m[i] : mmax;
    mmin = m[i] < mmin ? m[i] : mmin;
  }
  if (mmin == 99) return false;                                   // no e4 lane at all
  if (ar.prod_m > mmin) return false;                             // products must sit on every e4 grid
  if (ar.has_floor && !(ar.flush_thr <= pow2f(-7 - mmax))) return false;   // flush under half a step
  if (!(ar.sat_limit >= fast_prod_bound(e, m, size))) return false;   // saturation never reached
  if (e[size - 1] == 8) {
    if (prev > 7) return false;                                   // the bf16 lane holds the e4 sum exactly
    if (!ar.has_floor || !(ar.flush_thr >= pow2f(-126))) return false;   // products under 2^-126 are flushed
  }
  return true;
}

FastLanes make_fast_lanes(const int32_t* e, const int32_t* m, int size, const mxq_arith_spec& ar) {
  FastLanes fl{};
  int prev = -1;
  for (int i = 0; i < size; ++i) {
    fl.rescale[i] = 1.0f;
    if (e[i] == 8) continue;                                      // the bf16 lane: A staged unscaled
    const int mi = m[i];
    fl.a_exp[i] = 6 + mi;
    if (prev >= 0) fl.rescale[i] = pow2f(mi - prev);
    fl.half_m1[i] = (1u << (22 - mi)) - 1u;
    fl.lmask[i] = ~((1u << (23 - mi)) - 1u);
    fl.dsh[i] = (uint32_t)(23 - mi);
    prev = mi;
  }
  fl.out_scale = pow2f(-(6 + prev));
  fl.pmask = ~((1u << (23 - ar.prod_m)) - 1u);
  fl.flush_thr = ar.has_floor ? ar.flush_thr : 0.0f;
  return fl;
}

template <int SIZE>
void launch_fast_size(bool bf16_last, dim3 grid, hipStream_t st, const SysArgs& a, const FastLanes& fl) {
  if (bf16_last) k_systolic_fast<SIZE, true><<<grid, 256, 0, st>>>(a, fl);
  else k_systolic_fast<SIZE, false><<<grid, 256, 0, st>>>(a, fl);
}

void launch_fast(int size, bool bf16_last, dim3 grid, hipStream_t st, const SysArgs& a, const FastLanes& fl) {
  switch (size) {
    case 4: launch_fast_size<4>(bf16_last, grid, st, a, fl); break;
    case 8: launch_fast_size<8>(bf16_last, grid, st, a, fl); break;
    case 16: launch_fast_size<16>(bf16_last, grid, st, a, fl); break;
    default: launch_fast_size<32>(bf16_last, grid, st, a, fl); break;
  }
}

bool lanes_valid(const int32_t* e, const int32_t* m, int size, int kind) {
  for (int i = 0; i < size; ++i) {
    const bool ok = (e[i] == 8 && m[i] == 23) || (e[i] >= 1 && e[i] <= 8 && m[i] >= 1 && m[i] <= 22);
    if (!ok) return false;
  }
  (void)kind;
  return true;
}

}  // namespace

extern "C" int mxq_systolic(const float* P_A, const float* X_A, const float* P_B, const float* X_B, float* C,
                            int64_t K, int64_t M, int64_t N, const int32_t* lane_e, const int32_t* lane_m,
                            int32_t size, int32_t block_size, const mxq_arith_spec* arith, uint32_t* workspace,
                            int32_t force_general, mxq_stream_t stream) {
  if (!arith || !lane_e || !lane_m) return mxq::invalid("mxq_systolic: NULL spec or lanes");
  if (K < 0 || M < 0 || N < 0) return mxq::invalid("mxq_systolic: negative shape");
  if (size < 1 || size > kMaxLanes) return mxq::invalid("mxq_systolic: size must be in [1, 64]");
  if (block_size < 1 || block_size % size) return mxq::invalid("mxq_systolic: size must divide block_size");
  if (KT % size) return mxq::invalid("mxq_systolic: size must divide 32");
  if (arith->kind != MXQ_ARITH_MXGEMMINI && arith->kind != MXQ_ARITH_MXQUANT) return mxq::invalid("mxq_systolic: bad arithmetic");
  if (!lanes_valid(lane_e, lane_m, size, arith->kind)) return mxq::invalid("mxq_systolic: unsupported lane widths");
  if (M == 0 || N == 0) return MXQ_OK;
  if (!P_A || !X_A || !P_B || !X_B || !C || !workspace) return mxq::invalid("mxq_systolic: NULL pointer");
  hipStream_t st = mxq::as_stream(stream);

  SysArgs a{};
  a.A = P_A; a.XA = X_A; a.B = P_B; a.XB = X_B; a.C = C; a.stats = workspace;
  a.K = K; a.M = M; a.N = N; a.size = size; a.block_size = block_size; a.ar = *arith;
  for (int i = 0; i < size; ++i) { a.lane_e[i] = (int8_t)lane_e[i]; a.lane_m[i] = (int8_t)lane_m[i]; }
  a.fast_prod_max = 0.0f;

  const bool fast_lanes = !force_general && K > 0 && lanes_fast(lane_e, lane_m, size, *arith);
  const dim3 grid_f((unsigned)mxq::ceil_div(N, 64), (unsigned)mxq::ceil_div(M, 64));
  const dim3 grid_g((unsigned)mxq::ceil_div(N, 32), (unsigned)mxq::ceil_div(M, 32));
  if (fast_lanes) {
    a.fast_prod_max = fast_prod_bound(lane_e, lane_m, size);
    // statistics decide on the device between the fast and the general kernel; each exits unless it is chosen
    const int64_t nb = mxq::ceil_div(K, block_size);
    StatSrc src{{P_A, P_B, X_A, X_B}, {K * M, K * N, nb * M, nb * N}};
    const int64_t most = K * (M > N ? M : N);
    int64_t sb = mxq::ceil_div(most / 4 + 1, 256);
    sb = sb < 2048 ? sb : 2048;
    k_zero4<<<1, 64, 0, st>>>(workspace);
    k_stats<<<dim3((unsigned)sb, 4), 256, 0, st>>>(src, workspace);
    if (int rc = mxq::check_launch("mxq_systolic stats")) return rc;
    {
      mxq::KernelTimer timer("systolic_fast", st);
      launch_fast(size, lane_e[size - 1] == 8, grid_f, st, a, make_fast_lanes(lane_e, lane_m, size, *arith));
    }
    if (int rc = mxq::check_launch("mxq_systolic fast")) return rc;
    mxq::KernelTimer timer("systolic_general", st);
    k_systolic_gen<32, 32, 2, 2><<<grid_g, 256, 0, st>>>(a, 0);
  } else {
    mxq::KernelTimer timer("systolic_general", st);
    k_systolic_gen<32, 32, 2, 2><<<grid_g, 256, 0, st>>>(a, 1);
  }
  return mxq::check_launch("mxq_systolic");
}
