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
//   k_stats         max |code| bit pattern of A and of B (atomic max on the patterns of |x|: patterns of
//                   non-negative floats order like their values; >= 0x7F800000 means Inf or NaN present)
//   k_systolic_fast MXGEMMINI with lanes (4, m <= 9) of non-decreasing m, optionally a last (8, 7) lane,
//                   prod_m <= every e4 lane's m, when the stats show finite codes with max|a| * max|b| <= 8.
//                   Under those conditions the e4 datapath is exactly
//                      t = trunc(a * b)              float32 multiply, mask the dropped significand bits
//                      p = (t + C_m) - C_m           RNE onto the lane's fixed subnormal step 2^(-6-m); identity
//                                                    on t >= 2^-6 (its bits sit on that step); the flush below
//                                                    2^prod_floor is subsumed (it is under half a step)
//                      S = rne_m(S + p)              the sum is exact in float32 (2^4 - 1 + m <= 24), its
//                                                    rounding is bit RNE at m fraction bits; no lane overflows
//                                                    (16 * 8 * (1 + 2^-5)^16 < 2^8 - half a step)
//                   i.e. 8 VALU operations per emulated MAC.  The bf16 lane and the tile add run the general
//                   rule in float64 (exact sums of bf16 grid values, then bit RNE at 7 fraction bits).
//   k_systolic_gen  every other case: the full per-step rule for any codes, any lanes (e <= 8), MXGEMMINI or
//                   MXQUANT, NaN/Inf/saturation/overflow included.
// Both compute kernels run; each reads the stats and returns at once unless the case is its own.
#include "mxq_common.h"
#include "mxq_numerics.h"

namespace {

constexpr int kMaxLanes = 64;
constexpr float kFastProdMax = 8.0f;

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
};

// ---------------------------------------------------------------------------------------------- stats
__global__ void k_zero2(uint32_t* s) {
  if (threadIdx.x < 2) s[threadIdx.x] = 0u;
}

__global__ void __launch_bounds__(256) k_stats(const float* __restrict__ x, int64_t n, uint32_t* out) {
  __shared__ uint32_t red[4];
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
    atomicMax(out, m);
  }
}

__device__ __forceinline__ bool fast_ok(const uint32_t* stats) {
  const uint32_t ua = stats[0], ub = stats[1];
  if (ua >= 0x7F800000u || ub >= 0x7F800000u) return false;
  return u2f(ua) * u2f(ub) <= kFastProdMax;
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
// bf16 lane of MXGEMMINI: exact sum of two bf16 grid values (float64), RNE at 7 fraction bits; the zero
// short-circuit is the sum itself for +0-normalised operands.
__device__ __forceinline__ float bf16_exact_add(float a, float b) {
  const double d = (double)a + (double)b;
  uint64_t u = d2u(d);
  if ((u & 0x7FF0000000000000ull) == 0x7FF0000000000000ull) return (float)d;   // Inf / NaN
  u = (u + 0x00000FFFFFFFFFFFull + ((u >> 45) & 1ull)) & ~0x00001FFFFFFFFFFFull;
  return (float)u2d(u);
}

// tile_add of MXGEMMINI with C already on the bf16 grid (+0 for zero): exact_add(C, uz(bf16(tile)), 8, 7).
__device__ __forceinline__ float tile_add_bf16(float C, float tile) {
  const float t = unsigned_zero(bf16_rne(tile));
  if (C == 0.0f) return t;
  if (t == 0.0f) return C;
  return bf16_exact_add(C, t);
}

template <int TM, int TN>
__device__ __forceinline__ void fast_step_e4(float (&S)[TM][TN], const float (&a)[TM], const float (&b)[TN],
                                             uint32_t pmask, float cm, uint32_t half_m1, uint32_t lmask, uint32_t d) {
#pragma unroll
  for (int x = 0; x < TM; ++x)
#pragma unroll
    for (int y = 0; y < TN; ++y) {
      float t = u2f(f2u(a[x] * b[y]) & pmask);
      t = (t + cm) - cm;
      const uint32_t u = f2u(S[x][y] + t);
      S[x][y] = u2f((u + half_m1 + ((u >> d) & 1u)) & lmask);
    }
}

template <int TM, int TN>
__device__ __forceinline__ void fast_step_bf16(float (&S)[TM][TN], const float (&a)[TM], const float (&b)[TN],
                                               const mxq_arith_spec& ar) {
#pragma unroll
  for (int x = 0; x < TM; ++x)
#pragma unroll
    for (int y = 0; y < TN; ++y) {
      float t = truncate_significand(a[x] * b[y], ar.prod_m);
      if (ar.has_floor) t = flush_product(t, ar.flush_thr);
      const float p = unsigned_zero(bf16_rne(t));
      const float s = unsigned_zero(bf16_rne(S[x][y]));
      S[x][y] = (s == 0.0f) ? p : ((p == 0.0f) ? s : bf16_exact_add(s, p));
    }
}

template <int BM, int BN, int TM, int TN>
__global__ void __launch_bounds__((BM / TM) * (BN / TN)) k_systolic_fast(const SysArgs args) {
  constexpr int NT = (BM / TM) * (BN / TN);
  if (!fast_ok(args.stats)) return;
  __shared__ Smem<BM, BN> sm;
  const int tn = threadIdx.x % (BN / TN), tm = threadIdx.x / (BN / TN);
  const int64_t m0 = (int64_t)blockIdx.y * BM, n0 = (int64_t)blockIdx.x * BN;
  const bool va = (args.M % 4 == 0) && (reinterpret_cast<uintptr_t>(args.A) % 16 == 0);
  const bool vb = (args.N % 4 == 0) && (reinterpret_cast<uintptr_t>(args.B) % 16 == 0);
  const int size = args.size, bs = args.block_size;
  const uint32_t pmask = args.ar.prod_m >= 23 ? 0xFFFFFFFFu : ~((1u << (23 - args.ar.prod_m)) - 1u);
  const bool last_bf16 = args.lane_e[size - 1] == 8;

  float C[TM][TN];
#pragma unroll
  for (int x = 0; x < TM; ++x)
#pragma unroll
    for (int y = 0; y < TN; ++y) C[x][y] = 0.0f;

  TileLoader<BM, NT> la;
  TileLoader<BN, NT> lb;
  const int64_t K = args.K;
  // KT rows of LDS hold one K-block when block_size == KT; other block sizes walk KT-row stages inside blocks.
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
    // walk the stage in reductions; a reduction never straddles a stage because size | block_size and
    // both size and KT are handled so that stage boundaries are multiples of size (size | KT is required)
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
      // the reduction ends at its size, the block's end or K's end, whichever is first
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
        float a[TM], b[TN];
#pragma unroll
        for (int x = 0; x < TM; ++x) a[x] = sm.a[buf][kk][tm * TM + x];
#pragma unroll
        for (int y = 0; y < TN; ++y) b[y] = sm.b[buf][kk][tn * TN + y];
        if (last_bf16 && i == size - 1) {
          fast_step_bf16<TM, TN>(S, a, b, args.ar);
        } else {
          const int m = args.lane_m[i];
          const float cm = u2f(((uint32_t)(127 + 17 - m) << 23) | 0x00400000u);   // 1.5 * 2^(17 - m)
          fast_step_e4<TM, TN>(S, a, b, pmask, cm, (1u << (22 - m)) - 1u, ~((1u << (23 - m)) - 1u),
                               (uint32_t)(23 - m));
        }
      }
#pragma unroll
      for (int x = 0; x < TM; ++x)
#pragma unroll
        for (int y = 0; y < TN; ++y) C[x][y] = tile_add_bf16(C[x][y], S[x][y] * scale[x][y]);
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
  if (!force && fast_ok(args.stats)) return;
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

bool lanes_fast(const int32_t* e, const int32_t* m, int size, const mxq_arith_spec& ar) {
  if (ar.kind != MXQ_ARITH_MXGEMMINI || ar.prod_m > 7 || ar.prod_m < 0) return false;
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
  if (e[size - 1] == 8 && prev > 7) return false;                 // bf16 lane holds the e4 sum exactly
  if (!(ar.sat_limit >= kFastProdMax)) return false;               // saturation never reached
  return true;
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

  const bool fast_lanes = !force_general && K > 0 && lanes_fast(lane_e, lane_m, size, *arith);
  const dim3 grid_f((unsigned)mxq::ceil_div(N, 64), (unsigned)mxq::ceil_div(M, 64));
  const dim3 grid_g((unsigned)mxq::ceil_div(N, 32), (unsigned)mxq::ceil_div(M, 32));
  if (fast_lanes) {
    // statistics decide on the device between the fast and the general kernel; each exits unless it is chosen
    k_zero2<<<1, 64, 0, st>>>(workspace);
    auto sgrid = [](int64_t n) { int64_t b = mxq::ceil_div(n / 4 + 1, 256); return (unsigned)(b < 2048 ? b : 2048); };
    k_stats<<<sgrid(K * M), 256, 0, st>>>(P_A, K * M, workspace);
    k_stats<<<sgrid(K * N), 256, 0, st>>>(P_B, K * N, workspace + 1);
    if (int rc = mxq::check_launch("mxq_systolic stats")) return rc;
    k_systolic_fast<64, 64, 4, 4><<<grid_f, 256, 0, st>>>(a);
    if (int rc = mxq::check_launch("mxq_systolic fast")) return rc;
    k_systolic_gen<32, 32, 2, 2><<<grid_g, 256, 0, st>>>(a, 0);
  } else {
    k_systolic_gen<32, 32, 2, 2><<<grid_g, 256, 0, st>>>(a, 1);
  }
  return mxq::check_launch("mxq_systolic");
}
