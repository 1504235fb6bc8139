// The adder tree and the anchor tree (mxq/matmul/_adder.py, mxq/matmul/_anchor.py): systolic's operands and
// Arithmetic, a different summation of each reduction of `size` products.  Both stage K through LDS 32 rows at
// a time as the general systolic kernel does (size divides 32, so a reduction never straddles a stage) and
// leave the tile add, the block scale map and the K loop order as the reference has them.
//
//   k_adder_tree<SIZE>   2 x 2 outputs per thread.  The size products arrive in k order and are combined as a
//                        binary counter: product i lands on level 0; while bit l of i is set it is added (the
//                        Arithmetic's acc_add in level l's format) to the sum pending on level l, and the
//                        result moves up.  That is the reference's adjacent-pair halving, level by level, with
//                        one pending sum per level instead of all size products (zeros past a K tail).
//   k_anchor_tree<WIDTH> one output per thread.  Per tree of the reduction: pass 1 takes the anchor, the
//                        largest label among the nonzero products (code-exponent sums, frexp's, clamped at
//                        emin when asked) and the running sum c (its exponent minus one), plus headroom;
//                        pass 2 cuts each product (kept in registers from pass 1) and c to integers on the grid
//                        2^(anchor + 2 - bits[0]) (toward zero or to nearest even), then adds adjacent pairs
//                        level by level in float32 (exact: integers below 2^24), c last, an odd term passed up,
//                        regridding where the level width falls; the root goes to float32 once and through the
//                        Arithmetic's lane rounding (acc_add of +0 and the root).
//
// Fast kernels for the common configurations, launched first; as in systolic.hip, each workgroup checks that
// the codes and scales it read allow its shortcuts and otherwise writes only a flag, and the general kernel
// above then computes the flagged tiles alone.
//   k_adder_fast         MXGEMMINI, levels: e4 levels (4, m) of non-decreasing m, then bf16 levels.  With an e4
//                        first level A's rows are staged times 2^(6 + m_1), so a product is in units of that
//                        level's subnormal step and lane(p) = rint(trunc(a' b)) (the flush under half a step is
//                        subsumed).  Every add is one float32 add, exact on e4 levels (integers below 2^24), and
//                        RNE at the level's m (Veltkamp's split, split_rne), which needs no units (m never falls,
//                        so a later level's grid is never coarser than its inputs'); on bf16 levels the float32
//                        add of two 8-bit values rounds once more, harmlessly (24 >= 2 * 8 + 1).  3 + 4 VALU
//                        operations per product, all full-rate but the rint.
//   k_anchor_fast        MXGEMMINI, no emin, equal level widths within each tree (no regridding: a tree is the
//                        exact integer sum of its terms on one grid), bf16 tree lanes.  Pass 1 takes the anchor
//                        from labels kept in LDS as 16-bit integers, two outputs per packed add and max; a zero
//                        code's label is so low that its products never count.  Pass 2 forms each product again,
//                        scales it onto the grid, cuts it and adds it.  A flushed product (below 2^prod_floor)
//                        has a label below any kept one's and falls under one grid step, so neither pass needs
//                        the flush once the anchor is high enough; an output whose tree's anchor is not (all
//                        its products small: about one tree in 10^5 on block-quantized codes) has that tree
//                        computed again by the general rule, in the same kernel.
#include <algorithm>
#include <climits>
#include <cmath>
#include <string>

#include "reducer_common.h"

namespace {

using namespace mxq_red;

constexpr int kMaxStages = 32;   // levels of an adder tree, trees of an anchor reduction (size <= 32)
constexpr int kMaxBits = 8;      // level widths of one anchor tree (width <= 32: 7 entries)

struct TreeArgs {
  const float* A;    // K x M codes
  const float* XA;   // ceil(K / block_size) x M scales
  const float* B;    // K x N codes
  const float* XB;
  float* C;          // M x N
  int64_t K, M, N;
  int size, block_size;
  mxq_arith_spec ar;
  int8_t fe[kMaxStages], fm[kMaxStages];   // adder: per level; anchor: per tree
  int8_t bits[kMaxStages][kMaxBits];       // anchor: per tree, nbits level widths
  int width, nbits, drop_rne, headroom, has_emin, emin;
  uint32_t* flags;        // one per fast tile (1: the general kernel computes it)
  int64_t tiles_x;        // fast tiles per row of C
  int fbm;                // the fast kernel's tile height (64 or 32; its width is FBN)
  int only_flagged;       // general kernel: compute just the tiles whose flag is set
};

constexpr int FBN = 64;                           // the fast kernels' tile width
constexpr uint32_t kFastAMaxBits = 0x71800000u;   // 2^100: A's rows are staged times up to 2^15
constexpr int kZeroLabel = -8192;                 // a zero code's label in the fast anchor kernel

// Whether a general tree kernel's workgroup has a tile to compute: always when run alone, else only when the
// fast tile that holds it was flagged.
__device__ __forceinline__ bool general_tile_wanted(const TreeArgs& a, int BM, int BN) {
  if (!a.only_flagged) return true;
  const int64_t fy = (int64_t)blockIdx.y * BM / a.fbm, fx = (int64_t)blockIdx.x * BN / FBN;
  return a.flags[fy * a.tiles_x + fx] != 0u;
}

constexpr int ilog2(int n) { return n <= 1 ? 0 : 1 + ilog2(n / 2); }
constexpr int ceil_log2(int n) { return n <= 1 ? 0 : 1 + ceil_log2((n + 1) / 2); }

// The block's scale map for a thread's outputs (mxq/matmul/_common.py:32-34): X_A[g][m] * X_B[g][n].
__device__ __forceinline__ float scale_at(const TreeArgs& a, int64_t g, int64_t mm, int64_t nn) {
  const float xa = mm < a.M ? a.XA[g * a.M + mm] : 0.0f;
  const float xb = nn < a.N ? a.XB[g * a.N + nn] : 0.0f;
  return xa * xb;
}

// Number of real products in the reduction starting at row k of the K axis (the rest are zeros).
__device__ __forceinline__ int live_count(int64_t k, int size, int64_t K) {
  return (int)((K - k < size) ? (K - k) : size);
}

template <int SIZE>
__global__ void __launch_bounds__(256) k_adder_tree(const TreeArgs args) {
  constexpr int BM = 32, BN = 32, TM = 2, TN = 2, NT = 256, L = ilog2(SIZE);
  static_assert((1 << L) == SIZE && KT % SIZE == 0, "size: a power of two dividing 32");
  if (!general_tile_wanted(args, BM, BN)) return;
  __shared__ Smem<BM, BN> sm;
  const int tn = threadIdx.x % (BN / TN), tm = threadIdx.x / (BN / TN);
  const int64_t m0 = (int64_t)blockIdx.y * BM, n0 = (int64_t)blockIdx.x * BN;
  const int64_t K = args.K, M = args.M, N = args.N;
  const Operand oa{args.A, M, 0}, ob{args.B, N, 0};
  const bool va = vec_ok(oa, args.A), vb = vec_ok(ob, args.B);
  float C[TM][TN];
#pragma unroll
  for (int x = 0; x < TM; ++x)
#pragma unroll
    for (int y = 0; y < TN; ++y) C[x][y] = 0.0f;
  TileLoader<BM, NT> la;
  TileLoader<BN, NT> lb;
  int buf = 0;
  la.load(args.A, M, K, M, 0, m0, va);
  lb.load(args.B, N, K, N, 0, n0, vb);
  la.store(sm.a[0], va);
  lb.store(sm.b[0], vb);
  __syncthreads();
  float scale[TM][TN];
  int in_block = 0;
  int64_t g = 0;
  for (int64_t k0 = 0; k0 < K; k0 += KT) {
    const bool more = k0 + KT < K;
    if (more) {
      la.load(args.A, M, K, M, k0 + KT, m0, va);
      lb.load(args.B, N, K, N, k0 + KT, n0, vb);
    }
    const int kend = (int)((K - k0 < KT) ? (K - k0) : KT);
    for (int r0 = 0; r0 < kend; r0 += SIZE) {
      if (in_block == 0) {
#pragma unroll
        for (int x = 0; x < TM; ++x)
#pragma unroll
          for (int y = 0; y < TN; ++y) scale[x][y] = scale_at(args, g, m0 + tm * TM + x, n0 + tn * TN + y);
      }
      const int cnt = live_count(k0 + r0, SIZE, K);      // block ends are multiples of SIZE
      float pend[L > 0 ? L : 1][TM][TN];
      float root[TM][TN];
#pragma unroll
      for (int i = 0; i < SIZE; ++i) {
        const bool live = i < cnt;
        float a[TM], b[TN];
#pragma unroll
        for (int x = 0; x < TM; ++x) a[x] = sm.a[buf][r0 + i][tm * TM + x];
#pragma unroll
        for (int y = 0; y < TN; ++y) b[y] = sm.b[buf][r0 + i][tn * TN + y];
#pragma unroll
        for (int x = 0; x < TM; ++x)
#pragma unroll
          for (int y = 0; y < TN; ++y) {
            float v = live ? gen_product(a[x], b[y], args.ar) : 0.0f;
            bool carry = true;                         // v is still moving up
#pragma unroll
            for (int l = 0; l < L; ++l) {
              if (carry) {
                if ((i >> l) & 1) v = gen_acc(pend[l][x][y], v, args.fe[l], args.fm[l], args.ar);
                else {
                  pend[l][x][y] = v;
                  carry = false;
                }
              }
            }
            if (carry) root[x][y] = v;                 // i = SIZE - 1: every level has been added
          }
      }
#pragma unroll
      for (int x = 0; x < TM; ++x)
#pragma unroll
        for (int y = 0; y < TN; ++y) C[x][y] = gen_tile(C[x][y], root[x][y] * scale[x][y], args.ar);
      in_block += SIZE;
      if (in_block >= args.block_size) {
        in_block = 0;
        ++g;
      }
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
    if (mm >= M) continue;
#pragma unroll
    for (int y = 0; y < TN; ++y) {
      const int64_t nn = n0 + tn * TN + y;
      if (nn < N) args.C[mm * N + nn] = C[x][y];
    }
  }
}

// floor(log2|x|) as frexp gives it for a finite nonzero float (subnormals included); -1 for zero and non-finite
// values (mxq/matmul/_anchor.py:36-42).
__device__ __forceinline__ int frexp_label(float x) {
  const uint32_t a = f2u(x) & 0x7FFFFFFFu;
  return (a == 0u || a >= 0x7F800000u) ? -1 : __builtin_amdgcn_frexp_expf(x) - 1;
}

// The grid terms as float32: every term is an integer below 2^(bits[0] - headroom) <= 2^23 (a term's label is at
// most the anchor minus headroom and |term| < 2^(label + 2)), so are the width + 1 of them added in any order
// (headroom >= ceil(log2(width + 1)) + 1), and regridding divides by powers of two: float32 holds all of it
// exactly, as the reference's float64 does.  A term below 2^-126 after the shift rounds to an integer 0 either
// way.  The root's scaling back is the one rounding, as the reference's float64-to-float32 cast.
__device__ __forceinline__ float keep(float x, bool rne) { return rne ? rintf(x) : truncf(x); }

// One anchor tree of one output by the reference's rule (S1-S4, mxq/matmul/_anchor.py:50-82): products of the
// codes a[j * lda] and b[j * ldb] for j < live (zeros after), c the running sum; returns the tree's lane value.
template <int WIDTH>
__device__ __forceinline__ float anchor_tree_general(const float* a, int lda, const float* b, int ldb, int live,
                                                     float c, int t, const TreeArgs& args) {
  constexpr int NTERMS = WIDTH + 1, LG = ceil_log2(WIDTH + 1);
  const bool rne = args.drop_rne != 0;
  // S1: the anchor (the products are kept for S2)
  int top = c != 0.0f ? frexp_label(c) - 1 : INT_MIN;
  float pv[WIDTH];
#pragma unroll
  for (int j = 0; j < WIDTH; ++j) {
    pv[j] = 0.0f;
    if (j >= live) continue;
    const float av = a[j * lda], bv = b[j * ldb];
    pv[j] = gen_product(av, bv, args.ar);
    if (pv[j] == 0.0f) continue;
    int lab = frexp_label(av), lbb = frexp_label(bv);
    if (args.has_emin) {
      lab = max(lab, args.emin);
      lbb = max(lbb, args.emin);
    }
    top = max(top, lab + lbb);
  }
  const int anchor = (top == INT_MIN ? 0 : top) + args.headroom;
  // S2: every term on the grid 2^(anchor + 2 - bits[0]); products first, c last
  const int g0 = anchor + 2 - args.bits[t][0];
  float x[NTERMS];
#pragma unroll
  for (int j = 0; j < WIDTH; ++j) x[j] = keep(ldexpf(pv[j], -g0), rne);
  x[WIDTH] = keep(ldexpf(c, -g0), rne);
  // S3: adjacent pairs level by level, an odd last term passed up, regridding where the width falls
  int n = NTERMS;
#pragma unroll
  for (int lvl = 1; lvl <= LG; ++lvl) {
#pragma unroll
    for (int i = 0; i < NTERMS / 2; ++i)
      if (2 * i + 1 < n) x[i] = x[2 * i] + x[2 * i + 1];
    if (n % 2) x[n / 2] = x[n - 1];
    n = (n + 1) / 2;
    const int drop = args.bits[t][lvl - 1] - args.bits[t][lvl];
    if (drop != 0) {
#pragma unroll
      for (int i = 0; i < NTERMS; ++i)
        if (i < n) x[i] = keep(ldexpf(x[i], -drop), rne);
    }
  }
  // S4: one rounding to float32, then the tree's lane
  const float s = ldexpf(x[0], anchor + 2 - args.bits[t][args.nbits - 1]);
  return gen_acc(0.0f, s, args.fe[t], args.fm[t], args.ar);
}

template <int WIDTH>
__global__ void __launch_bounds__(256) k_anchor_tree(const TreeArgs args) {
  constexpr int BM = 16, BN = 16, NT = 256;
  static_assert(KT % WIDTH == 0, "width divides 32");
  static_assert(TileLoader<BM, NT>::PER < 4, "16-wide tiles stage two floats per thread, element by element");
  if (!general_tile_wanted(args, BM, BN)) return;
  __shared__ Smem<BM, BN> sm;
  const int tn = threadIdx.x % BN, tm = threadIdx.x / BN;
  const int64_t m0 = (int64_t)blockIdx.y * BM, n0 = (int64_t)blockIdx.x * BN;
  const int64_t K = args.K, M = args.M, N = args.N;
  const bool va = false, vb = false;
  const int size = args.size, trees = args.size / WIDTH;
  float C = 0.0f;
  TileLoader<BM, NT> la;
  TileLoader<BN, NT> lb;
  int buf = 0;
  la.load(args.A, M, K, M, 0, m0, va);
  lb.load(args.B, N, K, N, 0, n0, vb);
  la.store(sm.a[0], va);
  lb.store(sm.b[0], vb);
  __syncthreads();
  float scale = 0.0f;
  int in_block = 0;
  int64_t g = 0;
  for (int64_t k0 = 0; k0 < K; k0 += KT) {
    const bool more = k0 + KT < K;
    if (more) {
      la.load(args.A, M, K, M, k0 + KT, m0, va);
      lb.load(args.B, N, K, N, k0 + KT, n0, vb);
    }
    const int kend = (int)((K - k0 < KT) ? (K - k0) : KT);
    for (int r0 = 0; r0 < kend; r0 += size) {
      if (in_block == 0) scale = scale_at(args, g, m0 + tm, n0 + tn);
      const int cnt = live_count(k0 + r0, size, K);
      float c = 0.0f;
      for (int t = 0; t < trees; ++t) {
        const int base = r0 + t * WIDTH;
        c = anchor_tree_general<WIDTH>(&sm.a[buf][base][tm], BM, &sm.b[buf][base][tn], BN, cnt - t * WIDTH, c, t,
                                       args);
      }
      C = gen_tile(C, c * scale, args.ar);
      in_block += size;
      if (in_block >= args.block_size) {
        in_block = 0;
        ++g;
      }
    }
    if (more) {
      la.store(sm.a[buf ^ 1], va);
      lb.store(sm.b[buf ^ 1], vb);
    }
    __syncthreads();
    buf ^= 1;
  }
  const int64_t mm = m0 + tm, nn = n0 + tn;
  if (mm < M && nn < N) args.C[mm * N + nn] = C;
}

// ------------------------------------------------------------------------------------ fast kernels
// RNE of a float32 bit pattern at `dsh` = 23 - m fraction bits (finite values; see systolic.hip's bf16_bits).
__device__ __forceinline__ float rne_bits(float x, uint32_t half_m1, uint32_t dsh, uint32_t mask) {
  const uint32_t u = f2u(x);
  return u2f((u + half_m1 + ((u >> dsh) & 1u)) & mask);
}
__device__ __forceinline__ float bf16_rne(float x) { return rne_bits(x, 0x7FFFu, 16u, 0xFFFF0000u); }

// The workgroup's verdict from every thread's largest |a|, |b| and scale bit patterns: the fast results are
// exact when the codes and scales are finite, max|a| < 2^100 and max|a| * max|b| <= prod_max.  Writes the
// tile's flag; returns whether to write C.
__device__ __forceinline__ bool fast_verdict(const TreeArgs& a, uint32_t max_a, uint32_t max_b, uint32_t max_x,
                                             float prod_max) {
  __shared__ uint32_t red[3][4];
  for (int off = 32; off > 0; off >>= 1) {
    max_a = umax(max_a, (uint32_t)__shfl_xor((int)max_a, off, 64));
    max_b = umax(max_b, (uint32_t)__shfl_xor((int)max_b, off, 64));
    max_x = umax(max_x, (uint32_t)__shfl_xor((int)max_x, off, 64));
  }
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    red[0][wave] = max_a;
    red[1][wave] = max_b;
    red[2][wave] = max_x;
  }
  __syncthreads();
  const uint32_t wa = umax(umax(red[0][0], red[0][1]), umax(red[0][2], red[0][3]));
  const uint32_t wb = umax(umax(red[1][0], red[1][1]), umax(red[1][2], red[1][3]));
  const uint32_t wx = umax(umax(red[2][0], red[2][1]), umax(red[2][2], red[2][3]));
  const bool ok = wa < kFastAMaxBits && wb < 0x7F800000u && wx < 0x7F800000u &&
                  u2f(wa) * u2f(wb) <= prod_max;
  if (threadIdx.x == 0) a.flags[(int64_t)blockIdx.y * a.tiles_x + blockIdx.x] = ok ? 0u : 1u;
  return ok;
}

// The block's scales of a thread's TM x TN outputs (zero outside C), with the largest |scale| bit pattern.
template <int TM, int TN>
__device__ __forceinline__ void block_scales(const TreeArgs& a, int64_t g, int64_t mr, int64_t nc,
                                             float (&scale)[TM][TN], uint32_t& max_x) {
  float xa[TM], xb[TN];
#pragma unroll
  for (int x = 0; x < TM; ++x) {
    xa[x] = mr + x < a.M ? a.XA[g * a.M + mr + x] : 0.0f;
    max_x = umax(max_x, f2u(xa[x]) & 0x7FFFFFFFu);
  }
#pragma unroll
  for (int y = 0; y < TN; ++y) {
    xb[y] = nc + y < a.N ? a.XB[g * a.N + nc + y] : 0.0f;
    max_x = umax(max_x, f2u(xb[y]) & 0x7FFFFFFFu);
  }
#pragma unroll
  for (int x = 0; x < TM; ++x)
#pragma unroll
    for (int y = 0; y < TN; ++y) scale[x][y] = xa[x] * xb[y];
}

template <int TM, int TN>
__device__ __forceinline__ void write_tile(const TreeArgs& a, int64_t mr, int64_t nc, const float (&C)[TM][TN]) {
#pragma unroll
  for (int x = 0; x < TM; ++x) {
    if (mr + x >= a.M) continue;
#pragma unroll
    for (int y = 0; y < TN; ++y)
      if (nc + y < a.N) a.C[(mr + x) * a.N + nc + y] = C[x][y];
  }
}

// A thread's TM rows of one staged k row (TM = 4 or 2), and TN = 4 columns.
template <int TM, int W>
__device__ __forceinline__ void lds_row(const float (*src)[W], int r, int c, float (&v)[TM]) {
  if constexpr (TM == 4) {
    const float4 q = *reinterpret_cast<const float4*>(&src[r][c]);
    v[0] = q.x; v[1] = q.y; v[2] = q.z; v[3] = q.w;
  } else {
    const float2 q = *reinterpret_cast<const float2*>(&src[r][c]);
    v[0] = q.x; v[1] = q.y;
  }
}

// Per-level constants of the fast adder tree, built on the host (make_fast_levels).
struct FastLevels {
  float split[5];     // split_rne's constant 2^(23 - m) + 1 at each level's m (bf16: 7)
  float a_scale;      // A's rows are staged times this: 2^(6 + m_1) for an e4 first level, else 1
  float out_scale;    // root -> value: 1 / a_scale
  uint32_t pmask;     // product truncation to prod_m fraction bits
  float flush_thr;    // bf16 first level: |product| below this becomes +0
  float prod_max;     // bound on max|a| * max|b|: no e4 level overflows, no product saturates
};

// BM = 64: 4 x 4 outputs per thread; BM = 32: 2 x 4, for problems with too few 64 x 64 tiles to fill the chip.
template <int SIZE, int BM, bool FIRST_E4>
__global__ void __launch_bounds__(256) k_adder_fast(const TreeArgs args, const FastLevels fl) {
  constexpr int BN = FBN, TM = BM / 16, TN = 4, NT = 256, L = ilog2(SIZE);
  static_assert((1 << L) == SIZE && KT % SIZE == 0 && L <= 5, "size: a power of two dividing 32");
  static_assert((BM / TM) * (BN / TN) == NT, "256 threads");
  __shared__ __align__(16) Smem<BM, BN> sm;
  const int tn = threadIdx.x % (BN / TN), tm = threadIdx.x / (BN / TN);
  const int64_t m0 = (int64_t)blockIdx.y * BM, n0 = (int64_t)blockIdx.x * BN;
  const int64_t K = args.K, M = args.M, N = args.N;
  const Operand oa{args.A, M, 0}, ob{args.B, N, 0};
  const bool va = vec_ok(oa, args.A), vb = vec_ok(ob, args.B);
  const int bs = args.block_size;
  float C[TM][TN];
#pragma unroll
  for (int x = 0; x < TM; ++x)
#pragma unroll
    for (int y = 0; y < TN; ++y) C[x][y] = 0.0f;
  uint32_t max_a = 0u, max_b = 0u, max_x = 0u;
  TileLoader<BM, NT> la;
  TileLoader<BN, NT> lb;
  auto stage = [&](int to) {
    max_a = umax(max_a, la.max_bits());
    max_b = umax(max_b, lb.max_bits());
    if constexpr (FIRST_E4) {
#pragma unroll
      for (int j = 0; j < TileLoader<BM, NT>::PER; ++j) la.v[j] *= fl.a_scale;   // exact: |a| < 2^100
    }
    la.store(sm.a[to], va);
    lb.store(sm.b[to], vb);
  };
  int buf = 0;
  la.load(args.A, M, K, M, 0, m0, va);
  lb.load(args.B, N, K, N, 0, n0, vb);
  stage(0);
  __syncthreads();
  float scale[TM][TN];
  int in_block = 0;
  int64_t g = 0;
  for (int64_t k0 = 0; k0 < K; k0 += KT) {
    const bool more = k0 + KT < K;
    if (more) {
      la.load(args.A, M, K, M, k0 + KT, m0, va);
      lb.load(args.B, N, K, N, k0 + KT, n0, vb);
    }
    const int kend = (int)((K - k0 < KT) ? (K - k0) : KT);
    // rows past K are zero in LDS: zero products, which is what the reference adds past a K tail
    for (int r0 = 0; r0 < kend; r0 += SIZE) {
      if (in_block == 0) block_scales<TM, TN>(args, g, m0 + tm * TM, n0 + tn * TN, scale, max_x);
      float pend[L][TM][TN];
      float root[TM][TN];
#pragma unroll
      for (int i = 0; i < SIZE; ++i) {
        float a[TM], b[TN];
        lds_row<TM, BM>(sm.a[buf], r0 + i, tm * TM, a);
        lds_row<TN, BN>(sm.b[buf], r0 + i, tn * TN, b);
#pragma unroll
        for (int x = 0; x < TM; ++x)
#pragma unroll
          for (int y = 0; y < TN; ++y) {
            float v = u2f(f2u(a[x] * b[y]) & fl.pmask);
            if constexpr (FIRST_E4) v = __builtin_rintf(v);
            else v = fabsf(v) < fl.flush_thr ? 0.0f : v;
            bool carry = true;                           // i and l are compile-time: this folds away
#pragma unroll
            for (int l = 0; l < L; ++l) {
              if (carry) {
                if ((i >> l) & 1) v = split_rne(pend[l][x][y] + v, fl.split[l]);
                else {
                  pend[l][x][y] = v;
                  carry = false;
                }
              }
            }
            if (carry) root[x][y] = v;
          }
      }
      // tile_add: C (a bf16 value, never -0) plus bf16(root * scale), one rounding to bf16
#pragma unroll
      for (int x = 0; x < TM; ++x)
#pragma unroll
        for (int y = 0; y < TN; ++y) {
          const float r = FIRST_E4 ? root[x][y] * fl.out_scale : root[x][y];
          C[x][y] = bf16_rne(C[x][y] + bf16_rne(r * scale[x][y]));
        }
      in_block += SIZE;
      if (in_block == bs) {
        in_block = 0;
        ++g;
      }
    }
    if (more) stage(buf ^ 1);
    __syncthreads();
    buf ^= 1;
  }
  if (fast_verdict(args, max_a, max_b, max_x, fl.prod_max))
    write_tile<TM, TN>(args, m0 + tm * TM, n0 + tn * TN, C);
}

// Per-tree constants of the fast anchor tree, built on the host (make_fast_anchor).
struct FastAnchor {
  int32_t g_off[kMaxStages];    // grid exponent g0 = top + g_off: headroom + 2 - bits
  int32_t top_min[kMaxStages];  // the lowest top the shortcuts cover (make_fast_anchor)
  uint32_t pmask;
  float prod_max;               // bound on max|a| * max|b|: no product saturates
};

typedef short s16x2 __attribute__((ext_vector_type(2)));

// Two outputs' running label maxima (16-bit halves) against the labels of one k: max(top, la + lb).
__device__ __forceinline__ uint32_t pk_add_max(uint32_t top, uint32_t la, uint32_t lb) {
  const s16x2 t = __builtin_bit_cast(s16x2, top), a = __builtin_bit_cast(s16x2, la),
              b = __builtin_bit_cast(s16x2, lb);
  return __builtin_bit_cast(uint32_t, __builtin_elementwise_max(t, a + b));
}

// floor(log2|x|) of a code (frexp's, subnormals included); kZeroLabel for zero; -1 for non-finite codes
// (the workgroup's verdict rejects those).
__device__ __forceinline__ int code_label(float x) {
  const uint32_t a = f2u(x) & 0x7FFFFFFFu;
  if (a == 0u) return kZeroLabel;
  return a >= 0x7F800000u ? -1 : __builtin_amdgcn_frexp_expf(x) - 1;
}

template <int BM, int BN>
struct AnchorSmem {
  float a[2][KT][BM];
  float b[2][KT][BN];
  uint32_t la[2][KT][BM];    // A's labels, each in both 16-bit halves
  uint16_t lb[2][KT][BN];    // B's labels; a 32-bit read gives two adjacent columns
};

// Writes the labels of a thread's staged values (TileLoader's element order) into LDS.
template <int W, int NT, bool DUP, typename T>
__device__ __forceinline__ void store_labels(const TileLoader<W, NT>& ld, T (*dst)[W], bool vec) {
  const int t = threadIdx.x;
#pragma unroll
  for (int j = 0; j < TileLoader<W, NT>::PER; ++j) {
    const int e = vec ? (t + (j / 4) * NT) * 4 + (j % 4) : t + j * NT;
    const uint32_t l = (uint32_t)code_label(ld.v[j]) & 0xFFFFu;
    dst[e / W][e % W] = (T)(DUP ? (l | (l << 16)) : l);
  }
}

template <int WIDTH, int BM, bool RNE>
__global__ void __launch_bounds__(256) k_anchor_fast(const TreeArgs args, const FastAnchor fa) {
  constexpr int BN = FBN, TM = BM / 16, TN = 4, NT = 256;
  static_assert(KT % WIDTH == 0, "width divides 32");
  static_assert((BM / TM) * (BN / TN) == NT, "256 threads");
  __shared__ __align__(16) AnchorSmem<BM, BN> sm;
  const int tn = threadIdx.x % (BN / TN), tm = threadIdx.x / (BN / TN);
  const int64_t m0 = (int64_t)blockIdx.y * BM, n0 = (int64_t)blockIdx.x * BN;
  const int64_t K = args.K, M = args.M, N = args.N;
  const Operand oa{args.A, M, 0}, ob{args.B, N, 0};
  const bool va = vec_ok(oa, args.A), vb = vec_ok(ob, args.B);
  const int bs = args.block_size, size = args.size, trees = size / WIDTH;
  float C[TM][TN];
#pragma unroll
  for (int x = 0; x < TM; ++x)
#pragma unroll
    for (int y = 0; y < TN; ++y) C[x][y] = 0.0f;
  uint32_t max_a = 0u, max_b = 0u, max_x = 0u;
  TileLoader<BM, NT> la;
  TileLoader<BN, NT> lb;
  auto stage = [&](int to) {
    max_a = umax(max_a, la.max_bits());
    max_b = umax(max_b, lb.max_bits());
    la.store(sm.a[to], va);
    lb.store(sm.b[to], vb);
    store_labels<BM, NT, true>(la, sm.la[to], va);
    store_labels<BN, NT, false>(lb, sm.lb[to], vb);
  };
  int buf = 0;
  la.load(args.A, M, K, M, 0, m0, va);
  lb.load(args.B, N, K, N, 0, n0, vb);
  stage(0);
  __syncthreads();
  float scale[TM][TN];
  int in_block = 0;
  int64_t g = 0;
  for (int64_t k0 = 0; k0 < K; k0 += KT) {
    const bool more = k0 + KT < K;
    if (more) {
      la.load(args.A, M, K, M, k0 + KT, m0, va);
      lb.load(args.B, N, K, N, k0 + KT, n0, vb);
    }
    const int kend = (int)((K - k0 < KT) ? (K - k0) : KT);
    // rows past K are zero in LDS (zero codes): their products are zeros and never set the anchor, as the
    // reference's missing products
    for (int r0 = 0; r0 < kend; r0 += size) {
      if (in_block == 0) block_scales<TM, TN>(args, g, m0 + tm * TM, n0 + tn * TN, scale, max_x);
      float c[TM][TN];
#pragma unroll
      for (int x = 0; x < TM; ++x)
#pragma unroll
        for (int y = 0; y < TN; ++y) c[x][y] = 0.0f;
      for (int t = 0; t < trees; ++t) {
        const int base = r0 + t * WIDTH;
        // S1: the largest label among c (its exponent minus one) and the products (code exponent sums)
        uint32_t top2[TM][TN / 2];
#pragma unroll
        for (int x = 0; x < TM; ++x)
#pragma unroll
          for (int yp = 0; yp < TN / 2; ++yp) {
            uint32_t h[2];
#pragma unroll
            for (int q = 0; q < 2; ++q) {
              const float cv = c[x][2 * yp + q];
              h[q] = (uint32_t)(cv != 0.0f ? __builtin_amdgcn_frexp_expf(cv) - 2 : 2 * kZeroLabel) & 0xFFFFu;
            }
            top2[x][yp] = h[0] | (h[1] << 16);
          }
#pragma unroll
        for (int j = 0; j < WIDTH; ++j) {
          uint32_t lab_a[TM];
          if constexpr (TM == 4) {
            const uint4 q = *reinterpret_cast<const uint4*>(&sm.la[buf][base + j][tm * TM]);
            lab_a[0] = q.x; lab_a[1] = q.y; lab_a[2] = q.z; lab_a[3] = q.w;
          } else {
            const uint2 q = *reinterpret_cast<const uint2*>(&sm.la[buf][base + j][tm * TM]);
            lab_a[0] = q.x; lab_a[1] = q.y;
          }
          const uint2 lab_b = *reinterpret_cast<const uint2*>(&sm.lb[buf][base + j][tn * TN]);
#pragma unroll
          for (int x = 0; x < TM; ++x) {
            top2[x][0] = pk_add_max(top2[x][0], lab_a[x], lab_b.x);
            top2[x][1] = pk_add_max(top2[x][1], lab_a[x], lab_b.y);
          }
        }
        // the grid 2^g0, g0 = anchor + 2 - bits = top + g_off.  A top under top_min with any nonzero code
        // is outside the shortcuts: that output's tree is computed again below by the general rule (rare:
        // all its products small).  A top that low with no nonzero code means every term is zero, on any grid.
        int g0[TM][TN];
        float step_inv[TM][TN], sum[TM][TN];
        uint32_t slow = 0u;                              // bit x * TN + y: the general rule's outputs
        const int tmin = fa.top_min[t], goff = fa.g_off[t];
#pragma unroll
        for (int x = 0; x < TM; ++x)
#pragma unroll
          for (int y = 0; y < TN; ++y) {
            const uint32_t w = top2[x][y / 2];
            const int top = (y & 1) ? ((int)w >> 16) : (int)(short)(w & 0xFFFFu);
            if (top < tmin && top > kZeroLabel + 300) slow |= 1u << (x * TN + y);
            g0[x][y] = (top > tmin ? top : tmin) + goff;
            step_inv[x][y] = ldexpf(1.0f, -g0[x][y]);
            const float cs = c[x][y] * step_inv[x][y];
            sum[x][y] = RNE ? __builtin_rintf(cs) : truncf(cs);   // c's term; products' follow
          }
        // S2 + S3: each product truncated, put on the grid, cut to an integer and added; the sum is exact
        // (integers below 2^23), so its order does not matter
#pragma unroll
        for (int j = 0; j < WIDTH; ++j) {
          float a[TM], b[TN];
          lds_row<TM, BM>(sm.a[buf], base + j, tm * TM, a);
          lds_row<TN, BN>(sm.b[buf], base + j, tn * TN, b);
#pragma unroll
          for (int x = 0; x < TM; ++x)
#pragma unroll
            for (int y = 0; y < TN; ++y) {
              const float v = u2f(f2u(a[x] * b[y]) & fa.pmask) * step_inv[x][y];
              sum[x][y] += RNE ? __builtin_rintf(v) : truncf(v);
            }
        }
        // S4: the root back to float32 (exact), then the tree's bf16 lane
        float cn[TM][TN];
#pragma unroll
        for (int x = 0; x < TM; ++x)
#pragma unroll
          for (int y = 0; y < TN; ++y) cn[x][y] = bf16_rne(ldexpf(sum[x][y], g0[x][y]));
        // the general rule for the marked outputs, one at a time (the selects keep c and cn in registers)
        while (slow != 0u) {
          const int i = __builtin_ctz(slow);
          slow &= slow - 1u;
          float cv = 0.0f;
#pragma unroll
          for (int q = 0; q < TM * TN; ++q) cv = q == i ? c[q / TN][q % TN] : cv;
          const float r = anchor_tree_general<WIDTH>(&sm.a[buf][base][tm * TM + i / TN], BM,
                                                     &sm.b[buf][base][tn * TN + i % TN], BN, WIDTH, cv, t, args);
#pragma unroll
          for (int q = 0; q < TM * TN; ++q) cn[q / TN][q % TN] = q == i ? r : cn[q / TN][q % TN];
        }
#pragma unroll
        for (int x = 0; x < TM; ++x)
#pragma unroll
          for (int y = 0; y < TN; ++y) c[x][y] = cn[x][y];
      }
#pragma unroll
      for (int x = 0; x < TM; ++x)
#pragma unroll
        for (int y = 0; y < TN; ++y) C[x][y] = bf16_rne(C[x][y] + bf16_rne(c[x][y] * scale[x][y]));
      in_block += size;
      if (in_block == bs) {
        in_block = 0;
        ++g;
      }
    }
    if (more) stage(buf ^ 1);
    __syncthreads();
    buf ^= 1;
  }
  if (fast_verdict(args, max_a, max_b, max_x, fa.prod_max))
    write_tile<TM, TN>(args, m0 + tm * TM, n0 + tn * TN, C);
}

// ------------------------------------------------------------------------------------------- host side
bool lane_ok(int e, int m) { return (e == 8 && m == 23) || (e >= 1 && e <= 8 && m >= 1 && m <= 22); }

int check_tree_common(const float* P_A, const float* X_A, const float* P_B, const float* X_B, float* C, int64_t K,
                      int64_t M, int64_t N, int32_t block_size, const mxq_arith_spec* arith, const char* who) {
  if (!arith) return mxq::invalid(std::string(who) + ": NULL arithmetic");
  if (K < 0 || M < 0 || N < 0) return mxq::invalid(std::string(who) + ": negative shape");
  if (arith->kind != MXQ_ARITH_MXGEMMINI && arith->kind != MXQ_ARITH_MXQUANT)
    return mxq::invalid(std::string(who) + ": bad arithmetic");
  if (block_size < 1) return mxq::invalid(std::string(who) + ": bad block size");
  if (mxq::ceil_div(M, 16) > 65535) return mxq::invalid(std::string(who) + ": M too large");
  if (M > 0 && N > 0 && K > 0 && (!P_A || !X_A || !P_B || !X_B)) return mxq::invalid(std::string(who) + ": NULL operand");
  if (M > 0 && N > 0 && !C) return mxq::invalid(std::string(who) + ": NULL output");
  return MXQ_OK;
}

TreeArgs base_args(const float* P_A, const float* X_A, const float* P_B, const float* X_B, float* C, int64_t K,
                   int64_t M, int64_t N, int32_t size, int32_t block_size, const mxq_arith_spec* arith) {
  TreeArgs a{};
  a.A = P_A; a.XA = X_A; a.B = P_B; a.XB = X_B; a.C = C;
  a.K = K; a.M = M; a.N = N; a.size = size; a.block_size = block_size; a.ar = *arith;
  return a;
}

// The fast kernels' tiles: 64 x 64 while they give every CU at least 8 workgroups, else 32 x 64.
void set_fast_tiles(TreeArgs& a) {
  a.tiles_x = mxq::ceil_div(a.N, FBN);
  a.fbm = (mxq::ceil_div(a.M, 64) * a.tiles_x >= 8 * 256) ? 64 : 32;
}

float pow2_host(int k) { return (float)std::ldexp(1.0, k); }

// A bound on |product| under which no e4 level of the fast adder tree overflows.  A value after n e4 levels is
// at most 2^n (P + 2^-7) (1 + u)^(n + 1), u = 2^-(m_min + 1): the first level's rounding of a product adds at
// most half its subnormal step (<= 2^-7) or a relative u, each later one a relative u.  The sum is finite while
// that stays under 2^8 - 2^(6 - m_min), the midpoint between the largest finite value and 2^8.
float adder_e4_bound(int n, int mmin) {
  const double u = std::ldexp(1.0, -(mmin + 1));
  const double b = (256.0 - std::ldexp(1.0, 6 - mmin)) / (std::ldexp(1.0, n) * std::pow(1.0 + u, n + 1)) - 1.0 / 128.0;
  return (float)std::floor(b);
}

// Whether the fast adder kernel takes these levels (see k_adder_fast), and its constants.
bool adder_fast_levels(const int32_t* e, const int32_t* m, int levels, const mxq_arith_spec& ar, FastLevels* fl) {
  if (ar.kind != MXQ_ARITH_MXGEMMINI || ar.prod_m < 0 || ar.prod_m > 7 || levels < 2 || levels > 5) return false;
  int ne = 0, prev = -1, mmin = 99;
  bool bf16 = false;
  for (int l = 0; l < levels; ++l) {
    if (e[l] == 8 && m[l] == 7) {
      bf16 = true;
      continue;
    }
    if (e[l] != 4 || m[l] < 1 || m[l] > 9 || bf16 || m[l] < prev) return false;
    ++ne;
    prev = m[l];
    mmin = std::min(mmin, m[l]);
  }
  if (ne > 0 && bf16 && prev > 7) return false;                     // a bf16 level holds e4 values exactly
  const bool first_e4 = ne > 0;
  if (first_e4) {
    if (ar.prod_m > m[0]) return false;                              // products sit on level 1's grid
    if (ar.has_floor && !(ar.flush_thr <= pow2_host(-7 - m[0]))) return false;   // flush under half a step
  } else if (!ar.has_floor || !(ar.flush_thr >= pow2_host(-126))) {
    return false;                                                    // kept products are normal
  }
  float prod_max = ar.sat_limit;                                     // no product saturates
  if (first_e4) prod_max = std::min(prod_max, adder_e4_bound(ne, mmin));
  if (!(prod_max > 0.0f)) return false;
  *fl = FastLevels{};
  for (int l = 0; l < levels; ++l) {
    const int mm = e[l] == 8 ? 7 : m[l];
    fl->split[l] = (float)((1u << (23 - mm)) + 1u);
  }
  fl->a_scale = first_e4 ? pow2_host(6 + m[0]) : 1.0f;
  fl->out_scale = first_e4 ? pow2_host(-(6 + m[0])) : 1.0f;
  fl->pmask = ~((1u << (23 - ar.prod_m)) - 1u);
  fl->flush_thr = first_e4 ? 0.0f : ar.flush_thr;
  fl->prod_max = prod_max;
  return true;
}

// Whether the fast anchor kernel takes this configuration (see k_anchor_fast), and its constants.  With F the
// product floor's exponent, a tree's top must be at least
//   F                                    so that no flushed product's label (at most F - 1) sets it;
//   F + rne + bits - headroom - 2        so that the grid step 2^g0 is at least 2^(F + rne): a flushed product
//                                        then cuts to 0 (under one step, or under half of one for rne);
//   -120 + bits - headroom - 2           so that g0 >= -120: a product under 2^-126, whose truncation a float32
//                                        mask would misplace, also cuts to 0.
// Without a floor, -100 takes the first two places: a product whose label reaches it is nonzero in float32.
bool anchor_fast_spec(const TreeArgs& a, int width, const int32_t* tree_e, const int32_t* tree_m,
                      const int32_t* tree_bits, FastAnchor* fa) {
  const mxq_arith_spec& ar = a.ar;
  if (ar.kind != MXQ_ARITH_MXGEMMINI || ar.prod_m < 0 || ar.prod_m > 22 || a.has_emin) return false;
  if (width != 4 && width != 8 && width != 16 && width != 32) return false;
  int F = -100;
  if (ar.has_floor) {
    int ex = 0;
    const double fr = std::frexp((double)ar.flush_thr, &ex);
    if (fr != 0.5) return false;                                     // the floor is a power of two
    F = ex - 1;
  }
  const int rne = a.drop_rne ? 1 : 0, trees = a.size / width;
  *fa = FastAnchor{};
  for (int t = 0; t < trees; ++t) {
    if (tree_e[t] != 8 || tree_m[t] != 7) return false;              // bf16 tree lanes
    const int b0 = tree_bits[t * a.nbits];
    for (int l = 1; l < a.nbits; ++l)
      if (tree_bits[t * a.nbits + l] != b0) return false;            // no regridding
    int tmin = ar.has_floor ? std::max(F, F + rne + b0 - a.headroom - 2) : F;
    tmin = std::max(tmin, -120 + b0 - a.headroom - 2);
    fa->top_min[t] = tmin;
    fa->g_off[t] = a.headroom + 2 - b0;
  }
  fa->pmask = ar.prod_m >= 23 ? 0xFFFFFFFFu : ~((1u << (23 - ar.prod_m)) - 1u);
  // no product saturates; labels stay far from where the grid's step leaves float32's normal range
  fa->prod_max = std::min(ar.sat_limit, pow2_host(40));
  return fa->prod_max > 0.0f;
}

template <int SIZE>
void launch_adder_fast(bool first_e4, dim3 grid, hipStream_t st, const TreeArgs& a, const FastLevels& fl) {
  if (a.fbm == 64) {
    if (first_e4) k_adder_fast<SIZE, 64, true><<<grid, 256, 0, st>>>(a, fl);
    else k_adder_fast<SIZE, 64, false><<<grid, 256, 0, st>>>(a, fl);
  } else {
    if (first_e4) k_adder_fast<SIZE, 32, true><<<grid, 256, 0, st>>>(a, fl);
    else k_adder_fast<SIZE, 32, false><<<grid, 256, 0, st>>>(a, fl);
  }
}

template <int WIDTH>
void launch_anchor_fast(dim3 grid, hipStream_t st, const TreeArgs& a, const FastAnchor& fa) {
  if (a.fbm == 64) {
    if (a.drop_rne) k_anchor_fast<WIDTH, 64, true><<<grid, 256, 0, st>>>(a, fa);
    else k_anchor_fast<WIDTH, 64, false><<<grid, 256, 0, st>>>(a, fa);
  } else {
    if (a.drop_rne) k_anchor_fast<WIDTH, 32, true><<<grid, 256, 0, st>>>(a, fa);
    else k_anchor_fast<WIDTH, 32, false><<<grid, 256, 0, st>>>(a, fa);
  }
}

__global__ void __launch_bounds__(256) k_zero_f32(float* __restrict__ p, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    p[i] = 0.0f;
}

// K == 0: every output is +0 (the reference's zeros, with nothing added)
int write_zeros(float* C, int64_t M, int64_t N, hipStream_t st) {
  const int64_t n = M * N, blocks = mxq::ceil_div(n, 256);
  k_zero_f32<<<dim3((unsigned)(blocks < 4096 ? blocks : 4096)), 256, 0, st>>>(C, n);
  return mxq::check_launch("tree zeros");
}

}  // namespace

extern "C" int mxq_adder_tree(const float* P_A, const float* X_A, const float* P_B, const float* X_B, float* C,
                              int64_t K, int64_t M, int64_t N, const int32_t* level_e, const int32_t* level_m,
                              int32_t size, int32_t block_size, const mxq_arith_spec* arith, uint32_t* workspace,
                              int32_t force_general, mxq_stream_t stream) {
  if (int rc = check_tree_common(P_A, X_A, P_B, X_B, C, K, M, N, block_size, arith, "mxq_adder_tree")) return rc;
  if (size < 2 || size > KT || (size & (size - 1)) || block_size % size)
    return mxq::invalid("mxq_adder_tree: size must be a power of two in [2, 32] dividing block_size");
  if (!level_e || !level_m) return mxq::invalid("mxq_adder_tree: NULL level formats");
  const int levels = ilog2(size);
  TreeArgs a = base_args(P_A, X_A, P_B, X_B, C, K, M, N, size, block_size, arith);
  for (int l = 0; l < levels; ++l) {
    if (!lane_ok(level_e[l], level_m[l])) return mxq::invalid("mxq_adder_tree: unsupported level format");
    a.fe[l] = (int8_t)level_e[l];
    a.fm[l] = (int8_t)level_m[l];
  }
  if (M == 0 || N == 0) return MXQ_OK;
  if (!workspace) return mxq::invalid("mxq_adder_tree: NULL workspace");
  hipStream_t st = mxq::as_stream(stream);
  if (K == 0) return write_zeros(C, M, N, st);
  a.flags = workspace;
  set_fast_tiles(a);
  FastLevels fl;
  if (!force_general && adder_fast_levels(level_e, level_m, levels, a.ar, &fl)) {
    const dim3 grid_f((unsigned)a.tiles_x, (unsigned)mxq::ceil_div(M, a.fbm));
    const bool first_e4 = level_e[0] == 4;
    {
      mxq::KernelTimer timer("adder_fast", st);
      switch (size) {
        case 4: launch_adder_fast<4>(first_e4, grid_f, st, a, fl); break;
        case 8: launch_adder_fast<8>(first_e4, grid_f, st, a, fl); break;
        case 16: launch_adder_fast<16>(first_e4, grid_f, st, a, fl); break;
        default: launch_adder_fast<32>(first_e4, grid_f, st, a, fl); break;
      }
    }
    if (int rc = mxq::check_launch("mxq_adder_tree fast")) return rc;
    a.only_flagged = 1;
  }
  const dim3 grid((unsigned)mxq::ceil_div(N, 32), (unsigned)mxq::ceil_div(M, 32));
  mxq::KernelTimer timer("adder_tree", st);
  switch (size) {
    case 2: k_adder_tree<2><<<grid, 256, 0, st>>>(a); break;
    case 4: k_adder_tree<4><<<grid, 256, 0, st>>>(a); break;
    case 8: k_adder_tree<8><<<grid, 256, 0, st>>>(a); break;
    case 16: k_adder_tree<16><<<grid, 256, 0, st>>>(a); break;
    default: k_adder_tree<32><<<grid, 256, 0, st>>>(a); break;
  }
  return mxq::check_launch("mxq_adder_tree");
}

extern "C" int mxq_anchor_tree(const float* P_A, const float* X_A, const float* P_B, const float* X_B, float* C,
                               int64_t K, int64_t M, int64_t N, const int32_t* tree_e, const int32_t* tree_m,
                               const int32_t* tree_bits, int32_t size, int32_t block_size,
                               const mxq_anchor_spec* spec, const mxq_arith_spec* arith, uint32_t* workspace,
                               int32_t force_general, mxq_stream_t stream) {
  if (int rc = check_tree_common(P_A, X_A, P_B, X_B, C, K, M, N, block_size, arith, "mxq_anchor_tree")) return rc;
  if (!spec || !tree_e || !tree_m || !tree_bits) return mxq::invalid("mxq_anchor_tree: NULL spec or tree formats");
  const int width = spec->width;
  if (size < 1 || size > KT || KT % size || block_size % size || width < 1 || size % width)
    return mxq::invalid("mxq_anchor_tree: size must divide 32 and block_size, width must divide size");
  const int lg = ceil_log2(width + 1);
  if (spec->nbits != lg + 1 || spec->nbits > kMaxBits) return mxq::invalid("mxq_anchor_tree: nbits must be ceil(log2(width + 1)) + 1");
  if (spec->headroom < lg + 1 || spec->headroom > 64) return mxq::invalid("mxq_anchor_tree: headroom out of range");
  if (spec->drop != 0 && spec->drop != 1) return mxq::invalid("mxq_anchor_tree: drop must be 0 (truncate) or 1 (rne)");
  TreeArgs a = base_args(P_A, X_A, P_B, X_B, C, K, M, N, size, block_size, arith);
  a.width = width;
  a.nbits = spec->nbits;
  a.drop_rne = spec->drop;
  a.headroom = spec->headroom;
  a.has_emin = spec->has_emin != 0;
  a.emin = spec->emin;
  if (a.has_emin && (a.emin < -1000 || a.emin > 1000)) return mxq::invalid("mxq_anchor_tree: emin out of range");
  const int trees = size / width;
  for (int t = 0; t < trees; ++t) {
    if (!lane_ok(tree_e[t], tree_m[t])) return mxq::invalid("mxq_anchor_tree: unsupported tree format");
    a.fe[t] = (int8_t)tree_e[t];
    a.fm[t] = (int8_t)tree_m[t];
    for (int l = 0; l < spec->nbits; ++l) {
      const int b = tree_bits[t * spec->nbits + l];
      if (b < 1 || b > 24 || (l > 0 && b > tree_bits[t * spec->nbits + l - 1]))
        return mxq::invalid("mxq_anchor_tree: bits must be non-increasing, each in [1, 24]");
      a.bits[t][l] = (int8_t)b;
    }
  }
  if (M == 0 || N == 0) return MXQ_OK;
  if (!workspace) return mxq::invalid("mxq_anchor_tree: NULL workspace");
  hipStream_t st = mxq::as_stream(stream);
  if (K == 0) return write_zeros(C, M, N, st);
  a.flags = workspace;
  set_fast_tiles(a);
  FastAnchor fa;
  if (!force_general && anchor_fast_spec(a, width, tree_e, tree_m, tree_bits, &fa)) {
    const dim3 grid_f((unsigned)a.tiles_x, (unsigned)mxq::ceil_div(M, a.fbm));
    {
      mxq::KernelTimer timer("anchor_fast", st);
      switch (width) {
        case 4: launch_anchor_fast<4>(grid_f, st, a, fa); break;
        case 8: launch_anchor_fast<8>(grid_f, st, a, fa); break;
        case 16: launch_anchor_fast<16>(grid_f, st, a, fa); break;
        default: launch_anchor_fast<32>(grid_f, st, a, fa); break;
      }
    }
    if (int rc = mxq::check_launch("mxq_anchor_tree fast")) return rc;
    a.only_flagged = 1;
  }
  const dim3 grid((unsigned)mxq::ceil_div(N, 16), (unsigned)mxq::ceil_div(M, 16));
  mxq::KernelTimer timer("anchor_tree", st);
  switch (width) {
    case 1: k_anchor_tree<1><<<grid, 256, 0, st>>>(a); break;
    case 2: k_anchor_tree<2><<<grid, 256, 0, st>>>(a); break;
    case 4: k_anchor_tree<4><<<grid, 256, 0, st>>>(a); break;
    case 8: k_anchor_tree<8><<<grid, 256, 0, st>>>(a); break;
    case 16: k_anchor_tree<16><<<grid, 256, 0, st>>>(a); break;
    default: k_anchor_tree<32><<<grid, 256, 0, st>>>(a); break;
  }
  return mxq::check_launch("mxq_anchor_tree");
}
