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
#include <climits>
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
};

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

template <int WIDTH>
__global__ void __launch_bounds__(256) k_anchor_tree(const TreeArgs args) {
  constexpr int BM = 16, BN = 16, NT = 256, NTERMS = WIDTH + 1, LG = ceil_log2(WIDTH + 1);
  static_assert(KT % WIDTH == 0, "width divides 32");
  static_assert(TileLoader<BM, NT>::PER < 4, "16-wide tiles stage two floats per thread, element by element");
  __shared__ Smem<BM, BN> sm;
  const int tn = threadIdx.x % BN, tm = threadIdx.x / BN;
  const int64_t m0 = (int64_t)blockIdx.y * BM, n0 = (int64_t)blockIdx.x * BN;
  const int64_t K = args.K, M = args.M, N = args.N;
  const bool va = false, vb = false;
  const int size = args.size, trees = args.size / WIDTH, nb = args.nbits;
  const bool rne = args.drop_rne != 0;
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
        // S1: the anchor (the products are kept for S2)
        int top = c != 0.0f ? frexp_label(c) - 1 : INT_MIN;
        float pv[WIDTH];
#pragma unroll
        for (int j = 0; j < WIDTH; ++j) {
          pv[j] = 0.0f;
          if (t * WIDTH + j >= cnt) continue;
          const float a = sm.a[buf][base + j][tm], b = sm.b[buf][base + j][tn];
          pv[j] = gen_product(a, b, args.ar);
          if (pv[j] == 0.0f) continue;
          int lab = frexp_label(a), lbb = frexp_label(b);
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
        const float s = ldexpf(x[0], anchor + 2 - args.bits[t][nb - 1]);
        c = gen_acc(0.0f, s, args.fe[t], args.fm[t], args.ar);
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
                              int32_t size, int32_t block_size, const mxq_arith_spec* arith, mxq_stream_t stream) {
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
  hipStream_t st = mxq::as_stream(stream);
  if (K == 0) return write_zeros(C, M, N, st);
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
                               const mxq_anchor_spec* spec, const mxq_arith_spec* arith, mxq_stream_t stream) {
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
  hipStream_t st = mxq::as_stream(stream);
  if (K == 0) return write_zeros(C, M, N, st);
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
