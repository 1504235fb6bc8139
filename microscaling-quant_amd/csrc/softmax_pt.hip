// Softmax over the scores and the block quantization of its transpose in one kernel, for the batched attention
// path (mxq/nn/_attention.py:136-139: P = softmax(S), then pv.a(P^T) with blocks along the keys).
//
//   k_softmax_pt  S (R rows x T keys) -> P^T codes (T x R) and scales (ceil(T/32) x R), P never stored.
//                 The probabilities are torch's own: its persistent ("warp") softmax for rows of 32 < T <= 2048
//                 keys puts element l + 64 it in lane l (it < next_pow2(T) / 64, -Inf past T), takes the row
//                 maximum with `m > e ? m : e` over it and then an xor butterfly of `a < b ? b : a`, adds
//                 exp(e - max) over it in order and then in an xor butterfly of a + b, and writes exp(e - max) /
//                 sum (NaN for a zero sum).  The same operations in the same order, with the same expf and IEEE
//                 division (measured equal to torch's on MI355X over every float32 exponent argument <= 1), give
//                 the same bits.  Pass 1 takes those row statistics, one wave a row; in pass 2 a lane owns a row
//                 and recomputes the probabilities of one 32-key block of it at a time, quantizes them as the
//                 block they are (its maximum, the scale rule, the division, the element rule) and stores each
//                 code at P^T[key][row], so a wave's store is a run of 64 rows.  With `stage_live`, it also
//                 writes, per 32 keys and 32 rows of P^T, whether any code there is nonzero or any scale
//                 not finite: the answer the P V product's suffix pass would read P^T for (mxq_systolic_hints
//                 a_live).
//                 With a tail (attention under a causal or other absorbing mask), S holds each row's keys below
//                 the k_end of its 64-row group only.  A row whose largest stored score s is finite and at least
//                 128 above the largest score past k_end (tail_max, from the mask) has exp(score - s) = +0 for
//                 every key there: those keys cannot win torch's maximum and add +0 to each lane's sum, so the
//                 statistics over the stored keys are torch's, and their probabilities are +0.  Such a row reads
//                 nothing past k_end.  Any other row reads its scores there from the mask (the value the score
//                 step gives a skipped score, R(R(+0 * scale) + mask)) and takes the full row.  A 64-row group
//                 of rows of the first kind writes nothing of P^T past k_end (codes +0 and scales of a zero
//                 block, which the P V product, bound by k_end and the stage bytes, never reads) and stage
//                 bytes 0 there; a group with a row of the second kind writes every key.
#include <math.h>

#include "mxq_common.h"
#include "mxq_numerics.h"

namespace {

constexpr int H = 2;          // 64-row groups per workgroup
constexpr int RB = 64 * H;    // rows per workgroup
constexpr int NT = 256 * H;   // threads per workgroup: 4 waves per row group
static_assert(H == 2, "a workgroup pairs a front and a back row group");

// torch's statistics of one row: lane l's elements l + 64 it, keys at and past `stored` taken from `tail`
// (a mask row, through the score step) when it is not NULL, else -Inf (no part in the maximum, +0 in the sum)
template <int IT>
__device__ __forceinline__ void row_stats(const float* __restrict__ row, int T, int stored, const float* tail,
                                          float score_scale, int lane, float& mx, float& sum) {
  float e[IT];
#pragma unroll
  for (int it = 0; it < IT; ++it) {
    const int idx = lane + 64 * it;
    e[it] = idx < stored ? row[idx] : (tail && idx < T ? 0.0f * score_scale + tail[idx] : -INFINITY);
  }
  mx = e[0];
#pragma unroll
  for (int it = 0; it < IT; ++it) mx = mx > e[it] ? mx : e[it];
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const float b = __shfl_xor(mx, off, 64);
    mx = mx < b ? b : mx;
  }
  sum = 0.0f;
#pragma unroll
  for (int it = 0; it < IT; ++it) sum += expf(e[it] - mx);
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) sum = sum + __shfl_xor(sum, off, 64);
}

// Where a tail's scores come from: the mask row of S row r (problem r / cols, its row r % cols reading query
// (r % cols) % m of mask batch row (z0 + z) / z_per_b - z0 / z_per_b).
__device__ __forceinline__ const float* tail_row(const mxq_softmax_tail& tl, int64_t cols, int64_t r) {
  const mxq_systolic_epilogue& e = tl.score;
  const int64_t z = r / cols, rp = r - z * cols;
  const int64_t b = (e.z0 + z) / e.z_per_b - e.z0 / e.z_per_b;
  return e.mask + b * e.mask_b_stride + (rp % e.m) * e.mask_row_stride;
}

template <int ELEM, int MODE, int IT>
__global__ void __launch_bounds__(NT) k_softmax_pt(const float* __restrict__ S, int64_t R, int T,
                                                    float* __restrict__ PT_P, float* __restrict__ PT_X,
                                                    mxq_block_spec s, uint8_t* __restrict__ stage_live,
                                                    int64_t cols, mxq_softmax_tail tl, int has_tail) {
  __shared__ float mx_s[RB], sum_s[RB];
  __shared__ uint8_t full_s[RB];     // the row took the full-row path (its scores past k_end from the mask)
  __shared__ int group_full[H];      // some row of the 64-row group did
  // The workgroup's two 64-row groups: the x-th from the front and the x-th from the back of S's G groups.
  // Under a causal mask a group's work grows with its query rows, and every workgroup is resident at once,
  // so pairing a late group with an early one gives each workgroup (and CU) about the same work.
  const int64_t G = (R + 63) / 64;
  int64_t gbase[H];
  bool gvalid[H];
  gbase[0] = (int64_t)blockIdx.x * 64;
  gbase[1] = (G - 1 - (int64_t)blockIdx.x) * 64;
  gvalid[0] = true;
  gvalid[1] = G - 1 - (int64_t)blockIdx.x > (int64_t)blockIdx.x;   // the middle group of an odd G once
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  // k_end and tail_max of each 64-row group (rows of one group share a problem: cols % 64 == 0)
  int ke[H];
  float tmax[H];
#pragma unroll
  for (int g = 0; g < H; ++g) {
    ke[g] = T;
    tmax[g] = -INFINITY;
    if (has_tail && gvalid[g]) {
      const int64_t rg = gbase[g], z = rg / cols, t = (rg - z * cols) / 64;
      const int k = tl.k_end[z * (cols / 64) + t];
      ke[g] = k < 0 ? 0 : (k < T ? k : T);
      tmax[g] = tl.tail_max[z * (cols / 64) + t];
    }
  }
  if (threadIdx.x < H) group_full[threadIdx.x] = 0;
  __syncthreads();
  // pass 1: each wave takes every (4 H)th row
  for (int j = w; j < RB; j += 4 * H) {
    const int g = j / 64;
    const int64_t rr = gbase[g] + (j % 64);
    if (!gvalid[g] || rr >= R) continue;
    const float* row = S + rr * T;
    float mx, sm;
    row_stats<IT>(row, T, ke[g], nullptr, 0.0f, lane, mx, sm);
    bool full = false;
    if (ke[g] < T && !(mx < INFINITY && tmax[g] - mx <= -128.0f)) {       // the same in every lane
      full = true;
      row_stats<IT>(row, T, ke[g], tail_row(tl, cols, rr), tl.score.scale, lane, mx, sm);
    }
    if (lane == 0) {
      mx_s[j] = mx;
      sum_s[j] = sm;
      full_s[j] = full ? 1 : 0;
      if (full) group_full[g] = 1;
    }
  }
  __syncthreads();
  // pass 2: lane m takes row gbase[g] + m of row group g, one 32-key block at a time: the block's 32
  // probabilities recomputed, its maximum, scale and codes in the lane, and each code stored as P^T[key][row],
  // a run of 64 rows per store across the wave.  The two groups' blocks, the first group's first, are dealt to
  // the workgroup's 4 H waves in turn: under a causal mask one group of the pair is short and the other long,
  // and four waves on each left half the waves idle while the others worked through the long group.
  const int nb = (T + 31) / 32;
  int nbw[H];                                       // blocks of P^T written per group
  const float* srcv[H];
  const float* tailv[H];
  float mxv[H], smv[H];
  bool livev[H];
#pragma unroll
  for (int g = 0; g < H; ++g) {
    const int kw = group_full[g] ? T : ke[g];      // keys of P^T written
    nbw[g] = gvalid[g] ? (kw + 31) / 32 : 0;
    const int64_t r = gbase[g] + lane;
    livev[g] = gvalid[g] && r < R;
    mxv[g] = mx_s[64 * g + lane];
    smv[g] = sum_s[64 * g + lane];
    srcv[g] = S + (livev[g] ? r : gbase[0]) * T;
    tailv[g] = livev[g] && full_s[64 * g + lane] ? tail_row(tl, cols, r) : nullptr;
  }
  for (int i = w; i < nbw[0] + nbw[1]; i += 4 * H) {
    const int hg = i < nbw[0] ? 0 : 1;              // the same in every lane
    const int b = hg == 0 ? i : i - nbw[0];
    const int64_t r = gbase[hg] + lane;
    const bool live = livev[hg];
    const float mx = mxv[hg], sm = smv[hg];
    const float* src = srcv[hg];
    const float* tail = tailv[hg];
    const int kg = ke[hg];                          // keys stored in S for this group
    const int k0 = b * 32;
    float v[32];
    if ((T & 3) == 0 && k0 + 32 <= kg) {              // rows 16-byte aligned: 16-byte loads
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        const float4 x = *reinterpret_cast<const float4*>(src + k0 + 4 * q);
        v[4 * q] = x.x; v[4 * q + 1] = x.y; v[4 * q + 2] = x.z; v[4 * q + 3] = x.w;
      }
    } else {
#pragma unroll
      for (int q = 0; q < 32; ++q) {
        const int k = k0 + q;
        v[q] = k < kg ? src[k] : (tail && k < T ? 0.0f * tl.score.scale + tail[k] : -INFINITY);
      }
    }
    uint32_t am = 0u;
#pragma unroll
    for (int q = 0; q < 32; ++q) {
      const float pr = k0 + q < T ? (sm == 0.0f ? NAN : expf(v[q] - mx) / sm) : 0.0f;  // past T: padding
      v[q] = pr;
      am = max(am, f2u(pr) & 0x7FFFFFFFu);           // a NaN pattern lies above +Inf: NaN wins, as torch.amax
    }
    const float xs = block_scale(u2f(am), s);
    const Div d = make_div(xs);
    uint32_t nz = 0u;                                  // the OR of this row's |code| bits over the block
    if (live) {
      PT_X[(int64_t)b * R + r] = xs;
#pragma unroll
      for (int q = 0; q < 32; ++q)
        if (k0 + q < T) {
          const float code = elem_qm<ELEM, MODE>(s.scale_rule ? apply_div(v[q], d) : v[q], s);
          PT_P[(int64_t)(k0 + q) * R + r] = code;
          nz |= f2u(code) & 0x7FFFFFFFu;
        }
    }
    if (stage_live) {
      // per 32 rows (a half wave, inside one problem: cols % 32 == 0): any nonzero code or non-finite scale
      const uint64_t bal = __ballot(live && (nz != 0u || !(fabsf(xs) < INFINITY)));
      const int half = lane & 32;
      const int64_t rh = gbase[hg] + half;
      if ((lane & 31) == 0 && gvalid[hg] && rh < R) {
        const int64_t z = rh / cols, g = (rh - z * cols) / 32;
        stage_live[(z * nb + b) * (cols / 32) + g] = ((bal >> half) & 0xFFFFFFFFull) != 0ull ? 1u : 0u;
      }
    }
  }
  // the blocks past the written keys: codes +0, a zero block's scale, so their stage bytes are 0
  if (stage_live) {
    const int half = lane & 32;
#pragma unroll
    for (int hg = 0; hg < H; ++hg) {
      const int64_t rh = gbase[hg] + half;
      if ((lane & 31) == 0 && gvalid[hg] && rh < R && nbw[hg] < nb) {
        const int64_t z = rh / cols, g = (rh - z * cols) / 32;
        for (int b = nbw[hg] + w; b < nb; b += 4 * H) stage_live[(z * nb + b) * (cols / 32) + g] = 0u;
      }
    }
  }
}

template <int ELEM, int MODE>
void launch_it(int it, dim3 grid, hipStream_t st, const float* S, int64_t R, int T, float* PT_P, float* PT_X,
               const mxq_block_spec& s, uint8_t* live, int64_t cols, const mxq_softmax_tail& tl, int has_tail) {
  switch (it) {
    case 1: k_softmax_pt<ELEM, MODE, 1><<<grid, NT, 0, st>>>(S, R, T, PT_P, PT_X, s, live, cols, tl, has_tail); break;
    case 2: k_softmax_pt<ELEM, MODE, 2><<<grid, NT, 0, st>>>(S, R, T, PT_P, PT_X, s, live, cols, tl, has_tail); break;
    case 4: k_softmax_pt<ELEM, MODE, 4><<<grid, NT, 0, st>>>(S, R, T, PT_P, PT_X, s, live, cols, tl, has_tail); break;
    case 8: k_softmax_pt<ELEM, MODE, 8><<<grid, NT, 0, st>>>(S, R, T, PT_P, PT_X, s, live, cols, tl, has_tail); break;
    case 16: k_softmax_pt<ELEM, MODE, 16><<<grid, NT, 0, st>>>(S, R, T, PT_P, PT_X, s, live, cols, tl, has_tail); break;
    default: k_softmax_pt<ELEM, MODE, 32><<<grid, NT, 0, st>>>(S, R, T, PT_P, PT_X, s, live, cols, tl, has_tail); break;
  }
}

}  // namespace

extern "C" int mxq_softmax_quantize_t(const float* S, int64_t R, int64_t T, float* PT_P, float* PT_X,
                                      const mxq_block_spec* spec, uint8_t* stage_live, int64_t cols,
                                      const mxq_softmax_tail* tail, mxq_stream_t stream) {
  if (!spec) return mxq::invalid("mxq_softmax_quantize_t: spec is NULL");
  if (R < 0 || T <= 32 || T > 2048) return mxq::invalid("mxq_softmax_quantize_t: needs 32 < T <= 2048 keys");
  if (spec->elem != MXQ_ELEM_OCP || spec->e < 2 || spec->e > 5 || spec->m < 1 || spec->m > 3 || spec->rounding < 0 ||
      spec->rounding > 2 || spec->scale_rule != MXQ_SCALE_MXQUANT || spec->via_e < 0 || spec->via_e > 8)
    return mxq::invalid("mxq_softmax_quantize_t: the spec must be MX-Gemmini's");
  if (stage_live && (cols < 32 || cols % 32 || R % cols))
    return mxq::invalid("mxq_softmax_quantize_t: stage_live needs cols a multiple of 32 dividing R");
  mxq_softmax_tail tl{};
  if (tail) {
    const mxq_systolic_epilogue& e = tail->score;
    if (!stage_live || cols % 64)
      return mxq::invalid("mxq_softmax_quantize_t: a tail needs stage_live and cols a multiple of 64");
    if (!tail->k_end || !tail->tail_max || !e.mask || e.bf16 || e.m < 1 || e.z_per_b < 1 || e.z0 < 0 ||
        e.mask_b_stride < 0 || e.mask_row_stride < 0)
      return mxq::invalid("mxq_softmax_quantize_t: a tail needs k_end, tail_max and a float32 score step with "
                          "a mask (m and z_per_b at least 1)");
    tl = *tail;
  }
  if (R == 0) return MXQ_OK;
  if (!S || !PT_P || !PT_X) return mxq::invalid("mxq_softmax_quantize_t: NULL pointer");
  int it = 1;
  while (64 * it < T) it <<= 1;                        // next_pow2(T) / 64
  const dim3 grid((unsigned)mxq::ceil_div(mxq::ceil_div(R, 64), H));   // a front and a back 64-row group each
  hipStream_t st = mxq::as_stream(stream);
  const int ht = tail ? 1 : 0;
  switch (spec->rounding) {
    case MXQ_RNE: launch_it<MXQ_ELEM_OCP, MXQ_RNE>(it, grid, st, S, R, (int)T, PT_P, PT_X, *spec, stage_live, cols, tl, ht); break;
    case MXQ_TIES_AWAY: launch_it<MXQ_ELEM_OCP, MXQ_TIES_AWAY>(it, grid, st, S, R, (int)T, PT_P, PT_X, *spec, stage_live, cols, tl, ht); break;
    default: launch_it<MXQ_ELEM_OCP, MXQ_TRUNC>(it, grid, st, S, R, (int)T, PT_P, PT_X, *spec, stage_live, cols, tl, ht); break;
  }
  return mxq::check_launch("mxq_softmax_quantize_t");
}
