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
#include <math.h>

#include "mxq_common.h"
#include "mxq_numerics.h"

namespace {

constexpr int H = 2;          // 64-row groups per workgroup
constexpr int RB = 64 * H;    // rows per workgroup
constexpr int NT = 256 * H;   // threads per workgroup: 4 waves per row group

// torch's statistics of one row (lane l's elements l + 64 it)
template <int IT>
__device__ __forceinline__ void row_stats(const float* __restrict__ row, int T, int lane, float& mx, float& sum) {
  float e[IT];
#pragma unroll
  for (int it = 0; it < IT; ++it) {
    const int idx = lane + 64 * it;
    e[it] = idx < T ? row[idx] : -INFINITY;
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

template <int ELEM, int MODE, int IT>
__global__ void __launch_bounds__(NT) k_softmax_pt(const float* __restrict__ S, int64_t R, int T,
                                                    float* __restrict__ PT_P, float* __restrict__ PT_X,
                                                    mxq_block_spec s, uint8_t* __restrict__ stage_live,
                                                    int64_t cols) {
  __shared__ float mx_s[RB], sum_s[RB];
  const int64_t r0 = (int64_t)blockIdx.x * RB;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  // pass 1: each wave takes every (4 H)th row
  for (int j = w; j < RB; j += 4 * H) {
    if (r0 + j >= R) break;
    float mx, sm;
    row_stats<IT>(S + (r0 + j) * T, T, lane, mx, sm);
    if (lane == 0) {
      mx_s[j] = mx;
      sum_s[j] = sm;
    }
  }
  __syncthreads();
  // pass 2: lane m of wave w takes row r0 + 64 (w % H) + m and the key blocks w / H, w / H + 4, ...: the
  // block's 32 probabilities recomputed, its maximum, scale and codes in the lane, and each code stored as
  // P^T[key][row], a run of 64 rows per store across the wave and of 64 H rows across the H waves that take
  // the same blocks (128 rows: 382.5 us against 387.5 with 64 on 32 heads x 2048 causal queries x 2048 keys;
  // no gain at 256)
  const int hg = w % H, wb = w / H;                 // row group, and first key block, of the wave
  const int64_t r = r0 + 64 * hg + lane;
  const bool live = r < R;
  const float mx = mx_s[64 * hg + lane], sm = sum_s[64 * hg + lane];
  const float* src = S + (live ? r : r0) * T;
  const int nb = (T + 31) / 32;
  for (int b = wb; b < nb; b += 4) {
    const int k0 = b * 32;
    float v[32];
    if ((T & 3) == 0 && k0 + 32 <= T) {               // rows 16-byte aligned: 16-byte loads
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        const float4 x = *reinterpret_cast<const float4*>(src + k0 + 4 * q);
        v[4 * q] = x.x; v[4 * q + 1] = x.y; v[4 * q + 2] = x.z; v[4 * q + 3] = x.w;
      }
    } else {
#pragma unroll
      for (int q = 0; q < 32; ++q) v[q] = k0 + q < T ? src[k0 + q] : 0.0f;
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
      const int64_t rh = r0 + 64 * hg + half;
      if ((lane & 31) == 0 && rh < R) {
        const int64_t z = rh / cols, g = (rh - z * cols) / 32;
        stage_live[(z * nb + b) * (cols / 32) + g] = ((bal >> half) & 0xFFFFFFFFull) != 0ull ? 1u : 0u;
      }
    }
  }
}

template <int ELEM, int MODE>
void launch_it(int it, dim3 grid, hipStream_t st, const float* S, int64_t R, int T, float* PT_P, float* PT_X,
               const mxq_block_spec& s, uint8_t* live, int64_t cols) {
  switch (it) {
    case 1: k_softmax_pt<ELEM, MODE, 1><<<grid, NT, 0, st>>>(S, R, T, PT_P, PT_X, s, live, cols); break;
    case 2: k_softmax_pt<ELEM, MODE, 2><<<grid, NT, 0, st>>>(S, R, T, PT_P, PT_X, s, live, cols); break;
    case 4: k_softmax_pt<ELEM, MODE, 4><<<grid, NT, 0, st>>>(S, R, T, PT_P, PT_X, s, live, cols); break;
    case 8: k_softmax_pt<ELEM, MODE, 8><<<grid, NT, 0, st>>>(S, R, T, PT_P, PT_X, s, live, cols); break;
    case 16: k_softmax_pt<ELEM, MODE, 16><<<grid, NT, 0, st>>>(S, R, T, PT_P, PT_X, s, live, cols); break;
    default: k_softmax_pt<ELEM, MODE, 32><<<grid, NT, 0, st>>>(S, R, T, PT_P, PT_X, s, live, cols); break;
  }
}

}  // namespace

extern "C" int mxq_softmax_quantize_t(const float* S, int64_t R, int64_t T, float* PT_P, float* PT_X,
                                      const mxq_block_spec* spec, uint8_t* stage_live, int64_t cols,
                                      mxq_stream_t stream) {
  if (!spec) return mxq::invalid("mxq_softmax_quantize_t: spec is NULL");
  if (R < 0 || T <= 32 || T > 2048) return mxq::invalid("mxq_softmax_quantize_t: needs 32 < T <= 2048 keys");
  if (spec->elem != MXQ_ELEM_OCP || spec->e < 2 || spec->e > 5 || spec->m < 1 || spec->m > 3 || spec->rounding < 0 ||
      spec->rounding > 2 || spec->scale_rule != MXQ_SCALE_MXQUANT || spec->via_e < 0 || spec->via_e > 8)
    return mxq::invalid("mxq_softmax_quantize_t: the spec must be MX-Gemmini's");
  if (stage_live && (cols < 32 || cols % 32 || R % cols))
    return mxq::invalid("mxq_softmax_quantize_t: stage_live needs cols a multiple of 32 dividing R");
  if (R == 0) return MXQ_OK;
  if (!S || !PT_P || !PT_X) return mxq::invalid("mxq_softmax_quantize_t: NULL pointer");
  int it = 1;
  while (64 * it < T) it <<= 1;                        // next_pow2(T) / 64
  const dim3 grid((unsigned)mxq::ceil_div(R, RB));
  hipStream_t st = mxq::as_stream(stream);
  switch (spec->rounding) {
    case MXQ_RNE: launch_it<MXQ_ELEM_OCP, MXQ_RNE>(it, grid, st, S, R, (int)T, PT_P, PT_X, *spec, stage_live, cols); break;
    case MXQ_TIES_AWAY: launch_it<MXQ_ELEM_OCP, MXQ_TIES_AWAY>(it, grid, st, S, R, (int)T, PT_P, PT_X, *spec, stage_live, cols); break;
    default: launch_it<MXQ_ELEM_OCP, MXQ_TRUNC>(it, grid, st, S, R, (int)T, PT_P, PT_X, *spec, stage_live, cols); break;
  }
  return mxq::check_launch("mxq_softmax_quantize_t");
}
