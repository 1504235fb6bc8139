/* mxq_hip.h -- C ABI of libmxq_hip.so, the gfx950 implementation of mxq's block quantization, LUT and
 * systolic-emulation hot path.
 *
 * Conventions
 *   - Every pointer argument named as an array is device memory (HIP), allocated by the caller; the library
 *     allocates nothing except where an entry point says so.
 *   - Shapes are int64.  A tensor quantized along one axis is viewed as (outer, n, inner), row-major, with the
 *     block axis n in the middle: element (o, k, i) is at (o * n + k) * inner + i.  Its scales are
 *     (outer, ceil(n / block_size), inner).
 *   - `stream` is a hipStream_t (NULL: the default stream).  Kernels are enqueued asynchronously; an entry
 *     point returns before they run, except where it says it synchronises.
 *   - Every entry point returns 0 (MXQ_OK) or an error code; mxq_last_error() then describes the failure
 *     (thread-local, valid until the next call on that thread).
 *   - Rounding codes: 0 ties_away ("nearest"), 1 rne ("even"), 2 truncate ("floor"), the order of
 *     mxq.rounding.MODES.  Grid codes: 0 qtorch, 1 ieee, 2 ocp, the order of mxq.element_quant.float_em.GRIDS.
 *
 * Reference citations are relative to the chloe-wong/microscaling-quant repository.
 */
#ifndef MXQ_HIP_H
#define MXQ_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* mxq_stream_t;

/* ABI revision, returned by mxq_version().  A caller checks it against the header it was built with.
 *   1  the first release.
 *   2  mxq_lut_tables takes the code format (fmt_e, fmt_m) before the grid; mxq_systolic_hints gained a_live
 *      and c_end; mxq_softmax_quantize_t takes a tail; mxq_mask_minabs and mxq_attend_hints give the largest
 *      mask values; mxq_systolic_fast_lanes; the dither entry points.
 *   3  mxq_mx_pack_bytes; the MXQ_EBUSY status of mxq_systolic_noalloc.
 *   4  mxq_attend_windows writes one flag word per call and 64 query rows, each whole (was one per call, zeroed
 *      by the caller). */
#define MXQ_ABI_VERSION 4

enum { MXQ_OK = 0, MXQ_EINVAL = 1, MXQ_EHIP = 2, MXQ_EBUSY = 3 };

/* Input element types of the block quantizer. */
enum { MXQ_DT_F32 = 0, MXQ_DT_BF16 = 1, MXQ_DT_F16 = 2 };

/* Step 1 (scale factor) rules: mxq/scale_factor.py:40-81. */
enum { MXQ_SCALE_NONE = 0, MXQ_SCALE_MXQUANT = 1, MXQ_SCALE_OCP = 2, MXQ_SCALE_OCP_NO_CLIP = 3 };
/* Step 2 (element) rules: float_em grids (mxq/element_quant/float_em.py:53-123) and microxcaling's
 * _quantize_elemwise (mxq/element_quant/microsoft.py:18-23). */
enum { MXQ_ELEM_NONE = 0, MXQ_ELEM_QTORCH = 1, MXQ_ELEM_IEEE = 2, MXQ_ELEM_OCP = 3, MXQ_ELEM_MICROSOFT = 4 };

typedef struct mxq_block_spec {
  int32_t scale_rule;   /* MXQ_SCALE_* */
  float scale_floor;    /* MXQUANT: the float32 value of the floor (1e-38 or 2^-23) */
  int32_t scale_emax;   /* OCP, OCP_NO_CLIP: the format's emax (emax - 1 for placement "below_top") */
  int32_t scale_bits;   /* OCP, OCP_NO_CLIP: E8M0 width (8) */
  int32_t elem;         /* MXQ_ELEM_* */
  int32_t e, m;         /* float_em widths; MICROSOFT: ebits and mbits (sign and implicit bit included) */
  int32_t rounding;     /* rounding code */
  float max_norm;       /* OCP grid and MICROSOFT saturation */
  int32_t via_e, via_m; /* OCP grid only: round on the ieee float(via_e, via_m) grid first; via_e = 0: none */
} mxq_block_spec;

/* The rounding points of a reducer (mxq/matmul/_arithmetic.py:41-134). */
enum { MXQ_ARITH_MXGEMMINI = 0, MXQ_ARITH_MXQUANT = 1 };

typedef struct mxq_arith_spec {
  int32_t kind;          /* MXQ_ARITH_* */
  int32_t prod_e, prod_m;/* product format */
  int32_t has_floor;     /* MXGEMMINI: flush products below flush_thr to +0 */
  float flush_thr;       /* float32 value of 2^prod_floor */
  float sat_limit;       /* MXGEMMINI saturation: |p| > sat_limit becomes sign(p) * sat_value (float32 values) */
  float sat_value;
} mxq_arith_spec;

/* Library identity (MXQ_ABI_VERSION of the header the library was built from) and the last error of the
 * calling thread. */
const char* mxq_last_error(void);
int mxq_version(void);

/* Kernel timing for measurement tools; no counterpart in the reference (the benchmark's roofline needs the
 * dominant kernel's own duration, not the whole call's).  With mxq_timer_enable(1), every later launch of a
 * timed kernel records a pair of HIP events on its stream.  mxq_timer_read waits for the pairs recorded under
 * `kernel`, returns their summed milliseconds and their number, and forgets them.  Timed kernels:
 * "systolic_fast", "systolic_general", "block_quantize", "lut_kmeans", "mx_mfma", "adder_fast", "adder_tree",
 * "anchor_fast", "anchor_tree".  Not for use under graph capture. */
int mxq_timer_enable(int32_t on);
int mxq_timer_read(const char* kernel, double* total_ms, int64_t* launches);

/* VALU issue-rate probe for measurement tools; no counterpart in the reference (the VALU roofline of the
 * emulation kernels prices each instruction by its issue rate).  Launches `workgroups` x 256 threads, each
 * issuing 64 * iters independent instructions of one kind: 0 v_add_f32, 1 v_mul_f32, 2 v_and_b32,
 * 3 v_rndne_f32, 4 v_bfe_u32, 5 v_add3_u32, 6 v_pk_mul_f16, 7 v_pk_add_f16, 8 v_fma_mix_f32,
 * 9 v_cvt_pkrtz_f16_f32, 10 v_cvt_pk_bf16_f32; or one dependent chain of 64 * iters: 11 v_mul_f32,
 * 12 v_pk_mul_f16.  out: workgroups * 256 floats (a sink for the results). */
int mxq_valu_probe(int32_t kind, int32_t iters, int64_t workgroups, float* out, mxq_stream_t stream);

/* Fused block quantization: per block, amax -> scale X (step 1) -> z = block / X -> P = element rule (step 2).
 * V: (outer, n, inner) of type v_dtype; P: float32, same shape; X: float32 (outer, ceil(n/bs), inner).
 * The last block along n is zero-padded for the amax.
 * Replaces mxq/block/_driver.py:45-66 `compose` with the pairs of mxq/block/mxquant.py:26-32,
 * mxq/block/mxgemmini.py:37-59 and mxq/block/ocp.py:35-49. */
int mxq_block_quantize(const void* V, int32_t v_dtype, float* P, float* X, int64_t outer, int64_t n,
                       int64_t inner, int64_t block_size, const mxq_block_spec* spec, mxq_stream_t stream);

/* mxq_block_quantize of V = M^T along axis 0 (V: n x inner, blocks of block_size = 32 along n), reading M
 * (inner x n, row-major, type v_dtype) as it lies: P (n x inner) and X (ceil(n/32) x inner) as mxq_block_quantize
 * writes them for the contiguous V, with no copy of the transposed input.  Replaces the `.t().contiguous()` +
 * quantize of mxq/nn/_attention.py:139 (`pv.a(P.t().contiguous())`) and any axis-0 quantize of a transposed
 * view (mxq/block/_driver.py:45-66). */
int mxq_block_quantize_t(const void* M, int32_t v_dtype, float* P, float* X, int64_t n, int64_t inner,
                         int64_t block_size, const mxq_block_spec* spec, mxq_stream_t stream);

/* out = P * expand(X) along n.  Replaces mxq/block/_driver.py:69-72 `dequantize`. */
int mxq_block_dequantize(const float* P, const float* X, float* out, int64_t outer, int64_t n, int64_t inner,
                         int64_t block_size, mxq_stream_t stream);

/* ---- packed wire formats (no counterpart in the reference, whose codes and scales are float32 tensors) ----
 * Element codes are bytes in the OCP MX layout, sign | e exponent bits | m mantissa bits with bias
 * 2^(e-1) - 1 (the numbering of the reference's element codes, mxq/lut/formats.py:87-99, on every finite value;
 * E5M2 keeps Inf and NaN, E4M3's NaN is S.1111.111, FP6 and FP4 have no specials); (e, m) is one of (4, 3),
 * (5, 2), (3, 2), (2, 3), (2, 1).  Scales are E8M0 bytes: 2^k is k + 127 for k in [-127, 127], NaN is 0xFF; a
 * block whose codes are all zero may have any scale (its values are 0 under any) and gets 0.  Codes are shaped
 * like P and scales like X.  `err` is an int32 device word the caller clears: bit 0 is set when a code is not
 * a value of the format, bit 1 when a scale of a nonzero block is not an E8M0 value. */

/* mxq_block_quantize with the codes and scales written as bytes, in one pass (a quarter of the float32 output
 * bytes).  The element rule must be the qtorch grid (mxquant), the ocp grid (mxgemmini) or the microxcaling step
 * (block.ocp) of an OCP MX format; the code bytes are that format's. */
int mxq_block_quantize_packed(const void* V, int32_t v_dtype, uint8_t* codes, uint8_t* scales, int32_t* err,
                              int64_t outer, int64_t n, int64_t inner, int64_t block_size, const mxq_block_spec* spec,
                              mxq_stream_t stream);

/* float32 codes P and scales X of format (e, m) -> bytes. */
int mxq_pack(const float* P, const float* X, uint8_t* codes, uint8_t* scales, int32_t* err, int64_t outer, int64_t n,
             int64_t inner, int64_t block_size, int32_t e, int32_t m, mxq_stream_t stream);

/* bytes -> float32 codes P and scales X (either may be NULL to skip it).  For a block whose scale mxq_pack or
 * mxq_block_quantize_packed replaced (all-zero codes), X reads 2^-127. */
int mxq_unpack(const uint8_t* codes, const uint8_t* scales, float* P, float* X, int64_t outer, int64_t n,
               int64_t inner, int64_t block_size, int32_t e, int32_t m, mxq_stream_t stream);

/* bytes -> the dequantized values P * expand(X), float32, without materialising P or X; bit-identical to
 * mxq_block_dequantize of the float32 codes and scales the bytes hold. */
int mxq_dequantize_packed(const uint8_t* codes, const uint8_t* scales, float* out, int64_t outer, int64_t n,
                          int64_t inner, int64_t block_size, int32_t e, int32_t m, mxq_stream_t stream);

/* The systolic PE column: C = A^T B (M x N float32) from codes A (K x M), B (K x N) and block scales X_A
 * (ceil(K/block_size) x M), X_B (ceil(K/block_size) x N), all float32 row-major.  Per block of K the scale map
 * X_A[g] (x) X_B[g]; per reduction of `size` k a fresh sum accumulated lane by lane (lane i has the format
 * (lane_e[i], lane_m[i]), host arrays of `size` entries), rescaled and added into C; K tails as the reference.
 * size must divide block_size and 32.  `workspace` is device memory of mxq_systolic_workspace(K, M, N, 1) uint32
 * (which kernel computes each output tile is decided on the device; the call makes no host synchronisation).
 * force_general = 1 skips the fast kernel.  Replaces mxq/matmul/_systolic.py:23-62 with
 * mxq/matmul/_arithmetic.py:64-134. */
int mxq_systolic(const float* P_A, const float* X_A, const float* P_B, const float* X_B, float* C, int64_t K,
                 int64_t M, int64_t N, const int32_t* lane_e, const int32_t* lane_m, int32_t size,
                 int32_t block_size, const mxq_arith_spec* arith, uint32_t* workspace, int32_t force_general,
                 mxq_stream_t stream);

/* Row strides (ld_*) and problem strides (batch_*) in elements: element (r, c) of problem z of an operand is
 * at base + z * batch + r * ld + c. */
typedef struct mxq_systolic_layout {
  int64_t ld_a, batch_a;    /* codes A, K x M   */
  int64_t ld_xa, batch_xa;  /* scales X_A, nb x M */
  int64_t ld_b, batch_b;    /* codes B, K x N   */
  int64_t ld_xb, batch_xb;  /* scales X_B, nb x N */
  int64_t ld_c, batch_c;    /* C, M x N: problems one after another (batch_c >= (M - 1) * ld_c + N) or side
                             * by side within each row (batch_c >= N, (count - 1) * batch_c + N <= ld_c) */
} mxq_systolic_layout;

/* Optional hints to mxq_systolic_batched (no counterpart in the reference; they let attention skip the work its
 * causal mask makes moot).  Either pointer may be NULL; so may the struct.
 *   skip   per problem z, 32-row group i and 32-column group j of C: skip[(z * ceil(M/32) + i) * ceil(N/32) + j]
 *          != 0 marks outputs the caller does not need.  A fast tile made only of such groups is written as +0
 *          and not computed (the general kernel, when it runs alone, computes them); the tiles left to compute
 *          are dispatched first, spread over the whole chip.
 *   k_end  per problem z and 64-column group t of A: k_end[z * ceil(M/64) + t] bounds the rows of A where those
 *          columns hold a nonzero code.  Their reduction stops there (rounded up to 32 rows); the rows left out
 *          are checked by a pass over them (once per problem, not per tile), and unless A is +-0 there and B
 *          and the block scales finite, the tile is recomputed by the general kernel: a wrong k_end costs time,
 *          never bits.  Tiles are dispatched longest reduction first.
 *   a_live with k_end, the check's answer for A made by the caller (attention's softmax writes it with P^T,
 *          mxq_softmax_quantize_t): per problem z, 32-row stage s and 32-column group g of A,
 *          a_live[(z * ceil(K/32) + s) * ceil(M/32) + g] != 0 unless every code of A in those rows and columns
 *          is +-0 and every block scale over them finite.  The pass then reads B only.  A byte that wrongly
 *          says 0 for a stage some tile leaves out gives wrong results: this one is a promise, not a hint.
 *          When the fast kernel runs (mxq_systolic_fast_lanes), a tile it hands to the general kernel for
 *          another reason is recomputed over the same rows when its left-out rows passed the check, so rows of
 *          A past k_end whose a_live bytes are 0 are never read: they need not hold codes or scales at all.
 *   c_end  with skip: per problem z and 64-row group t of C, a fast tile made only of skipped groups whose first
 *          column is at or past c_end[z * ceil(M/64) + t] is not stored at all (those outputs keep what the
 *          buffer held).  Attention's scores past a 64-row group's last seen key are never read: the softmax
 *          takes them from the mask (mxq_softmax_quantize_t's tail). */
typedef struct mxq_systolic_hints {
  const uint8_t* skip;
  const int32_t* k_end;
  const uint8_t* a_live;
  const int32_t* c_end;
} mxq_systolic_hints;

/* 1 when mxq_systolic and mxq_systolic_batched run the fast kernel for these lanes and this arithmetic (any
 * other case runs the general kernel alone, which reads every row of A and computes every tile), else 0.  No
 * counterpart in the reference: a caller that leaves rows of A unwritten under k_end asks this first. */
int mxq_systolic_fast_lanes(const int32_t* lane_e, const int32_t* lane_m, int32_t size, const mxq_arith_spec* arith);

/* An elementwise step mxq_systolic_batched applies to every output as it is stored (no counterpart in the
 * reference as a fused step: it is attention's score step, mxq/nn/_attention.py:128-135, done where the scores
 * are written instead of in a pass of its own).  Output (r, c) of problem z becomes R(R(C * scale) + mask value)
 * in float32, R the identity (bf16 == 0) or bf16 RNE (bf16 != 0); without a mask, R(C * scale).  The mask value
 * is mask[b * mask_b_stride + (r % m) * mask_row_stride + c] with b = (z0 + z) / z_per_b - z0 / z_per_b.  Tiles
 * the skip hint marks take C = +0.  The same step as mxq_scores_scale_mask, bit for bit.  m and z_per_b are at
 * least 1, z0 at least 0, and m, z_per_b and z0 + count below 2^31 (MXQ_EINVAL otherwise). */
typedef struct mxq_systolic_epilogue {
  float scale;
  int32_t bf16;
  const float* mask;
  int64_t mask_b_stride, mask_row_stride;
  int64_t z0, z_per_b, m;
} mxq_systolic_epilogue;

/* `count` independent systolic problems of one shape in one launch, operands addressed through `layout` (any
 * column slice of a larger matrix, any spacing of the problems).  Each problem's result is bit-identical to
 * mxq_systolic on that problem alone (then `epilogue`, when not NULL).  workspace: mxq_systolic_workspace(K, M,
 * N, count) uint32.  The reference
 * calls matmul.systolic once per problem (mxq/nn/_attention.py:108-141, once per head and query chunk);
 * this is that loop as one launch. */
int mxq_systolic_batched(const float* P_A, const float* X_A, const float* P_B, const float* X_B, float* C,
                         const mxq_systolic_layout* layout, int64_t count, int64_t K, int64_t M, int64_t N,
                         const int32_t* lane_e, const int32_t* lane_m, int32_t size, int32_t block_size,
                         const mxq_arith_spec* arith, const mxq_systolic_hints* hints,
                         const mxq_systolic_epilogue* epilogue, uint32_t* workspace, int32_t force_general,
                         mxq_stream_t stream);

/* mxq_systolic without the workspace argument, for callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc).  No counterpart in the reference.  The
 * fast kernel's per-tile flags live in a 1 MiB array the library holds on each GPU (kept until the process
 * ends), so ceil(M/32) * ceil(N/32) may be at most 262144 (M * N up to 2^28 outputs); larger shapes return
 * MXQ_EINVAL.  The call allocates nothing and makes no host synchronisation; the current device must be the
 * stream's.  Every call on one GPU shares that GPU's array, so calls must not overlap on one GPU: a call on
 * another stream than the previous call's, made while that call's kernels may still run (an event recorded
 * behind them is pending), is refused with MXQ_EBUSY before any launch; calls on one stream are ordered by it.
 * Calls made while their stream is captured into a graph are not checked (the caller orders the replays).
 * Results are bit-identical to mxq_systolic's. */
int mxq_systolic_noalloc(const float* P_A, const float* X_A, const float* P_B, const float* X_B, float* C,
                         int64_t K, int64_t M, int64_t N, const int32_t* lane_e, const int32_t* lane_m, int32_t size,
                         int32_t block_size, const mxq_arith_spec* arith, int32_t force_general,
                         mxq_stream_t stream);

/* uint32 elements of workspace mxq_systolic / mxq_systolic_batched need for `count` problems of K x M codes A
 * and K x N codes B (at least 1); mxq_adder_tree and mxq_anchor_tree need the same with count 1. */
int64_t mxq_systolic_workspace(int64_t K, int64_t M, int64_t N, int64_t count);

/* Per contraction row k of codes P (K x cols) with scales X (ceil(K/block_size) x cols), float32 row-major, and
 * per group g of cols/groups adjacent columns: out[k * groups + g] = max over the group of |P[k, c]| *
 * X[k / block_size, c] (float32 products; NaN wins), as float64.  Replaces `_code_amax` of
 * mxq/nn/_attention.py:65-67 for the calls of a batch side by side (one group per call). */
int mxq_group_amax(const float* P, const float* X, int64_t K, int64_t cols, int64_t groups, int64_t block_size,
                   double* out, mxq_stream_t stream);

/* For each of Z attention calls, whether it keeps every key: bound = max(slack_scale * sum over d < D of
 * amax_a[d * lda + z] * amax_k[d * ldk + z], FLT_MIN) (float64), b32 = float(bound); a mask value c absorbs
 * the call's scores when c + b32 == c and c - b32 == c in float32.  flags (Z x ceil(m/64) int32, each written
 * whole: nothing to clear first): word z * ceil(m/64) + c gets bit 0 when the first key block (`block` keys)
 * holds a key that some of the call's query rows [64 c, 64 c + 64) does not absorb, bit 1 for the last block;
 * Tk <= block sets both.  A call keeps every key iff the OR of its words is 3.  Mask rows are addressed as in
 * mxq_scores_scale_mask.  Replaces the bound and `_live_span` == (0, Tk) test of
 * mxq/nn/_attention.py:117-127 for a batch of calls. */
int mxq_attend_windows(const double* amax_a, int64_t lda, const double* amax_k, int64_t ldk, int64_t D, int64_t Z,
                       double slack_scale, const float* mask, int64_t mask_b_stride, int64_t mask_row_stride,
                       int64_t z0, int64_t z_per_b, int64_t m, int64_t Tk, int64_t block, int32_t* flags,
                       mxq_stream_t stream);

/* The batched attention's softmax and P^T quantize in one pass over the scores: for each row of S (R x T
 * float32, 32 < T <= 2048), softmax computed exactly as torch's persistent softmax computes it on this GPU (its
 * element-to-lane order, reduction trees, expf and IEEE division), then P^T (T x R) block-quantized along T in
 * blocks of 32 by spec (MX-Gemmini's: the mxquant scale and the OCP element grid): PT_P (T x R float32 codes),
 * PT_X (ceil(T/32) x R float32 scales), as block.mxgemmini.quantize(softmax(S).t(), axis=0) gives them.
 * Replaces mxq/nn/_attention.py:136-139 (softmax, then pv.a(P.t())) for the batched path.  With stage_live
 * (NULL for none), P^T's columns are R / cols problems of cols each (cols a multiple of 32 dividing R), and
 * stage_live[(z * ceil(T/32) + s) * (cols / 32) + g] gets 1 when problem z's 32 rows s and 32 columns g of P^T
 * hold a nonzero code or a non-finite scale, else 0: the a_live answer of mxq_systolic_hints for the P V
 * product on these codes.
 * With `tail` (NULL for none; needs stage_live and cols a multiple of 64), S holds of each row only the keys
 * below k_end of its 64-row group; a key at or past it has the score R(R(+0 * score.scale) + mask value) of
 * the epilogue `score` (bf16 = 0), whose largest value over the group is tail_max.  A row whose largest stored
 * score s is finite and exceeds tail_max by at least 128 (tail_max - s <= -128 in float32) has every such
 * probability exp(tail - s) / sum = +0 and its maximum and sum over the stored keys alone: it reads nothing
 * else.  Any other row reads those scores from the mask.  When every row of a 64-row group is of the first
 * kind, P^T's rows at and past k_end for those columns are not written (codes +0 and scales of a zero block,
 * which a reader bound by k_end and these stage_live bytes, all 0 there, never reads); otherwise they are. */
typedef struct mxq_softmax_tail {
  const int32_t* k_end;          /* per problem and 64-row group: [z * (cols / 64) + t] */
  const float* tail_max;         /* the same layout */
  mxq_systolic_epilogue score;   /* how the scores were stored: scale, mask rows, z0, z_per_b, m (bf16 = 0) */
} mxq_softmax_tail;

int mxq_softmax_quantize_t(const float* S, int64_t R, int64_t T, float* PT_P, float* PT_X,
                           const mxq_block_spec* spec, uint8_t* stage_live, int64_t cols,
                           const mxq_softmax_tail* tail, mxq_stream_t stream);

/* attend's two elementwise steps on the scores, in place: S (Z problems x n heads x m queries x Tk keys, float32,
 * contiguous) becomes r(r(S * scale) + mask_row), r the identity or (round_bf16 = 1) rounding.bf16; the add and its
 * rounding are skipped when mask is NULL.  Query j of problem z reads the Tk contiguous floats at
 * mask + (floor((z0 + z) / z_per_b) - floor(z0 / z_per_b)) * mask_b_stride + j * mask_row_stride: z0 is the first
 * problem's global index, z_per_b the problems per batch row of the mask (mask_b_stride 0: one shared row set).
 * Replaces mxq/nn/_attention.py:128-135 (`S = r(... * scale)`, `S = r(S + mb[...])`) for a batch of calls. */
int mxq_scores_scale_mask(float* S, int64_t Z, int64_t n, int64_t m, int64_t Tk, float scale, const float* mask,
                          int64_t mask_b_stride, int64_t mask_row_stride, int64_t z0, int64_t z_per_b,
                          int32_t round_bf16, mxq_stream_t stream);

/* The batched attention path's hints to its two systolic launches (no counterpart in the reference: they skip
 * work its computation makes moot, without changing a bit).  mxq_mask_minabs: per mask batch row, 32-row group
 * of the call's `rows` = n*m score rows (row r reads the mask row of query r % m) and 32-key group, the
 * smallest |mask| (0 for a NaN) into out[(batch * ceil(rows/32) + group) * ceil(Tk/32) + key group].
 * With maxval (NULL for none), also the largest mask value of each group, NaN aside (-Inf for none), in the same
 * layout.  mxq_attend_hints: per call z (mask batch row (z0 + z) / z_per_b - z0 / z_per_b when `batched`, else
 * 0), its masked-key bound b as mxq_attend_windows takes it; skip[(z * ceil(rows/32) + g) * ceil(Tk/32) + j] = 1
 * when that group's smallest |mask| c absorbs 2b in float32 (scores there do not matter: the mask absorbs any
 * the call can produce); k_end[z * ceil(rows/64) + t] = 32 * (1 + the last key group some row of 64-row group t
 * still sees), 0 when none; with tail_max (NULL for none; needs maxval), tail_max[z * ceil(rows/64) + t] = the
 * largest maxval of the groups of t past k_end (all of them skipped), -Inf when there are none. */
int mxq_mask_minabs(const float* mask, int64_t mask_b_stride, int64_t mask_row_stride, int64_t batches, int64_t rows,
                    int64_t m, int64_t Tk, float* out, float* maxval, mxq_stream_t stream);
int mxq_attend_hints(const double* amax_a, int64_t lda, const double* amax_k, int64_t ldk, int64_t D, int64_t Z,
                     double slack_scale, const float* minabs, int64_t z0, int64_t z_per_b, int32_t batched,
                     int64_t rows, int64_t Tk, uint8_t* skip, int32_t* k_end, const float* maxval, float* tail_max,
                     mxq_stream_t stream);

/* The adder tree: the operands, Arithmetic, scales and output of mxq_systolic; each reduction of `size` products
 * (zeros past a K tail) summed by log2(size) levels of adjacent-pair acc_adds, level l in (level_e[l],
 * level_m[l]), the root rescaled and tile-added into C.  size: a power of two in [2, 32] dividing block_size.
 * workspace: device memory of mxq_systolic_workspace(K, M, N, 1) uint32.
 * force_general: run the general kernel alone, also where the fast one applies (the two are bit-identical).
 * Replaces mxq/matmul/_adder.py:42-71 (the reduction of :24-32). */
int mxq_adder_tree(const float* P_A, const float* X_A, const float* P_B, const float* X_B, float* C, int64_t K,
                   int64_t M, int64_t N, const int32_t* level_e, const int32_t* level_m, int32_t size,
                   int32_t block_size, const mxq_arith_spec* arith, uint32_t* workspace, int32_t force_general,
                   mxq_stream_t stream);

/* The anchor tree's configuration (mxq/matmul/_anchor.py:96-124): width products per tree; drop 0 truncate,
 * 1 rne; headroom; emin applied to code labels when has_emin; nbits = ceil(log2(width + 1)) + 1 level widths
 * per tree. */
typedef struct mxq_anchor_spec {
  int32_t width, drop, headroom, has_emin, emin, nbits;
} mxq_anchor_spec;

/* The anchor tree: each reduction of `size` products summed by size / width trees chained through a running
 * sum; a tree aligns its products and the sum to one anchor on an integer grid, adds adjacent pairs level by
 * level (tree_bits: trees x nbits widths, non-increasing, each <= 24) and rounds the root once to the tree's
 * lane (tree_e[t], tree_m[t]).  size must divide 32 and block_size, width must divide size.  workspace and
 * force_general as for mxq_adder_tree.
 * Replaces mxq/matmul/_anchor.py:96-138 (trees of :50-82). */
int mxq_anchor_tree(const float* P_A, const float* X_A, const float* P_B, const float* X_B, float* C, int64_t K,
                    int64_t M, int64_t N, const int32_t* tree_e, const int32_t* tree_m, const int32_t* tree_bits,
                    int32_t size, int32_t block_size, const mxq_anchor_spec* spec, const mxq_arith_spec* arith,
                    uint32_t* workspace, int32_t force_general, mxq_stream_t stream);

/* ---- matrix-core comparison product (no counterpart in the reference, whose unrounded comparison is
 * fp64_accum, mxq/_fp64_accum.py:24-29) ---------------------------------------------------------------- */

/* Codes P (K x n float32, exact values of an FP8/FP6/FP4 element format) and block-of-32 scales X
 * (ceil(K/32) x n, powers of two) -> the matrix cores' operand type `kind` (0 FP8 E4M3, 1 BF8 E5M2, 2 FP6 E2M3,
 * 3 BF6 E3M2, 4 FP4 E2M1: w = 8, 8, 6, 6, 4 bits a code; E4M3 also holds every E3M2, E2M3 and E2M1 value) in
 * `codes` (n32 * K64 * w / 8 bytes, n32 = n rounded up to 32, K64 = K rounded up to 64, 16-byte aligned) and
 * E8M0 bytes `scales` (n32 * K64 / 32), both in the matrix-core lane order: for 32-column tile t and 64-deep K
 * step s, lane l = 32h + r (column 32t + r) owns the BPL = 4 w bytes at ((t * K64/64 + s) * 64 + l) * BPL --
 * code j in bits [w j, w j + w): for FP8 codes [16h, 16h + 16) of block 2s, then of block 2s + 1; for FP6 and
 * FP4 the 32 codes of block 2s + h -- and the scale byte (t * K64/64 + s) * 64 + l, block 2s + h's.  Padding is zero codes with scale 1.  *err gets bit 0 set when a
 * code is not exact in that type or a block with nonzero codes has a scale that is not a power of two in
 * [2^-127, 2^127]; the caller clears it first. */
int mxq_mx_pack(const float* P, const float* X, int64_t K, int64_t n, int32_t kind, uint8_t* codes,
                uint8_t* scales, int32_t* err, mxq_stream_t stream);

/* mxq_mx_pack's output from the byte wire format of mxq.packed (no counterpart in the reference): P (K x n
 * bytes, an OCP MX code of `kind` in the low w bits of each) and X (ceil(K/32) x n E8M0 bytes).  The fields are
 * the codes as they are (no conversion).  *err gets bit 0 set when a byte is no finite code of the type (E4M3
 * S.1111.111, E5M2 with its exponent field all ones, FP6 or FP4 bits above w) or a block with a nonzero code
 * has the scale byte 0xFF (NaN); the caller clears it first.  Same layout, padding and limits as mxq_mx_pack. */
int mxq_mx_pack_bytes(const uint8_t* P, const uint8_t* X, int64_t K, int64_t n, int32_t kind, uint8_t* codes,
                      uint8_t* scales, int32_t* err, mxq_stream_t stream);

/* C (M x N float32) = A^T B from packed operands (mxq_mx_pack of A's K x M and B's K x N, of types a_kind and
 * b_kind) on the scaled matrix-core instruction.  Not float32 sums: each group of 8 consecutive k is summed
 * with its products truncated toward zero at 2^(E_g - 13), E_g the group's largest exponent sum; groups and the
 * accumulator then combine with about float32 precision.  Each output adds, in this order, the four float32
 * chains over K steps 0, 4, 8, ...; 1, 5, 9, ...; 2, ...; 3, ... (64 k a step), whatever M and N.
 * |C - exact| <= (2^-7 + ceil(K/64) * 2^-22) * sum_k |a_k b_k|.  K64 must be a
 * positive multiple of 64 (MXQ_EINVAL otherwise, before any launch): an empty contraction is the caller's zeros. */
int mxq_mx_mfma(const uint8_t* A, const uint8_t* SA, int32_t a_kind, const uint8_t* B, const uint8_t* SB,
                int32_t b_kind, float* C, int64_t K64, int64_t M, int64_t N, mxq_stream_t stream);

/* ---- MX-Gemmini look-up tables (K x n float32 block codes, one 16-entry table per 2^group columns) ------ */

/* lut.tables: per column group, the counts of each distinct code value, then weighted k-means in float64
 * (quantile seeds, Lloyd passes until numpy.allclose or max_iters), snap to the finder-safe values, pad with
 * unused safe values smallest magnitude first (safe_order: indices of `safe` sorted by |value|, negative
 * first), sort.  grid: the format's nv distinct finite values ascending; safe: its ns finder-safe values
 * ascending.  (fmt_e, fmt_m): the element format whose codes P holds (a code's grid bin is then read off its
 * bits; 0, 0 or a grid the format does not give: a binary search of the grid instead).  T: ceil(n / 2^group)
 * x 16 float32.  workspace: int32 of ceil(n/2^group) * nv + 1 elements; its last element is set nonzero when P
 * holds a value that is not a code (the caller reports it).
 * Replaces mxq/lut/kmeans.py:46-122. */
int mxq_lut_tables(const float* P, int64_t K, int64_t n, int32_t group, int32_t max_iters, const float* grid,
                   int32_t nv, const float* safe, int32_t ns, const int32_t* safe_order, int32_t fmt_e,
                   int32_t fmt_m, float* T, int32_t* workspace, mxq_stream_t stream);

/* lut.pick: each code's nearest entry of its group's ascending table of `width` entries, ties to the lower
 * index; writes int64 indices to I, or (I NULL) the entries themselves to P_lut (pick then lookup, fused).
 * Replaces mxq/lut/kmeans.py:125-138 (and :141-146 when fused). */
int mxq_lut_pick(const float* P, int64_t K, int64_t n, int32_t group, const float* T, int32_t width, int64_t* I,
                 float* P_lut, mxq_stream_t stream);

/* lut.lookup: out[k][j] = T[j >> group][I[k][j]] (indices already checked in range by the caller).
 * Replaces mxq/lut/kmeans.py:141-146. */
int mxq_lut_lookup(const int64_t* I, int64_t K, int64_t n, int32_t group, const float* T, int32_t width,
                   float* out, mxq_stream_t stream);

/* mxq_lut_pick's indices as the wire's 4-bit nibbles (no counterpart in the reference, which returns int64):
 * row k's byte j / 2 holds column j's index in its low nibble (j even) and column j + 1's in its high one
 * (0 past n); I4 is K x ceil(n / 2) bytes.  width <= 16. */
int mxq_lut_pick_packed(const float* P, int64_t K, int64_t n, int32_t group, const float* T, int32_t width,
                        uint8_t* I4, mxq_stream_t stream);

/* mxq_lut_lookup of 4-bit indices in mxq_lut_pick_packed's layout. */
int mxq_lut_lookup_packed(const uint8_t* I4, int64_t K, int64_t n, int32_t group, const float* T, int32_t width,
                          float* out, mxq_stream_t stream);

/* block.lut along axis 0 in one call: V (K x n, row-major, float32 / bf16 / f16 by v_dtype) block-quantized
 * in blocks of 32 rows by spec (mxgemmini's: the OCP element grid of a LUT format at its own max_norm, no via),
 * the element codes kept as bytes in the workspace while their grid bins are counted per column group, the
 * tables fitted as mxq_lut_tables fits them (T: ceil(n / 2^group) x 16), and every code replaced by its nearest
 * entry: P_lut
 * (K x n float32) and X (ceil(K / 32) x n float32 scales) are what block.lut returns.  grid, nv, safe, ns,
 * safe_order: as mxq_lut_tables, for spec's format.  K >= 1, n % 16 == 0, V, P_lut and X 16-byte aligned.
 * workspace: device memory of mxq_block_lut_workspace bytes, 256-byte aligned.  *err (device) gets bit 0 set
 * when V yields a value that is not a code of the format (a non-finite V), which block.lut reports as
 * lut.tables does; the caller clears it first.
 * Replaces mxq/block/lut.py:23-34 (axis 0: the quantize, mxq/lut/kmeans.py:46-122 and :125-146). */
int mxq_block_lut(const void* V, int32_t v_dtype, int64_t K, int64_t n, const mxq_block_spec* spec, int32_t group,
                  int32_t max_iters, const float* grid, int32_t nv, const float* safe, int32_t ns,
                  const int32_t* safe_order, float* P_lut, float* X, float* T, void* workspace,
                  int64_t workspace_bytes, int32_t* err, mxq_stream_t stream);

/* The bytes of workspace mxq_block_lut needs for a K x n tensor of the element format (fmt_e, fmt_m) whose grid
 * has nv values, at `group` (0 when K or n is 0).  MXQ_EINVAL for what mxq_block_lut refuses (n % 16, a
 * format with no LUT). */
int mxq_block_lut_workspace(int64_t K, int64_t n, int32_t group, int32_t fmt_e, int32_t fmt_m, int32_t nv,
                            int64_t* bytes);

/* lut.finder: fx_all[c] is element code c's fixed point (ncodes entries), lut_fx the fixed points of each
 * group's 16 entries (ceil(n/2^group) x 16); out = argmin over entries of |fx - lut_fx| & mask (mask 0: none),
 * first minimum.  Codes already checked in range by the caller.  Replaces mxq/lut/formats.py:140-159. */
int mxq_lut_finder(const int64_t* codes, int64_t K, int64_t n, int32_t group, const int64_t* fx_all,
                   int32_t ncodes, const int64_t* lut_fx, int64_t mask, int64_t* out, mxq_stream_t stream);

/* ---- elementwise primitives over flat arrays of n elements (the caller broadcasts) ---------------------- */

/* rounding.round_bits on int64 arrays of uint32 patterns; keep per element (int64 array) or, when keep is
 * NULL, keep_scalar.  Replaces mxq/rounding/__init__.py:51-55. */
int mxq_round_bits(const int64_t* bits, const int64_t* keep, int32_t keep_scalar, int64_t* out, int64_t n,
                   int32_t mode, mxq_stream_t stream);

/* rounding.round_int on float32 (dtype 0) or float64 (dtype 3).  Replaces mxq/rounding/__init__.py:58-61. */
int mxq_round_int(const void* k, int32_t dtype, void* out, int64_t n, int32_t mode, mxq_stream_t stream);

/* rounding.bf16.  Replaces mxq/rounding/__init__.py:64-85. */
int mxq_bf16(const float* x, float* out, int64_t n, mxq_stream_t stream);

/* float_em.quantize on a float32 (dtype 0) or float64 (dtype 3) input, float32 out; max_norm for grid ocp.
 * Replaces mxq/element_quant/float_em.py:39-50. */
int mxq_float_em(const void* z, int32_t dtype, float* out, int64_t n, int32_t e, int32_t m, int32_t mode,
                 int32_t grid, float max_norm, mxq_stream_t stream);

/* microxcaling _quantize_elemwise (float formats, allow_denorm) on float32.  Replaces
 * mxq/element_quant/microsoft.py:18-23 (mxq/microxcaling/elemwise.py:63-169). */
int mxq_microsoft(const float* z, float* out, int64_t n, int32_t ebits, int32_t mbits, float max_norm,
                  int32_t mode, int32_t saturate, mxq_stream_t stream);

/* A scale-factor rule of `spec` (MXQUANT, OCP or OCP_NO_CLIP with the MICROSOFT element fields) applied to
 * block maxima.  Replaces mxq/scale_factor.py:40-81. */
int mxq_scale_factor(const float* amax, float* out, int64_t n, const mxq_block_spec* spec, mxq_stream_t stream);

/* microxcaling's "dither" rounding, sign(A) * floor(|A| + u), with the uniforms the caller drew as the reference
 * does (torch.rand_like of the tensor it rounds, in [0, 1)).  mxq_microsoft_dither: mxq_microsoft with u[i]
 * for element i (replaces mxq/element_quant/microsoft.py:18-23 with round="dither",
 * mxq/microxcaling/elemwise.py:41-43).  mxq_scale_factor_dither: OCP_NO_CLIP's rule with u[i] for maximum i
 * (replaces mxq/scale_factor.py:68-81 with rounding_mode="dither").  mxq_block_quantize_dither:
 * mxq_block_quantize for spec's MICROSOFT element rule (its `rounding` field ignored) rounding by dither: element
 * (o, k, i) of V viewed as (outer, n, inner) takes u[((o * inner + i) * nb + k / block_size) * block_size +
 * k % block_size], nb = ceil(n / block_size), the order of the reference's blocked tensor (the block axis moved
 * last, then zero-padded); with OCP_NO_CLIP its block's rounding of amax / X takes u_amax[(o * inner + i) * nb +
 * k / block_size] (NULL otherwise).  Replaces mxq/block/ocp.py:35-49 with rounding_mode="dither". */
int mxq_microsoft_dither(const float* z, const float* u, float* out, int64_t n, int32_t ebits, int32_t mbits,
                         float max_norm, int32_t saturate, mxq_stream_t stream);
int mxq_scale_factor_dither(const float* amax, const float* u, float* out, int64_t n, const mxq_block_spec* spec,
                            mxq_stream_t stream);
int mxq_block_quantize_dither(const void* V, int32_t v_dtype, const float* u_amax, const float* u, float* P,
                              float* X, int64_t outer, int64_t n, int64_t inner, int64_t block_size,
                              const mxq_block_spec* spec, mxq_stream_t stream);

/* arith.exact_add (float32 operands).  Replaces mxq/arith.py:68-103. */
int mxq_exact_add(const float* a, const float* b, float* out, int64_t n, int32_t e, int32_t m, int32_t mode,
                  int32_t grid, float max_norm, mxq_stream_t stream);

/* arith.truncate_significand, flush_product (threshold = float32 2^floor_exp), saturate.
 * Replace mxq/arith.py:106-117, :120-124, :127-137. */
int mxq_truncate_significand(const float* x, float* out, int64_t n, int32_t m, mxq_stream_t stream);
int mxq_flush_product(const float* x, float* out, int64_t n, float threshold, mxq_stream_t stream);
int mxq_saturate(const float* x, float* out, int64_t n, float limit, float value, mxq_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* MXQ_HIP_H */
