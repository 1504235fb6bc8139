// Issue-rate probe behind the VALU roofline of the emulation kernels (no counterpart in the reference; the
// benchmark's --valu-rates mode runs it).  Kinds 0-10 stream one gfx950 VALU instruction through eight
// independent register chains, 64 instructions per loop trip, so consecutive instructions never wait on each
// other and the launch's duration gives that instruction's issue rate: wave instructions per SIMD per clock, or
// lane-operations per second over the chip.  Kinds 11 and 12 run one dependent chain (v_mul_f32, v_pk_mul_f16):
// launched with one wave per SIMD, the time from an instruction to the next that reads its result.
#include "mxq_common.h"

namespace {

#define MXQ_REP8(X) X X X X X X X X
#define MXQ_CHAINS(OP, A)                                                                                       \
  MXQ_REP8(OP " %0, " A "%0\n " OP " %1, " A "%1\n " OP " %2, " A "%2\n " OP " %3, " A "%3\n " OP " %4, " A       \
           "%4\n " OP " %5, " A "%5\n " OP " %6, " A "%6\n " OP " %7, " A "%7\n")

template <int KIND>
__global__ void __launch_bounds__(256) k_valu_probe(int iters, float* __restrict__ out) {
  float r0 = (float)threadIdx.x, r1 = r0 + 1.0f, r2 = r0 + 2.0f, r3 = r0 + 3.0f, r4 = r0 + 4.0f, r5 = r0 + 5.0f,
        r6 = r0 + 6.0f, r7 = r0 + 7.0f;
  for (int it = 0; it < iters; ++it) {
    if constexpr (KIND == 0)
      asm volatile(MXQ_CHAINS("v_add_f32", "1.0, ") : "+v"(r0), "+v"(r1), "+v"(r2), "+v"(r3), "+v"(r4), "+v"(r5), "+v"(r6), "+v"(r7));
    else if constexpr (KIND == 1)
      asm volatile(MXQ_CHAINS("v_mul_f32", "0.5, ") : "+v"(r0), "+v"(r1), "+v"(r2), "+v"(r3), "+v"(r4), "+v"(r5), "+v"(r6), "+v"(r7));
    else if constexpr (KIND == 2)
      asm volatile(MXQ_CHAINS("v_and_b32", "0x7fffffff, ") : "+v"(r0), "+v"(r1), "+v"(r2), "+v"(r3), "+v"(r4), "+v"(r5), "+v"(r6), "+v"(r7));
    else if constexpr (KIND == 3)
      asm volatile(MXQ_CHAINS("v_rndne_f32", "") : "+v"(r0), "+v"(r1), "+v"(r2), "+v"(r3), "+v"(r4), "+v"(r5), "+v"(r6), "+v"(r7));
    else if constexpr (KIND == 4)
      asm volatile(MXQ_REP8("v_bfe_u32 %0, %0, 19, 1\n v_bfe_u32 %1, %1, 19, 1\n v_bfe_u32 %2, %2, 19, 1\n "
                            "v_bfe_u32 %3, %3, 19, 1\n v_bfe_u32 %4, %4, 19, 1\n v_bfe_u32 %5, %5, 19, 1\n "
                            "v_bfe_u32 %6, %6, 19, 1\n v_bfe_u32 %7, %7, 19, 1\n")
                   : "+v"(r0), "+v"(r1), "+v"(r2), "+v"(r3), "+v"(r4), "+v"(r5), "+v"(r6), "+v"(r7));
    else if constexpr (KIND == 5)
      asm volatile(MXQ_REP8("v_add3_u32 %0, %0, 1, %1\n v_add3_u32 %1, %1, 1, %2\n v_add3_u32 %2, %2, 1, %3\n "
                            "v_add3_u32 %3, %3, 1, %4\n v_add3_u32 %4, %4, 1, %5\n v_add3_u32 %5, %5, 1, %6\n "
                            "v_add3_u32 %6, %6, 1, %7\n v_add3_u32 %7, %7, 1, %0\n")
                   : "+v"(r0), "+v"(r1), "+v"(r2), "+v"(r3), "+v"(r4), "+v"(r5), "+v"(r6), "+v"(r7));
    else if constexpr (KIND == 6)
      asm volatile(MXQ_CHAINS("v_pk_mul_f16", "%0, ") : "+v"(r0), "+v"(r1), "+v"(r2), "+v"(r3), "+v"(r4), "+v"(r5), "+v"(r6), "+v"(r7));
    else if constexpr (KIND == 7)
      asm volatile(MXQ_CHAINS("v_pk_add_f16", "%0, ") : "+v"(r0), "+v"(r1), "+v"(r2), "+v"(r3), "+v"(r4), "+v"(r5), "+v"(r6), "+v"(r7));
    else if constexpr (KIND == 8)
      asm volatile(MXQ_REP8("v_fma_mix_f32 %0, %0, %0, %0 op_sel_hi:[1,0,0]\n v_fma_mix_f32 %1, %1, %1, %1 op_sel_hi:[1,0,0]\n "
                            "v_fma_mix_f32 %2, %2, %2, %2 op_sel_hi:[1,0,0]\n v_fma_mix_f32 %3, %3, %3, %3 op_sel_hi:[1,0,0]\n "
                            "v_fma_mix_f32 %4, %4, %4, %4 op_sel_hi:[1,0,0]\n v_fma_mix_f32 %5, %5, %5, %5 op_sel_hi:[1,0,0]\n "
                            "v_fma_mix_f32 %6, %6, %6, %6 op_sel_hi:[1,0,0]\n v_fma_mix_f32 %7, %7, %7, %7 op_sel_hi:[1,0,0]\n")
                   : "+v"(r0), "+v"(r1), "+v"(r2), "+v"(r3), "+v"(r4), "+v"(r5), "+v"(r6), "+v"(r7));
    else if constexpr (KIND == 9)
      asm volatile(MXQ_CHAINS("v_cvt_pkrtz_f16_f32", "%0, ") : "+v"(r0), "+v"(r1), "+v"(r2), "+v"(r3), "+v"(r4), "+v"(r5), "+v"(r6), "+v"(r7));
    else if constexpr (KIND == 10)
      asm volatile(MXQ_CHAINS("v_cvt_pk_bf16_f32", "0, ") : "+v"(r0), "+v"(r1), "+v"(r2), "+v"(r3), "+v"(r4), "+v"(r5), "+v"(r6), "+v"(r7));
    else if constexpr (KIND == 11)      // one dependent chain: issue-to-issue latency of v_mul_f32
      asm volatile(MXQ_REP8("v_mul_f32 %0, 0.5, %0\n v_mul_f32 %0, 0.5, %0\n v_mul_f32 %0, 0.5, %0\n v_mul_f32 %0, 0.5, %0\n "
                            "v_mul_f32 %0, 0.5, %0\n v_mul_f32 %0, 0.5, %0\n v_mul_f32 %0, 0.5, %0\n v_mul_f32 %0, 0.5, %0\n")
                   : "+v"(r0));
    else                                // one dependent chain of v_pk_mul_f16
      asm volatile(MXQ_REP8("v_pk_mul_f16 %0, %0, %0\n v_pk_mul_f16 %0, %0, %0\n v_pk_mul_f16 %0, %0, %0\n v_pk_mul_f16 %0, %0, %0\n "
                            "v_pk_mul_f16 %0, %0, %0\n v_pk_mul_f16 %0, %0, %0\n v_pk_mul_f16 %0, %0, %0\n v_pk_mul_f16 %0, %0, %0\n")
                   : "+v"(r0));
  }
  out[(int64_t)blockIdx.x * 256 + threadIdx.x] = r0 + r1 + r2 + r3 + r4 + r5 + r6 + r7;
}

#undef MXQ_CHAINS
#undef MXQ_REP8

}  // namespace

extern "C" int mxq_valu_probe(int32_t kind, int32_t iters, int64_t workgroups, float* out, mxq_stream_t stream) {
  if (kind < 0 || kind > 12) return mxq::invalid("mxq_valu_probe: kind must be 0..12");
  if (iters < 1 || workgroups < 1 || workgroups > (int64_t(1) << 20))
    return mxq::invalid("mxq_valu_probe: needs iters >= 1 and 1 <= workgroups <= 2^20");
  if (!out) return mxq::invalid("mxq_valu_probe: out is NULL");
  const dim3 grid((unsigned)workgroups);
  hipStream_t st = mxq::as_stream(stream);
  switch (kind) {
    case 0: k_valu_probe<0><<<grid, 256, 0, st>>>(iters, out); break;
    case 1: k_valu_probe<1><<<grid, 256, 0, st>>>(iters, out); break;
    case 2: k_valu_probe<2><<<grid, 256, 0, st>>>(iters, out); break;
    case 3: k_valu_probe<3><<<grid, 256, 0, st>>>(iters, out); break;
    case 4: k_valu_probe<4><<<grid, 256, 0, st>>>(iters, out); break;
    case 5: k_valu_probe<5><<<grid, 256, 0, st>>>(iters, out); break;
    case 6: k_valu_probe<6><<<grid, 256, 0, st>>>(iters, out); break;
    case 7: k_valu_probe<7><<<grid, 256, 0, st>>>(iters, out); break;
    case 8: k_valu_probe<8><<<grid, 256, 0, st>>>(iters, out); break;
    case 9: k_valu_probe<9><<<grid, 256, 0, st>>>(iters, out); break;
    case 10: k_valu_probe<10><<<grid, 256, 0, st>>>(iters, out); break;
    case 11: k_valu_probe<11><<<grid, 256, 0, st>>>(iters, out); break;
    default: k_valu_probe<12><<<grid, 256, 0, st>>>(iters, out); break;
  }
  return mxq::check_launch("mxq_valu_probe");
}
