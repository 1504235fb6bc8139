// block.lut in one call on gfx950 (mxq/block/lut.py:23-34): the fused quantize-and-count kernel
// (lut_operand_impl.h), k-means over the summed counts (lut.hip), and k_lut_pick_codes, which turns the code
// bytes into table entries through each group's code map.
//
// Workspace layout (each part 256-byte aligned): the K x n code bytes, the nsplit partial histograms, the
// ceil(n / 2^group) x 2^(e+m+1) code maps.
#include "lut_operand_impl.h"

namespace {

using mxq_lut::CodeGrid;

// The LDS word of (unit u, code c) in the pick's per-block code maps: unit u's ncodes words, the code's low
// bits XORed with the unit's first column / 4 (mod 32), so the 32 lanes of a row, which look up the same hot
// codes in different units, land in different banks.
__device__ __forceinline__ int map_key(int u, int group, int ncodes) {
  return u * ncodes + (((u << group) >> 2) & 31);
}

// P_lut (K x n float32) from the code bytes: each code's entry read from its group's code map in LDS.
// Block: cw columns by a stripe of rows_per_block rows; a lane takes 4 adjacent columns (a 4-byte load and a
// 16-byte store per row, so a row's cw / 4 lanes load and store contiguous runs), and the block's 256 / (cw / 4)
// row lanes take the stripe's rows in turn.  n % 16 == 0.
__global__ void __launch_bounds__(256) k_lut_pick_codes(const uint8_t* __restrict__ codes, int64_t K, int64_t n,
                                                        int group, const uint32_t* __restrict__ code_map, int ncodes,
                                                        int cw, int units, int64_t rows_per_block,
                                                        float* __restrict__ out) {
  extern __shared__ uint32_t map_s[];                // units x ncodes
  const int64_t c0 = (int64_t)blockIdx.x * cw;
  const int64_t g0 = c0 >> group;
  const int64_t ng = (n + (int64_t(1) << group) - 1) >> group;
  // the block's maps are the code_map words [g0 * ncodes, + units * ncodes): 16-byte loads, all of a thread's
  // issued before its LDS stores (a multiple of 64 words; groups past the last read as 0)
  {
    const int total = units * ncodes;
    const int64_t avail = (ng - g0) * ncodes;
    const uint4* src = reinterpret_cast<const uint4*>(code_map + g0 * ncodes);
    const int lg = __builtin_ctz((unsigned)ncodes);
    for (int base = 0; base < total; base += 256 * 16) {
      uint4 w[4];
#pragma unroll
      for (int f = 0; f < 4; ++f) {
        const int i = base + (f * 256 + (int)threadIdx.x) * 4;
        w[f] = (i < total && i < avail) ? src[i >> 2] : make_uint4(0, 0, 0, 0);
      }
#pragma unroll
      for (int f = 0; f < 4; ++f) {
        const int i = base + (f * 256 + (int)threadIdx.x) * 4;
        if (i >= total) continue;
        const int u = i >> lg, code = i & (ncodes - 1);
        const int key = map_key(u, group, ncodes);
        map_s[key ^ code] = w[f].x;
        map_s[key ^ (code + 1)] = w[f].y;
        map_s[key ^ (code + 2)] = w[f].z;
        map_s[key ^ (code + 3)] = w[f].w;
      }
    }
  }
  __syncthreads();
  const int lpr = cw / 4;
  const int c = threadIdx.x % lpr, rl = threadIdx.x / lpr, nrl = blockDim.x / lpr;
  const int64_t j = c0 + c * 4;
  if (j >= n) return;
  const uint32_t cmask = (uint32_t)ncodes - 1u;       // a code byte stays inside its unit's map
  int key[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) key[e] = map_key((c * 4 + e) >> group, group, ncodes);
  const int64_t k0 = (int64_t)blockIdx.y * rows_per_block;
  const int64_t kend = (k0 + rows_per_block < K) ? k0 + rows_per_block : K;
  const int64_t kfirst = k0 + rl;
  const int64_t rows = kfirst < kend ? (kend - kfirst + nrl - 1) / nrl : 0;
  const int64_t rstep = (int64_t)nrl * n;
  const int64_t at0 = kfirst * n + j;
  constexpr int U = 8;
  using Buf = uint32_t[U];
  auto load = [&](Buf& v, int64_t batch, int count) {
    const uint8_t* p = codes + at0 + batch * U * rstep;
#pragma unroll
    for (int t = 0; t < U; ++t) v[t] = t < count ? *reinterpret_cast<const uint32_t*>(p + t * rstep) : 0u;
  };
  auto use = [&](const Buf& v, int64_t batch, int count) {
#pragma unroll
    for (int t = 0; t < U; ++t) {
      if (t >= count) break;
      float val[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) val[e] = u2f(map_s[key[e] ^ (int)((v[t] >> (8 * e)) & cmask)]);
      const mxq_quant::f32x4 r = {val[0], val[1], val[2], val[3]};
      __builtin_nontemporal_store(r, reinterpret_cast<mxq_quant::f32x4*>(out + at0 + (batch * U + t) * rstep));
    }
  };
  mxq_lut::stream_rows<U, Buf>(rows, load, use);
}

}  // namespace

namespace {

struct Plan {
  int cw;                    // the quantize kernel's tile: 128 columns, or 32 when the histogram of 128
                             // would not fit 48 KiB of LDS
  int64_t ntiles, nsplit, blocks_per_split;
  int units;                 // histogram units per tile
  int shift;                 // a group owns 2^shift tiles' units when it is wider than a tile
  int64_t nunits, split_stride;
  int pick_cw, pick_units;   // the pick's columns per block and code maps per block (at most 32 KiB)
  int64_t ng, ncodes;
  int64_t off_partial, off_map, bytes;
};

int64_t align256(int64_t x) { return (x + 255) / 256 * 256; }

Plan plan_of(int64_t K, int64_t n, int group, int nv, int ncodes) {
  Plan p{};
  const auto units_of = [&](int cw) { return (cw >> group) > 0 ? (cw >> group) : 1; };
  p.cw = (int64_t)units_of(128) * nv * 4 <= 48 * 1024 ? 128 : 32;
  const int log2cw = p.cw == 128 ? 7 : 5;
  p.ntiles = mxq::ceil_div(n, p.cw);
  p.units = units_of(p.cw);
  p.shift = group > log2cw ? group - log2cw : 0;
  p.nunits = p.ntiles * p.units;
  p.split_stride = p.nunits * nv;
  // about one 16-wave workgroup per CU (256 on MI355X), each wave at least one row block
  const int64_t nb = mxq::ceil_div(K, 32);
  int64_t nsplit = mxq::ceil_div(256, p.ntiles);
  const int64_t most = nb / 16 > 1 ? nb / 16 : 1;
  if (nsplit > most) nsplit = most;
  if (nsplit > 65535) nsplit = 65535;
  p.blocks_per_split = mxq::ceil_div(nb, nsplit);
  p.nsplit = mxq::ceil_div(nb, p.blocks_per_split);
  p.pick_cw = 128;
  while (p.pick_cw > 16 && (int64_t)units_of(p.pick_cw) * ncodes * 4 > 32 * 1024) p.pick_cw >>= 1;
  p.pick_units = units_of(p.pick_cw);
  p.ng = (n + (int64_t(1) << group) - 1) >> group;
  p.ncodes = ncodes;
  p.off_partial = align256(K * n);
  p.off_map = p.off_partial + align256(p.nsplit * p.split_stride * 4);
  p.bytes = p.off_map + align256(p.ng * ncodes * 4);
  return p;
}

int check_args(int64_t K, int64_t n, int group, int fmt_e, int fmt_m, int nv, CodeGrid* cg, const char* who) {
  if (K < 0 || n < 0 || group < 0 || group > 30) return mxq::invalid(std::string(who) + ": bad shape or group");
  if (n % 16) return mxq::invalid(std::string(who) + ": n must be a multiple of 16");
  *cg = mxq_lut::code_grid_of(fmt_e, fmt_m, nv);
  if (!cg->ok) return mxq::invalid(std::string(who) + ": (e, m, nv) is not a LUT format's code grid");
  return MXQ_OK;
}

}  // namespace

extern "C" int mxq_block_lut_workspace(int64_t K, int64_t n, int32_t group, int32_t fmt_e, int32_t fmt_m, int32_t nv,
                                       int64_t* bytes) {
  CodeGrid cg;
  if (!bytes) return mxq::invalid("mxq_block_lut_workspace: bytes is NULL");
  if (int rc = check_args(K, n, group, fmt_e, fmt_m, nv, &cg, "mxq_block_lut_workspace")) return rc;
  *bytes = (K == 0 || n == 0) ? 0 : plan_of(K, n, group, nv, 2 << cg.sign_at).bytes;
  return MXQ_OK;
}

extern "C" int mxq_block_lut(const void* V, int32_t v_dtype, int64_t K, int64_t n, const mxq_block_spec* spec,
                             int32_t group, int32_t max_iters, const float* grid, int32_t nv, const float* safe,
                             int32_t ns, const int32_t* safe_order, float* P_lut, float* X, float* T, void* workspace,
                             int64_t workspace_bytes, int32_t* err, mxq_stream_t stream) {
  if (!spec) return mxq::invalid("mxq_block_lut: spec is NULL");
  if (int rc = mxq_quant::validate(*spec)) return rc;
  if (spec->scale_rule != MXQ_SCALE_MXQUANT || spec->elem != MXQ_ELEM_OCP || spec->via_e != 0 ||
      !mxq_ocp_hw::has_hw(spec->e, spec->m) || spec->max_norm != mxq_ocp_hw::fmt_max(spec->e, spec->m))
    return mxq::invalid("mxq_block_lut: the spec must be MX-Gemmini's (its scale, the OCP element grid at the format's own "
                         "max_norm, no via)");
  CodeGrid cg;
  if (int rc = check_args(K, n, group, spec->e, spec->m, nv, &cg, "mxq_block_lut")) return rc;
  if (max_iters < 0 || ns < 1 || ns > mxq_lut::kMaxGrid) return mxq::invalid("mxq_block_lut: bad max_iters or ns");
  if (K == 0) return mxq::invalid("mxq_block_lut: K must be positive (tables of no codes are lut.tables')");
  if (n == 0) return MXQ_OK;
  if (!V || !P_lut || !X || !T || !grid || !safe || !safe_order || !workspace || !err)
    return mxq::invalid("mxq_block_lut: NULL pointer");
  if ((reinterpret_cast<uintptr_t>(V) | reinterpret_cast<uintptr_t>(P_lut) | reinterpret_cast<uintptr_t>(X)) % 16)
    return mxq::invalid("mxq_block_lut: V, P_lut and X must be 16-byte aligned");
  const int ncodes = 2 << cg.sign_at;
  const Plan p = plan_of(K, n, group, nv, ncodes);
  if (reinterpret_cast<uintptr_t>(workspace) % 256 || workspace_bytes < p.bytes)
    return mxq::invalid("mxq_block_lut: the workspace must be 256-byte aligned and mxq_block_lut_workspace bytes long");
  hipStream_t st = mxq::as_stream(stream);
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  uint8_t* codes = ws;
  int* partial = reinterpret_cast<int*>(ws + p.off_partial);
  uint32_t* map = reinterpret_cast<uint32_t*>(ws + p.off_map);
  const mxq_quant::CodeConsts k = mxq_quant::code_consts(spec->e, spec->m);
  const mxq_quant::ByteSink sink{codes, nullptr, err, spec->e, spec->m, k, (k.maxbits >> k.nshift) - k.nsub};
  const mxq_lut::LutQuantArgs a{codes, X, partial, err, K, n, group, nv, p.units, cg, p.blocks_per_split,
                                p.split_stride, sink};
  {
    mxq::KernelTimer timer("lut_quant", st);
    int rc;
    switch (v_dtype) {
      case MXQ_DT_F32: rc = mxq_lut_quant_f32(V, a, *spec, p.cw, p.ntiles, p.nsplit, st); break;
      case MXQ_DT_BF16: rc = mxq_lut_quant_bf16(V, a, *spec, p.cw, p.ntiles, p.nsplit, st); break;
      case MXQ_DT_F16: rc = mxq_lut_quant_f16(V, a, *spec, p.cw, p.ntiles, p.nsplit, st); break;
      default: return mxq::invalid("mxq_block_lut: unsupported input dtype");
    }
    if (rc) return rc;
  }
  const mxq_lut::CountSource src{partial, (int)p.nsplit, p.split_stride, p.nunits, p.shift};
  const int64_t per_group = K * ((int64_t(1) << group) < n ? (int64_t(1) << group) : n);
  if (int rc = mxq_lut::launch_kmeans(src, p.ng, nv, grid, safe, ns, safe_order, max_iters, T, map, cg,
                                      mxq_lut::sums_exact(per_group, spec->e, spec->m), st))
    return rc;
  {
    mxq::KernelTimer timer("lut_pick_codes", st);
    const int64_t col_blocks = mxq::ceil_div(n, p.pick_cw);
    const int64_t rpb = mxq_lut::stripe_rows(K, col_blocks, 1024);
    const dim3 g((unsigned)col_blocks, (unsigned)mxq::ceil_div(K, rpb));
    const size_t lds = (size_t)p.pick_units * ncodes * sizeof(uint32_t);
    k_lut_pick_codes<<<g, 256, lds, st>>>(codes, K, n, group, map, ncodes, p.pick_cw, p.pick_units, rpb, P_lut);
  }
  return mxq::check_launch("mxq_block_lut pick");
}
