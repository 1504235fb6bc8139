// Host build of the kernels' numerics header (microscaling-quant_amd/csrc/mxq_numerics.h), for the CPU test
// suite: every device primitive is compiled here with g++ (-ffp-contract=off, IEEE float, denormals kept) and
// driven over numpy arrays, so its logic is checked against the oracle without a GPU.  Test infrastructure
// only; the product never loads this library.
#include "mxq_numerics.h"

extern "C" {

void h_round_bits(const int64_t* bits, int64_t* out, int64_t n, int keep, int mode) {
  for (int64_t i = 0; i < n; ++i) out[i] = (int64_t)round_bits32((uint32_t)bits[i], keep, mode);
}
void h_bf16(const float* x, float* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = bf16_rne(x[i]);
}
void h_floor_log2(const float* x, int32_t* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = floor_log2_pos(x[i]);
}
void h_float_em32(const float* z, float* out, int64_t n, int e, int m, int mode, int grid, float max_norm) {
  for (int64_t i = 0; i < n; ++i) out[i] = float_em_quantize32(z[i], e, m, mode, grid, max_norm);
}
void h_float_em64(const double* z, float* out, int64_t n, int e, int m, int mode, int grid, float max_norm) {
  for (int64_t i = 0; i < n; ++i) out[i] = float_em_quantize64(z[i], e, m, mode, grid, max_norm);
}
void h_ocp_grid_fast(const float* z, float* out, int64_t n, int e, int m, int mode, float max_norm) {
  for (int64_t i = 0; i < n; ++i) out[i] = ocp_grid_fast(z[i], e, m, mode, max_norm);
}
void h_microsoft(const float* z, float* out, int64_t n, int ebits, int mbits, float max_norm, int mode, int sat) {
  for (int64_t i = 0; i < n; ++i) out[i] = microsoft_quantize(z[i], ebits, mbits, max_norm, mode, sat != 0);
}
void h_scale(const float* a, float* out, int64_t n, const mxq_block_spec* s) {
  for (int64_t i = 0; i < n; ++i) out[i] = block_scale(a[i], *s);
}
void h_exact_add(const float* a, const float* b, float* out, int64_t n, int e, int m, int mode, int grid,
                 float max_norm) {
  for (int64_t i = 0; i < n; ++i) out[i] = exact_add(a[i], b[i], e, m, mode, grid, max_norm);
}
void h_truncate(const float* x, float* out, int64_t n, int m) {
  for (int64_t i = 0; i < n; ++i) out[i] = truncate_significand(x[i], m);
}
void h_flush(const float* x, float* out, int64_t n, float thr) {
  for (int64_t i = 0; i < n; ++i) out[i] = flush_product(x[i], thr);
}
void h_div_inv(const float* x, float* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = make_div(x[i]).inv;
}
void h_saturate(const float* x, float* out, int64_t n, float limit, float value) {
  for (int64_t i = 0; i < n; ++i) out[i] = saturate(x[i], limit, value);
}

// Block quantization of an (outer, n, inner) float32 tensor with the kernels' per-block step sequence.
void h_block_quantize(const float* V, float* P, float* X, int64_t outer, int64_t n, int64_t inner, int64_t bs,
                      const mxq_block_spec* sp) {
  const mxq_block_spec& s = *sp;
  const int64_t nb = (n + bs - 1) / bs;
  for (int64_t o = 0; o < outer; ++o)
    for (int64_t b = 0; b < nb; ++b)
      for (int64_t i = 0; i < inner; ++i) {
        const int64_t k0 = b * bs, rows = (n - k0 < bs) ? n - k0 : bs;
        float a = 0.0f;
        for (int64_t r = 0; r < rows; ++r) a = amax_combine(a, fabsf(V[(o * n + k0 + r) * inner + i]));
        const float x = block_scale(a, s);
        const Div d = make_div(x);
        for (int64_t r = 0; r < rows; ++r) {
          const int64_t idx = (o * n + k0 + r) * inner + i;
          const float v = V[idx];
          float q;
          const float z = s.scale_rule ? apply_div(v, d) : v;
          switch (s.elem) {
            case MXQ_ELEM_QTORCH: q = elem_q<MXQ_ELEM_QTORCH>(z, s); break;
            case MXQ_ELEM_IEEE: q = elem_q<MXQ_ELEM_IEEE>(z, s); break;
            case MXQ_ELEM_OCP: q = elem_q<MXQ_ELEM_OCP>(z, s); break;
            case MXQ_ELEM_MICROSOFT: q = elem_q<MXQ_ELEM_MICROSOFT>(z, s); break;
            default: q = z;
          }
          P[idx] = q;
        }
        X[(o * nb + b) * inner + i] = x;
      }
}

// Packed byte codes: codes[i] = mx_encode(q[i]) with ok[i] its flag; mx_decode; E8M0 both ways.
void h_mx_encode(const float* q, uint8_t* codes, uint8_t* ok, int64_t n, int e, int m) {
  for (int64_t i = 0; i < n; ++i) {
    bool good = true;
    codes[i] = (uint8_t)mx_encode(q[i], e, m, &good);
    ok[i] = good ? 1 : 0;
  }
}
void h_mx_decode(const uint8_t* codes, float* out, int64_t n, int e, int m) {
  for (int64_t i = 0; i < n; ++i) out[i] = mx_decode(codes[i], e, m);
}
void h_e8m0_encode(const float* x, const uint8_t* zero, uint8_t* b, uint8_t* ok, int64_t n) {
  for (int64_t i = 0; i < n; ++i) {
    bool good = true;
    b[i] = (uint8_t)e8m0_encode(x[i], zero[i] != 0, &good);
    ok[i] = good ? 1 : 0;
  }
}
void h_e8m0_decode(const uint8_t* b, float* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = e8m0_decode(b[i]);
}

}  // extern "C"
