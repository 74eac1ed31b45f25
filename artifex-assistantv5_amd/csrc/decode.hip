// Type dispatch of the decode kernels (decode_impl.hpp, one translation unit
// per ggml type: decode_<type>.hip).
#include "decode_types.hpp"

namespace gguf {

// One f32 activation row with a fused prologue / epilogue (decode_m1_kernel).
// hipErrorNotSupported: no fused kernel for this shape.
hipError_t launch_decode_fused(const float *x, const uint8_t *tiles, int type, int64_t n,
                               int64_t k, float *y, int prologue, const float *pw, float eps,
                               int epi, hipStream_t s) {
  switch (type) {
    case 2: return decode_fused_q4_0(x, tiles, (int)n, (int)k, y, prologue, pw, eps, epi, s);
    case 6: return decode_fused_q5_0(x, tiles, (int)n, (int)k, y, prologue, pw, eps, epi, s);
    case 8: return decode_fused_q8_0(x, tiles, (int)n, (int)k, y, prologue, pw, eps, epi, s);
    case 10: return decode_fused_q2_k(x, tiles, (int)n, (int)k, y, prologue, pw, eps, epi, s);
    case 11: return decode_fused_q3_k(x, tiles, (int)n, (int)k, y, prologue, pw, eps, epi, s);
    case 12: return decode_fused_q4_k(x, tiles, (int)n, (int)k, y, prologue, pw, eps, epi, s);
    case 13: return decode_fused_q5_k(x, tiles, (int)n, (int)k, y, prologue, pw, eps, epi, s);
    case 14: return decode_fused_q6_k(x, tiles, (int)n, (int)k, y, prologue, pw, eps, epi, s);
    case 20: return decode_fused_iq4_nl(x, tiles, (int)n, (int)k, y, prologue, pw, eps, epi, s);
    case 23: return decode_fused_iq4_xs(x, tiles, (int)n, (int)k, y, prologue, pw, eps, epi, s);
    case 16: return decode_fused_iq2_xxs(x, tiles, (int)n, (int)k, y, prologue, pw, eps, epi, s);
    case 17: return decode_fused_iq2_xs(x, tiles, (int)n, (int)k, y, prologue, pw, eps, epi, s);
    case 22: return decode_fused_iq2_s(x, tiles, (int)n, (int)k, y, prologue, pw, eps, epi, s);
    case 18: return decode_fused_iq3_xxs(x, tiles, (int)n, (int)k, y, prologue, pw, eps, epi, s);
    case 21: return decode_fused_iq3_s(x, tiles, (int)n, (int)k, y, prologue, pw, eps, epi, s);
    case 29: return decode_fused_iq1_m(x, tiles, (int)n, (int)k, y, prologue, pw, eps, epi, s);
    default: return hipErrorNotSupported;
  }
}

// The attention output projection with the record merge as its prologue
// (decode_m1_kernel, PRO 3): K = nh * hd.
hipError_t launch_decode_attn_merge(const AttnRecords &ar, const uint8_t *tiles, int type,
                                    int64_t n, float *y, int epi, hipStream_t s) {
  switch (type) {
    case 2: return decode_merge_q4_0(ar, tiles, (int)n, y, epi, s);
    case 6: return decode_merge_q5_0(ar, tiles, (int)n, y, epi, s);
    case 8: return decode_merge_q8_0(ar, tiles, (int)n, y, epi, s);
    case 10: return decode_merge_q2_k(ar, tiles, (int)n, y, epi, s);
    case 11: return decode_merge_q3_k(ar, tiles, (int)n, y, epi, s);
    case 12: return decode_merge_q4_k(ar, tiles, (int)n, y, epi, s);
    case 13: return decode_merge_q5_k(ar, tiles, (int)n, y, epi, s);
    case 14: return decode_merge_q6_k(ar, tiles, (int)n, y, epi, s);
    case 20: return decode_merge_iq4_nl(ar, tiles, (int)n, y, epi, s);
    case 23: return decode_merge_iq4_xs(ar, tiles, (int)n, y, epi, s);
    case 16: return decode_merge_iq2_xxs(ar, tiles, (int)n, y, epi, s);
    case 17: return decode_merge_iq2_xs(ar, tiles, (int)n, y, epi, s);
    case 22: return decode_merge_iq2_s(ar, tiles, (int)n, y, epi, s);
    case 18: return decode_merge_iq3_xxs(ar, tiles, (int)n, y, epi, s);
    case 21: return decode_merge_iq3_s(ar, tiles, (int)n, y, epi, s);
    case 29: return decode_merge_iq1_m(ar, tiles, (int)n, y, epi, s);
    default: return hipErrorNotSupported;
  }
}

// Workspace floats of one pass of mc <= 32 rows.
static int64_t pass_work(int type, int x_type, int n, int k, int mc) {
  switch (type) {
    case 2: return decode_work_q4_0(x_type, n, k, mc);
    case 6: return decode_work_q5_0(x_type, n, k, mc);
    case 8: return decode_work_q8_0(x_type, n, k, mc);
    case 10: return decode_work_q2_k(x_type, n, k, mc);
    case 11: return decode_work_q3_k(x_type, n, k, mc);
    case 12: return decode_work_q4_k(x_type, n, k, mc);
    case 13: return decode_work_q5_k(x_type, n, k, mc);
    case 14: return decode_work_q6_k(x_type, n, k, mc);
    case 20: return decode_work_iq4_nl(x_type, n, k, mc);
    case 23: return decode_work_iq4_xs(x_type, n, k, mc);
    case 16: return decode_work_iq2_xxs(x_type, n, k, mc);
    case 17: return decode_work_iq2_xs(x_type, n, k, mc);
    case 22: return decode_work_iq2_s(x_type, n, k, mc);
    case 18: return decode_work_iq3_xxs(x_type, n, k, mc);
    case 21: return decode_work_iq3_s(x_type, n, k, mc);
    case 29: return decode_work_iq1_m(x_type, n, k, mc);
    default: return 0;
  }
}

int64_t launch_decode_work(int type, int x_type, int64_t n, int64_t k, int64_t m) {
  int64_t w = 0;
  if (m >= 32) w = pass_work(type, x_type, (int)n, (int)k, 32);
  if (m % 32) {
    const int64_t v = pass_work(type, x_type, (int)n, (int)k, (int)(m % 32));
    w = v > w ? v : w;
  }
  return w;
}

// Rows are processed in groups of at most 32 (one pass over the weights each).
hipError_t launch_decode(const void *x, int x_type, int64_t ldx, const uint8_t *tiles, int type,
                         int64_t n, int64_t k, float *y, int64_t ldy, int64_t m, float *work,
                         int64_t work_floats, hipStream_t s) {
  const int esize = x_type == 0 ? 4 : 2;
  hipError_t e = hipSuccess;
  for (int64_t m0 = 0; m0 < m && e == hipSuccess; m0 += 32) {
    const int mc = (int)((m - m0) < 32 ? (m - m0) : 32);
    const char *xb = (const char *)x + m0 * ldx * esize;
    float *yb = y + m0 * ldy;
    switch (type) {
      case 2: e = decode_q4_0(xb, x_type, ldx, tiles, (int)n, (int)k, yb, ldy, mc, work, work_floats, s); break;
      case 6: e = decode_q5_0(xb, x_type, ldx, tiles, (int)n, (int)k, yb, ldy, mc, work, work_floats, s); break;
      case 8: e = decode_q8_0(xb, x_type, ldx, tiles, (int)n, (int)k, yb, ldy, mc, work, work_floats, s); break;
      case 10: e = decode_q2_k(xb, x_type, ldx, tiles, (int)n, (int)k, yb, ldy, mc, work, work_floats, s); break;
      case 11: e = decode_q3_k(xb, x_type, ldx, tiles, (int)n, (int)k, yb, ldy, mc, work, work_floats, s); break;
      case 12: e = decode_q4_k(xb, x_type, ldx, tiles, (int)n, (int)k, yb, ldy, mc, work, work_floats, s); break;
      case 13: e = decode_q5_k(xb, x_type, ldx, tiles, (int)n, (int)k, yb, ldy, mc, work, work_floats, s); break;
      case 14: e = decode_q6_k(xb, x_type, ldx, tiles, (int)n, (int)k, yb, ldy, mc, work, work_floats, s); break;
      case 20: e = decode_iq4_nl(xb, x_type, ldx, tiles, (int)n, (int)k, yb, ldy, mc, work, work_floats, s); break;
      case 23: e = decode_iq4_xs(xb, x_type, ldx, tiles, (int)n, (int)k, yb, ldy, mc, work, work_floats, s); break;
      case 16: e = decode_iq2_xxs(xb, x_type, ldx, tiles, (int)n, (int)k, yb, ldy, mc, work, work_floats, s); break;
      case 17: e = decode_iq2_xs(xb, x_type, ldx, tiles, (int)n, (int)k, yb, ldy, mc, work, work_floats, s); break;
      case 22: e = decode_iq2_s(xb, x_type, ldx, tiles, (int)n, (int)k, yb, ldy, mc, work, work_floats, s); break;
      case 18: e = decode_iq3_xxs(xb, x_type, ldx, tiles, (int)n, (int)k, yb, ldy, mc, work, work_floats, s); break;
      case 21: e = decode_iq3_s(xb, x_type, ldx, tiles, (int)n, (int)k, yb, ldy, mc, work, work_floats, s); break;
      case 29: e = decode_iq1_m(xb, x_type, ldx, tiles, (int)n, (int)k, yb, ldy, mc, work, work_floats, s); break;
      default: e = hipErrorNotSupported;
    }
  }
  return e;
}

}  // namespace gguf
