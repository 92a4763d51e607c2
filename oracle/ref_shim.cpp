// C-linkage shim over the reference's own scalar kernels, so that the oracle
// can be checked against them from Python (ctypes). Built only by
// oracle/Makefile into oracle/_ref/ from the sources where they lie in the
// reference tree; nothing is copied. TEST INFRASTRUCTURE ONLY.
#include <cstdint>
#include <stdexcept>

#include "linear8/linear8.h"
#include "linear32/linear32.h"
#include "layernorm/layernorm.h"
#include "gelu/gelu.h"
#include "residual15/residual15.h"
#include "add_requant15/add_requant15.h"
#include "conv1d/conv1d.h"
#include "classifier/classifier.h"
#include "attention/attention.h"

extern "C" {

void ref_linear8(const int8_t *x, const int8_t *w, const int32_t *bias, const int8_t *wz,
                 const uint32_t *m, const int8_t *s, int8_t *out, int64_t M, int64_t K,
                 int64_t N, int has_bias, int asym) {
  iwhisper::linear8_scalar(x, w, bias, wz, m, s, out, M, K, N, has_bias, asym);
}

void ref_linear8_accum(const int8_t *x, const int8_t *w, const int32_t *bias,
                       const int8_t *wz, int32_t *out, int64_t M, int64_t K, int64_t N,
                       int has_bias, int asym) {
  iwhisper::linear8_accum_scalar(x, w, bias, wz, out, M, K, N, has_bias, asym);
}

void ref_linear32(const int8_t *x, const int8_t *w, const int32_t *bias, const int8_t *wz,
                  const uint32_t *m, const int8_t *s, int32_t *out, int64_t M, int64_t K,
                  int64_t N, int has_bias, int asym) {
  iwhisper::linear32_scalar(x, w, bias, wz, m, s, out, M, K, N, has_bias, asym);
}

int ref_layernorm32(const int16_t *x, const int8_t *g, const int32_t *b, uint8_t lnm,
                    int8_t lns, uint32_t om, int8_t os, uint32_t off, int8_t *out,
                    int64_t rows, int64_t hidden, int has_bias) {
  try {
    iwhisper::layernorm32_scalar(x, g, b, lnm, lns, om, os, off, out, rows, hidden, has_bias);
  } catch (const std::exception &) {
    return -1;
  }
  return 0;
}

void ref_rsqrt(const int32_t *x, int32_t *out, int64_t n, uint32_t off) {
  iwhisper::layernorm32_rsqrt_scalar(x, out, n, off);
}

void ref_gelu(const int8_t *x, const uint8_t *lut, const uint8_t *lim, const int8_t *lis,
              const uint8_t *lom, const int8_t *los, int8_t *out, int64_t numel,
              int64_t channels, int64_t lic, int64_t loc) {
  iwhisper::gelu_scalar(x, lut, lim, lis, lom, los, out, numel, channels, lic, loc);
}

void ref_residual15(const int32_t *br, const int16_t *res, uint16_t m, int16_t *out,
                    int64_t n) {
  iwhisper::residual15_scalar(br, res, m, out, n);
}

void ref_add_requant15(const int8_t *x, const int8_t *a, const uint16_t *m, const int8_t *s,
                       int16_t *out, int64_t B, int64_t T, int64_t C, int64_t mc,
                       int64_t sc) {
  iwhisper::add_requant15_scalar(x, a, m, s, out, B, T, C, mc, sc);
}

void ref_conv1d(const int8_t *x, const int8_t *w, const int32_t *bias, uint32_t m, int8_t s,
                int8_t *out, int64_t B, int64_t cin, int64_t tin, int64_t cout, int64_t ks,
                int64_t stride, int64_t pad, int has_bias) {
  iwhisper::conv1d_scalar(x, w, bias, m, s, out, B, cin, tin, cout, ks, stride, pad, has_bias);
}

void ref_classifier(const int8_t *x, const int8_t *w, uint32_t m, int8_t s, int8_t *out,
                    int64_t M, int64_t K, int64_t N) {
  iwhisper::classifier_scalar(x, w, m, s, out, M, K, N);
}

void ref_qk_requant_rowmax(const int8_t *q, const int8_t *k, const bool *mask, int16_t *qk,
                           int16_t *rmp1, int64_t B, int64_t H, int64_t tq, int64_t tk,
                           int64_t D, uint8_t m, int32_t s, int has_mask) {
  iwhisper::qk_requant_rowmax_scalar(q, k, mask, qk, rmp1, B, H, tq, tk, D, m, s, has_mask);
}

void ref_shift_exp(const int16_t *qk, const int16_t *rmp1, const bool *mask, uint8_t *p,
                   int32_t *rs, int64_t B, int64_t H, int64_t tq, int64_t tk, int32_t f,
                   int has_mask) {
  iwhisper::shift_exp_scalar(qk, rmp1, mask, p, rs, B, H, tq, tk, f, has_mask);
}

int ref_pv_norm_requant(const uint8_t *p, const int8_t *v, const int32_t *rs, uint8_t am,
                        int8_t as, uint32_t off, int8_t *out, int64_t B, int64_t H,
                        int64_t tq, int64_t tk, int64_t D) {
  try {
    iwhisper::pv_norm_requant_scalar(p, v, rs, am, as, off, out, B, H, tq, tk, D);
  } catch (const std::exception &) {
    return -1;
  }
  return 0;
}

}  // extern "C"
