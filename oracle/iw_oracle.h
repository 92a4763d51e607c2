/*
 * CPU oracle for the I-Whisper integer encoder/decoder path.
 *
 * TEST INFRASTRUCTURE ONLY. The tests compare the HIP path against this
 * library; it is also timed as the CPU baseline in bench.py. The product
 * (i-whisper_amd/) never links, loads or calls it.
 *
 * Every function restates the reference's scalar kernel named in its comment
 * (paths relative to the reference repository root). All arithmetic that the
 * reference performs modulo 2^32 or 2^16 is done on unsigned types here so
 * that it is defined behaviour in C.
 */
#ifndef IW_ORACLE_H
#define IW_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* i_whisper/kernels/csrc/common/fixedpoint.h:35-102 */
int32_t iwo_mulh(int32_t x, uint32_t multiplier);
int32_t iwo_rshift(int32_t x, uint32_t shift);
int32_t iwo_requant(int32_t x, uint32_t multiplier, uint32_t shift);

/* linear8/linear8_scalar.cpp:87-128 (accumulator only) */
void iwo_linear_accum(const int8_t *x, const int8_t *w, const int32_t *bias,
                      const int8_t *wz, int32_t *out, int64_t M, int64_t K,
                      int64_t N, int has_bias, int asym, int nthreads);
/* linear8/linear8_scalar.cpp:30-85 */
void iwo_linear8(const int8_t *x, const int8_t *w, const int32_t *bias,
                 const int8_t *wz, const uint32_t *mult, const int8_t *shift,
                 int8_t *out, int64_t M, int64_t K, int64_t N, int has_bias,
                 int asym, int nthreads);
/* linear32/linear32_scalar.cpp:9-129 */
void iwo_linear32(const int8_t *x, const int8_t *w, const int32_t *bias,
                  const int8_t *wz, const uint32_t *mult, const int8_t *shift,
                  int32_t *out, int64_t M, int64_t K, int64_t N, int has_bias,
                  int asym, int nthreads);

/* layernorm/layernorm_scalar.cpp:383-454 */
int32_t iwo_fisr(int32_t x, uint32_t offset);
void iwo_rsqrt(const int32_t *x, int32_t *out, int64_t n, uint32_t offset);
/* layernorm/layernorm_scalar.cpp:133-214 */
int iwo_layernorm32_stats(const int16_t *x, int32_t *mean, int32_t *var,
                          int32_t *renorm_shift, int64_t rows, int64_t hidden);
/* layernorm/layernorm_scalar.cpp:464-624 ; returns -1 for unsupported width */
int iwo_layernorm32(const int16_t *x, const int8_t *gamma, const int32_t *beta,
                    uint8_t ln_mult, int8_t ln_shift, uint32_t out_mult,
                    int8_t out_shift, uint32_t rsqrt_offset, int8_t *out,
                    int64_t rows, int64_t hidden, int has_bias);

/* gelu/gelu_scalar.cpp:10-181 */
void iwo_gelu(const int8_t *x, const uint8_t *lut, const uint8_t *luti_mult,
              const int8_t *luti_shift, const uint8_t *luto_mult,
              const int8_t *luto_shift, int8_t *out, int64_t numel,
              int64_t channels, int64_t luti_count, int64_t luto_count);

/* residual15/residual15_scalar.cpp:9-28 */
void iwo_residual15(const int32_t *branch, const int16_t *residual,
                    uint16_t mult, int16_t *out, int64_t numel);

/* add_requant15/add_requant15_scalar.cpp:29-81 */
void iwo_add_requant15(const int8_t *x, const int8_t *addend,
                       const uint16_t *mult, const int8_t *shift, int16_t *out,
                       int64_t batch, int64_t positions, int64_t channels,
                       int64_t mult_count, int64_t shift_count);

/* conv1d/conv1d_scalar.cpp:186-288 */
void iwo_conv1d(const int8_t *x, const int8_t *w, const int32_t *bias,
                uint32_t mult, int8_t shift, int8_t *out, int64_t batch,
                int64_t cin, int64_t tin, int64_t cout, int64_t ksize,
                int64_t stride, int64_t padding, int has_bias, int nthreads);

/* classifier/classifier_scalar.cpp:91-142 */
void iwo_classifier(const int8_t *x, const int8_t *w, uint32_t mult,
                    int8_t shift, int8_t *out, int64_t M, int64_t K, int64_t N,
                    int nthreads);

/* attention/attention_scalar.cpp:216-334 */
void iwo_qk_requant_rowmax(const int8_t *q, const int8_t *k,
                           const uint8_t *mask, int16_t *qk, int16_t *rmp1,
                           int64_t batch, int64_t heads, int64_t tq, int64_t tk,
                           int64_t dim, uint8_t mult, int32_t shift,
                           int has_mask, int nthreads);
/* attention/attention_scalar.cpp:388-568, one lane: x_sub -> uint8 */
uint8_t iwo_shift_exp_one(int16_t x_sub, int32_t frac_bits);
void iwo_shift_exp(const int16_t *qk, const int16_t *rmp1, const uint8_t *mask,
                   uint8_t *p, int32_t *row_sum, int64_t batch, int64_t heads,
                   int64_t tq, int64_t tk, int32_t frac_bits, int has_mask,
                   int nthreads);
/* attention/attention_scalar.cpp:676-814 ; returns -1 on a negative row sum */
int iwo_pv_norm_requant(const uint8_t *p, const int8_t *v,
                        const int32_t *row_sum, uint8_t av_mult, int8_t av_shift,
                        uint32_t rsqrt_offset, int8_t *out, int64_t batch,
                        int64_t heads, int64_t tq, int64_t tk, int64_t dim,
                        int nthreads);

#ifdef __cplusplus
}
#endif
#endif
