/*
 * SIMD-shaped CPU restatement of the reference's integer kernels, timed as
 * the CPU baseline.
 *
 * TEST INFRASTRUCTURE ONLY: bench.py's cpu_baseline leg (and the tests that
 * check it against the scalar oracle) load it; the product library in
 * i-whisper_amd/ never links or calls it.
 *
 * The reference's CPU backend ("simd") runs its GEMM-shaped kernels as int8
 * dot-product tiles split over rows with at::parallel_for, and its
 * row/element kernels single-threaded (paths relative to the reference
 * repository root):
 *   linear8/linear8_simd.cpp:326-669, linear32/linear32_simd.cpp:247-560:
 *     4 x 4 tiles (4 rows of x, 4 output channels) for M >= 32, 2 x 4 tiles
 *     for M >= 16, one row x 4 channels otherwise, rows split over threads;
 *   classifier/classifier_simd.cpp:347-369: 1 x 4 tiles, one thread;
 *   attention/attention_simd.cpp:1317, 2438: q.k and p.v dot tiles split
 *     over (batch, head);
 *   conv1d/conv1d_simd.cpp:670-760: output channels in groups of 4.
 * On ARM the dot products are NEON vdotq_s32. Here they are AVX-512 VNNI
 * (vpdpbusd: unsigned x signed bytes summed in groups of four into int32)
 * where the CPU has it, else AVX2 (bytes widened to int16, vpmaddwd). A
 * signed A operand enters vpdpbusd as a + 128 (a byte xor 0x80) and the
 * product is corrected by -128 * sum(b); every sum is taken modulo 2^32, as
 * the reference's int32 accumulators wrap, so the results are bit-identical
 * to the scalar kernels (the scalar oracle, iw_oracle.c). The epilogues are
 * the oracle's, element by element.
 */
#include "iw_oracle.h"

#include <immintrin.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

static inline int nthr(int n) { return n > 0 ? n : 1; }
static inline int32_t clampi(int32_t v, int32_t lo, int32_t hi) {
  return v < lo ? lo : (v > hi ? hi : v);
}

/* ------------------------------------------------------------------------
 * dot tiles: acc[i * 4 + j] = sum_k a_i[k] * b_j[k] (mod 2^32) for RM rows
 * a_i (stride lda) and NB <= 4 rows b_j (stride ldb); A bytes signed or, with
 * a_unsigned, unsigned (the attention probabilities); B bytes signed.
 * ---------------------------------------------------------------------- */

static int g_isa = -1; /* 1: AVX-512 VNNI, 0: AVX2 */

static int isa(void) {
  if (g_isa < 0) {
    __builtin_cpu_init();
    g_isa = __builtin_cpu_supports("avx512vnni") && __builtin_cpu_supports("avx512bw") ? 1 : 0;
  }
  return g_isa;
}

__attribute__((target("avx512f,avx512bw,avx512vnni"))) static void tile_vnni(
    const int8_t *a, int64_t lda, int rm, const int8_t *b, int64_t ldb, int nb, int64_t K, int a_unsigned,
    uint32_t *acc) {
  __m512i c[4][4], bs[4];
  const __m512i flip = _mm512_set1_epi8((char)0x80), ones = _mm512_set1_epi8(1);
  for (int i = 0; i < 4; ++i) {
    bs[i] = _mm512_setzero_si512();
    for (int j = 0; j < 4; ++j) c[i][j] = _mm512_setzero_si512();
  }
  for (int64_t k = 0; k < K; k += 64) {
    const __mmask64 mk = K - k >= 64 ? ~(__mmask64)0 : (((__mmask64)1 << (K - k)) - 1);
    __m512i bv[4], av[4];
    for (int j = 0; j < nb; ++j) {
      bv[j] = _mm512_maskz_loadu_epi8(mk, b + j * ldb + k);
      if (!a_unsigned) bs[j] = _mm512_dpbusd_epi32(bs[j], ones, bv[j]);
    }
    for (int i = 0; i < rm; ++i) {
      av[i] = _mm512_maskz_loadu_epi8(mk, a + i * lda + k);
      /* a + 128 as an unsigned byte; re-masking keeps the bytes past K at 0 */
      if (!a_unsigned) av[i] = _mm512_maskz_mov_epi8(mk, _mm512_xor_si512(av[i], flip));
    }
    for (int i = 0; i < rm; ++i)
      for (int j = 0; j < nb; ++j) c[i][j] = _mm512_dpbusd_epi32(c[i][j], av[i], bv[j]);
  }
  for (int j = 0; j < nb; ++j) {
    const uint32_t corr = a_unsigned ? 0u : 128u * (uint32_t)_mm512_reduce_add_epi32(bs[j]);
    for (int i = 0; i < rm; ++i) acc[i * 4 + j] = (uint32_t)_mm512_reduce_add_epi32(c[i][j]) - corr;
  }
}

__attribute__((target("avx2"))) static inline uint32_t hsum8(__m256i v) {
  __m128i s = _mm_add_epi32(_mm256_castsi256_si128(v), _mm256_extracti128_si256(v, 1));
  s = _mm_add_epi32(s, _mm_shuffle_epi32(s, 0x4e));
  s = _mm_add_epi32(s, _mm_shuffle_epi32(s, 0xb1));
  return (uint32_t)_mm_cvtsi128_si32(s);
}

__attribute__((target("avx2"))) static void tile_avx2(const int8_t *a, int64_t lda, int rm, const int8_t *b,
                                                      int64_t ldb, int nb, int64_t K, int a_unsigned,
                                                      uint32_t *acc) {
  __m256i c[4][4];
  for (int i = 0; i < 4; ++i)
    for (int j = 0; j < 4; ++j) c[i][j] = _mm256_setzero_si256();
  int64_t k = 0;
  for (; k + 16 <= K; k += 16) {
    __m256i bv[4], av[4];
    for (int j = 0; j < nb; ++j)
      bv[j] = _mm256_cvtepi8_epi16(_mm_loadu_si128((const __m128i *)(b + j * ldb + k)));
    for (int i = 0; i < rm; ++i) {
      const __m128i x = _mm_loadu_si128((const __m128i *)(a + i * lda + k));
      av[i] = a_unsigned ? _mm256_cvtepu8_epi16(x) : _mm256_cvtepi8_epi16(x);
    }
    for (int i = 0; i < rm; ++i)
      for (int j = 0; j < nb; ++j) c[i][j] = _mm256_add_epi32(c[i][j], _mm256_madd_epi16(av[i], bv[j]));
  }
  for (int i = 0; i < rm; ++i)
    for (int j = 0; j < nb; ++j) {
      uint32_t s = hsum8(c[i][j]);
      for (int64_t kk = k; kk < K; ++kk) {
        const int32_t av = a_unsigned ? (int32_t)(uint8_t)a[i * lda + kk] : (int32_t)a[i * lda + kk];
        s += (uint32_t)(av * (int32_t)b[j * ldb + kk]);
      }
      acc[i * 4 + j] = s;
    }
}

static void tile(const int8_t *a, int64_t lda, int rm, const int8_t *b, int64_t ldb, int nb, int64_t K,
                 int a_unsigned, uint32_t *acc) {
  if (isa())
    tile_vnni(a, lda, rm, b, ldb, nb, K, a_unsigned, acc);
  else
    tile_avx2(a, lda, rm, b, ldb, nb, K, a_unsigned, acc);
}

/* Rows per tile as the reference picks them for a GEMM of M rows. */
static int tile_rows(int64_t M) { return M >= 32 ? 4 : (M >= 16 ? 2 : 1); }

/* acc[m * N + n] = sum_k a[m][k] * b[n][k] (mod 2^32) over all rows, the
 * row tiles split over nthreads threads (nthreads = 1: one thread). */
static void gemm_acc(const int8_t *a, int64_t lda, int64_t M, const int8_t *b, int64_t ldb, int64_t N, int64_t K,
                     int a_unsigned, uint32_t *acc, int nthreads) {
  const int rm = tile_rows(M);
  const int64_t tiles = (M + rm - 1) / rm;
#pragma omp parallel for schedule(static) num_threads(nthr(nthreads))
  for (int64_t t = 0; t < tiles; ++t) {
    const int64_t m0 = t * rm;
    const int r = (int)(M - m0 < rm ? M - m0 : rm);
    uint32_t c[16];
    for (int64_t n0 = 0; n0 < N; n0 += 4) {
      const int nb = (int)(N - n0 < 4 ? N - n0 : 4);
      tile(a + m0 * lda, lda, r, b + n0 * ldb, ldb, nb, K, a_unsigned, c);
      for (int i = 0; i < r; ++i)
        for (int j = 0; j < nb; ++j) acc[(m0 + i) * N + n0 + j] = c[i * 4 + j];
    }
  }
}

static uint32_t row_sum(const int8_t *a, int64_t K) {
  uint32_t s = 0;
  for (int64_t k = 0; k < K; ++k) s += (uint32_t)(int32_t)a[k];
  return s;
}

/* x.w + bias - wz * rowsum(x), modulo 2^32 (linear8_scalar.cpp:52-69) */
static uint32_t *linear_corrected(const int8_t *x, const int8_t *w, const int32_t *bias, const int8_t *wz,
                                  int64_t M, int64_t K, int64_t N, int has_bias, int asym, int nthreads) {
  uint32_t *acc = (uint32_t *)malloc(sizeof(uint32_t) * (size_t)(M * N > 0 ? M * N : 1));
  gemm_acc(x, K, M, w, K, N, K, 0, acc, nthreads);
  for (int64_t m = 0; m < M; ++m) {
    const uint32_t xs = asym ? row_sum(x + m * K, K) : 0u;
    for (int64_t n = 0; n < N; ++n) {
      uint32_t v = acc[m * N + n];
      if (asym) v -= (uint32_t)((int32_t)wz[n]) * xs;
      if (has_bias) v += (uint32_t)bias[n];
      acc[m * N + n] = v;
    }
  }
  return acc;
}

/* linear8_simd.cpp:307-669 (epilogue as linear8_scalar.cpp:71-80: a shift
 * outside [0, 31] gives 0) */
void iws_linear8(const int8_t *x, const int8_t *w, const int32_t *bias, const int8_t *wz, const uint32_t *mult,
                 const int8_t *shift, int8_t *out, int64_t M, int64_t K, int64_t N, int has_bias, int asym,
                 int nthreads) {
  uint32_t *acc = linear_corrected(x, w, bias, wz, M, K, N, has_bias, asym, nthreads);
  for (int64_t m = 0; m < M; ++m)
    for (int64_t n = 0; n < N; ++n)
      out[m * N + n] = (int8_t)clampi(iwo_requant((int32_t)acc[m * N + n], mult[n], (uint32_t)(int32_t)shift[n]),
                                      -127, 127);
  free(acc);
}

/* linear32_simd.cpp:247-560 (epilogue as linear32_scalar.cpp:65-94) */
void iws_linear32(const int8_t *x, const int8_t *w, const int32_t *bias, const int8_t *wz, const uint32_t *mult,
                  const int8_t *shift, int32_t *out, int64_t M, int64_t K, int64_t N, int has_bias, int asym,
                  int nthreads) {
  uint32_t *acc = linear_corrected(x, w, bias, wz, M, K, N, has_bias, asym, nthreads);
  for (int64_t m = 0; m < M; ++m)
    for (int64_t n = 0; n < N; ++n) {
      const int32_t h = iwo_mulh((int32_t)acc[m * N + n], mult[n]);
      const int32_t s = shift[n];
      out[m * N + n] = (s < 0 || s >= 32) ? 0 : (int32_t)((uint32_t)h << s);
    }
  free(acc);
}

/* classifier_simd.cpp:347-369: one thread */
void iws_classifier(const int8_t *x, const int8_t *w, uint32_t mult, int8_t shift, int8_t *out, int64_t M,
                    int64_t K, int64_t N, int nthreads) {
  (void)nthreads;
  const uint32_t rs = (uint32_t)((int32_t)shift < 0 ? 0 : (int32_t)shift);
  uint32_t c[16];
  for (int64_t m = 0; m < M; ++m)
    for (int64_t n0 = 0; n0 < N; n0 += 4) {
      const int nb = (int)(N - n0 < 4 ? N - n0 : 4);
      tile(x + m * K, K, 1, w + n0 * K, K, nb, K, 0, c);
      for (int j = 0; j < nb; ++j)
        out[m * N + n0 + j] = (int8_t)clampi(iwo_rshift(iwo_mulh((int32_t)c[j], mult), rs), -127, 127);
    }
}

/* conv1d_simd.cpp:670-760: the window of output position t (kernel index
 * fastest, zero padding) gathered into a row, then dot tiles against the
 * [Cout][Cin * ksize] weight; per-tensor requant as conv1d_scalar.cpp:42-109 */
void iws_conv1d(const int8_t *x, const int8_t *w, const int32_t *bias, uint32_t mult, int8_t shift, int8_t *out,
                int64_t batch, int64_t cin, int64_t tin, int64_t cout, int64_t ksize, int64_t stride,
                int64_t padding, int has_bias, int nthreads) {
  const int64_t tout = (tin + 2 * padding - ksize) / stride + 1;
  const int64_t kk = cin * ksize;
  const uint32_t rs = (uint32_t)((int32_t)shift < 0 ? 0 : (int32_t)shift);
  int8_t *col = (int8_t *)malloc((size_t)(tout * kk > 0 ? tout * kk : 1));
  uint32_t *acc = (uint32_t *)malloc(sizeof(uint32_t) * (size_t)(tout * cout > 0 ? tout * cout : 1));
  for (int64_t b = 0; b < batch; ++b) {
    const int8_t *xb = x + b * cin * tin;
#pragma omp parallel for schedule(static) num_threads(nthr(nthreads))
    for (int64_t t = 0; t < tout; ++t)
      for (int64_t ic = 0; ic < cin; ++ic)
        for (int64_t k = 0; k < ksize; ++k) {
          const int64_t p = t * stride - padding + k;
          col[t * kk + ic * ksize + k] = (p < 0 || p >= tin) ? 0 : xb[ic * tin + p];
        }
    gemm_acc(col, kk, tout, w, kk, cout, kk, 0, acc, nthreads);
    for (int64_t oc = 0; oc < cout; ++oc)
      for (int64_t t = 0; t < tout; ++t) {
        uint32_t v = acc[t * cout + oc];
        if (has_bias) v += (uint32_t)bias[oc];
        out[(b * cout + oc) * tout + t] = (int8_t)clampi(iwo_rshift(iwo_mulh((int32_t)v, mult), rs), -127, 127);
      }
  }
  free(col);
  free(acc);
}

/* attention_simd.cpp:1317 (qk_requant_rowmax_simd): q.k dot tiles per
 * (batch, head); requant, mask and row max as attention_scalar.cpp:216-334 */
void iws_qk_requant_rowmax(const int8_t *q, const int8_t *k, const uint8_t *mask, int16_t *qk, int16_t *rmp1,
                           int64_t batch, int64_t heads, int64_t tq, int64_t tk, int64_t dim, uint8_t mult,
                           int32_t shift, int has_mask, int nthreads) {
  const uint32_t rs = (uint32_t)(shift > 0 ? shift : 0);
#pragma omp parallel for schedule(dynamic, 1) num_threads(nthr(nthreads))
  for (int64_t bh = 0; bh < batch * heads; ++bh) {
    uint32_t *acc = (uint32_t *)malloc(sizeof(uint32_t) * (size_t)(tq * tk > 0 ? tq * tk : 1));
    gemm_acc(q + bh * tq * dim, dim, tq, k + bh * tk * dim, dim, tk, dim, 0, acc, 1);
    for (int64_t i = 0; i < tq; ++i) {
      int16_t *o = qk + (bh * tq + i) * tk;
      int16_t mx = -32768;
      for (int64_t j = 0; j < tk; ++j) {
        if (has_mask && mask[i * tk + j]) {
          o[j] = -32768;
          continue;
        }
        const int32_t v = iwo_rshift((int32_t)(acc[i * tk + j] * (uint32_t)mult), rs);
        const int16_t h = (int16_t)clampi(v, -32768, 32767);
        o[j] = h;
        if (h > mx) mx = h;
      }
      rmp1[bh * tq + i] = (int16_t)(uint16_t)((uint32_t)(uint16_t)mx + 1u);
    }
    free(acc);
  }
}

void iws_shift_exp(const int16_t *qk, const int16_t *rmp1, const uint8_t *mask, uint8_t *p, int32_t *row_sum,
                   int64_t batch, int64_t heads, int64_t tq, int64_t tk, int32_t frac_bits, int has_mask,
                   int nthreads) {
  iwo_shift_exp(qk, rmp1, mask, p, row_sum, batch, heads, tq, tk, frac_bits, has_mask, nthreads);
}

/* attention_simd.cpp:2438 (pv_norm_requant_simd): p.v dot tiles per
 * (batch, head) with the unsigned probabilities; normalisation and requant
 * as attention_scalar.cpp:676-814 */
int iws_pv_norm_requant(const uint8_t *p, const int8_t *v, const int32_t *row_sum, uint8_t av_mult,
                        int8_t av_shift, uint32_t rsqrt_offset, int8_t *out, int64_t batch, int64_t heads,
                        int64_t tq, int64_t tk, int64_t dim, int nthreads) {
  for (int64_t i = 0; i < batch * heads * tq; ++i)
    if (row_sum[i] < 0) return -1;
  const int32_t avs = av_shift;
  const uint32_t rs = (uint32_t)(avs < 0 ? 0 : (avs > 32 ? 32 : avs));
#pragma omp parallel for schedule(dynamic, 1) num_threads(nthr(nthreads))
  for (int64_t bh = 0; bh < batch * heads; ++bh) {
    const int64_t b = bh / heads, h = bh % heads;
    uint32_t *acc = (uint32_t *)malloc(sizeof(uint32_t) * (size_t)(tq * dim > 0 ? tq * dim : 1));
    gemm_acc((const int8_t *)(p + bh * tq * tk), tk, tq, v + bh * dim * tk, tk, dim, tk, 1, acc, 1);
    for (int64_t i = 0; i < tq; ++i) {
      const int32_t inv = iwo_fisr(row_sum[bh * tq + i], rsqrt_offset);
      for (int64_t d = 0; d < dim; ++d) {
        int32_t y = iwo_rshift((int32_t)(acc[i * dim + d] * (uint32_t)inv), rsqrt_offset);
        y = iwo_rshift((int32_t)((uint32_t)y * (uint32_t)inv), rsqrt_offset);
        y = iwo_rshift((int32_t)((uint32_t)y * (uint32_t)av_mult), rs);
        out[(b * tq + i) * heads * dim + h * dim + d] = (int8_t)clampi(y, -127, 127);
      }
    }
    free(acc);
  }
  return 0;
}

/* The row and element kernels run single-threaded in the reference's SIMD
 * backend (layernorm_simd.cpp:982, gelu_simd.cpp:309, residual15 and
 * add_requant15): the oracle's restatements, one thread. */
int iws_layernorm32(const int16_t *x, const int8_t *gamma, const int32_t *beta, uint8_t ln_mult, int8_t ln_shift,
                    uint32_t out_mult, int8_t out_shift, uint32_t rsqrt_offset, int8_t *out, int64_t rows,
                    int64_t hidden, int has_bias) {
  return iwo_layernorm32(x, gamma, beta, ln_mult, ln_shift, out_mult, out_shift, rsqrt_offset, out, rows, hidden,
                         has_bias);
}

void iws_gelu(const int8_t *x, const uint8_t *lut, const uint8_t *luti_mult, const int8_t *luti_shift,
              const uint8_t *luto_mult, const int8_t *luto_shift, int8_t *out, int64_t numel, int64_t channels,
              int64_t luti_count, int64_t luto_count) {
  iwo_gelu(x, lut, luti_mult, luti_shift, luto_mult, luto_shift, out, numel, channels, luti_count, luto_count);
}

void iws_residual15(const int32_t *branch, const int16_t *residual, uint16_t mult, int16_t *out, int64_t numel) {
  iwo_residual15(branch, residual, mult, out, numel);
}

void iws_add_requant15(const int8_t *x, const int8_t *addend, const uint16_t *mult, const int8_t *shift,
                       int16_t *out, int64_t batch, int64_t positions, int64_t channels, int64_t mult_count,
                       int64_t shift_count) {
  iwo_add_requant15(x, addend, mult, shift, out, batch, positions, channels, mult_count, shift_count);
}

/* 1: the dot tiles use AVX-512 VNNI, 0: AVX2 */
int iws_isa(void) { return isa(); }

/* Test hook: 0 forces the AVX2 tiles, 1 the VNNI tiles (where present), -1
 * returns to the run-time choice. */
void iws_force_isa(int which) { g_isa = which < 0 ? -1 : (which ? isa() : 0); }
