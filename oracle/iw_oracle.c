/*
 * CPU oracle for the I-Whisper integer encoder/decoder path.
 *
 * TEST INFRASTRUCTURE ONLY: tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py compare the HIP results with it. The product
 * library in i-whisper_amd/ never links or calls it.
 *
 * Each function restates the scalar kernel cited above it (paths relative to
 * the reference repository root). Wrapping arithmetic is written on uint32_t /
 * uint16_t so that it is defined C. The GEMM-shaped loops take an OpenMP
 * thread count so the same code doubles as the multi-threaded CPU baseline;
 * the integer results do not depend on it.
 */
#include "iw_oracle.h"

#include <stdlib.h>

#ifdef _OPENMP
#include <omp.h>
#endif

static inline int32_t s32(uint32_t v) { return (int32_t)v; }
static inline int16_t s16(uint32_t v) { return (int16_t)(uint16_t)v; }
static inline int32_t clampi(int32_t v, int32_t lo, int32_t hi) {
  return v < lo ? lo : (v > hi ? hi : v);
}
static inline int nthr(int n) { return n > 0 ? n : 1; }

/* ---------------- fixed point: common/fixedpoint.h:35-102 ---------------- */

int32_t iwo_mulh(int32_t x, uint32_t multiplier) {
  /* (int64)x * (uint32)m >> 32, arithmetic. |product| < 2^63. */
  int64_t p = (int64_t)x * (int64_t)multiplier;
  return (int32_t)(p >> 32);
}

int32_t iwo_rshift(int32_t x, uint32_t shift) {
  /* Round half away from zero: (x + 2^(s-1) - signbit(x)) >> s, with the add
   * wrapping modulo 2^32; s == 0 is the identity and s >= 32 gives 0. */
  if (shift == 0) return x;
  if (shift >= 32) return 0;
  uint32_t bias = (1u << (shift - 1)) - ((uint32_t)x >> 31);
  return s32((uint32_t)x + bias) >> shift;
}

int32_t iwo_requant(int32_t x, uint32_t multiplier, uint32_t shift) {
  return iwo_rshift(iwo_mulh(x, multiplier), shift);
}

/* ---------------- GEMM accumulators ---------------- */

/* Sum_k x[k]*w[k] modulo 2^32 (linear8_scalar.cpp:13-28). */
static inline uint32_t dot_s8(const int8_t *a, const int8_t *b, int64_t K) {
  int32_t acc = 0; /* |acc| < K * 2^14: wraps only for K > 2^17 */
  if (K <= (1 << 17)) {
    for (int64_t k = 0; k < K; ++k) acc += (int32_t)a[k] * (int32_t)b[k];
    return (uint32_t)acc;
  }
  uint32_t u = 0;
  for (int64_t k = 0; k < K; ++k) u += (uint32_t)((int32_t)a[k] * (int32_t)b[k]);
  return u;
}

static inline uint32_t row_sum_s8(const int8_t *a, int64_t K) {
  uint32_t s = 0;
  for (int64_t k = 0; k < K; ++k) s += (uint32_t)(int32_t)a[k];
  return s;
}

/* acc = x.w + bias - wz*rowsum(x), all modulo 2^32
 * (linear8_scalar.cpp:52-69, linear32_scalar.cpp:21-62). */
static inline uint32_t linear_acc(const int8_t *xr, const int8_t *wr, uint32_t xsum,
                                  const int32_t *bias, const int8_t *wz, int64_t n,
                                  int64_t K, int has_bias, int asym) {
  uint32_t acc = dot_s8(xr, wr, K);
  if (asym) acc -= (uint32_t)((int32_t)wz[n]) * xsum;
  if (has_bias) acc += (uint32_t)bias[n];
  return acc;
}

void iwo_linear_accum(const int8_t *x, const int8_t *w, const int32_t *bias,
                      const int8_t *wz, int32_t *out, int64_t M, int64_t K,
                      int64_t N, int has_bias, int asym, int nthreads) {
#pragma omp parallel for schedule(static) num_threads(nthr(nthreads))
  for (int64_t m = 0; m < M; ++m) {
    const int8_t *xr = x + m * K;
    uint32_t xsum = asym ? row_sum_s8(xr, K) : 0u;
    for (int64_t n = 0; n < N; ++n)
      out[m * N + n] = s32(linear_acc(xr, w + n * K, xsum, bias, wz, n, K, has_bias, asym));
  }
}

/* linear8/linear8_scalar.cpp:30-85: the shift is cast int8 -> uint32, so a
 * negative shift is >= 32 and the requant yields 0. */
void iwo_linear8(const int8_t *x, const int8_t *w, const int32_t *bias,
                 const int8_t *wz, const uint32_t *mult, const int8_t *shift,
                 int8_t *out, int64_t M, int64_t K, int64_t N, int has_bias,
                 int asym, int nthreads) {
#pragma omp parallel for schedule(static) num_threads(nthr(nthreads))
  for (int64_t m = 0; m < M; ++m) {
    const int8_t *xr = x + m * K;
    uint32_t xsum = asym ? row_sum_s8(xr, K) : 0u;
    for (int64_t n = 0; n < N; ++n) {
      int32_t acc = s32(linear_acc(xr, w + n * K, xsum, bias, wz, n, K, has_bias, asym));
      acc = iwo_requant(acc, mult[n], (uint32_t)(int32_t)shift[n]);
      out[m * N + n] = (int8_t)clampi(acc, -127, 127);
    }
  }
}

/* linear32/linear32_scalar.cpp:65-94: y = (int32)(mulh(acc, m) * 2^shift).
 * For shift in [0, 31] that is the low 32 bits of mulh << shift; for shift in
 * [32, 63] the low 32 bits are 0. Other shifts are undefined behaviour in the
 * reference C++ (and 0 in its torch golden, linear.py:185); this gives 0. */
static inline int32_t linear32_epilogue(int32_t acc, uint32_t m, int8_t shift) {
  int32_t h = iwo_mulh(acc, m);
  int32_t s = shift;
  if (s < 0 || s >= 32) return 0;
  return s32((uint32_t)h << s);
}

void iwo_linear32(const int8_t *x, const int8_t *w, const int32_t *bias,
                  const int8_t *wz, const uint32_t *mult, const int8_t *shift,
                  int32_t *out, int64_t M, int64_t K, int64_t N, int has_bias,
                  int asym, int nthreads) {
#pragma omp parallel for schedule(static) num_threads(nthr(nthreads))
  for (int64_t m = 0; m < M; ++m) {
    const int8_t *xr = x + m * K;
    uint32_t xsum = asym ? row_sum_s8(xr, K) : 0u;
    for (int64_t n = 0; n < N; ++n) {
      int32_t acc = s32(linear_acc(xr, w + n * K, xsum, bias, wz, n, K, has_bias, asym));
      out[m * N + n] = linear32_epilogue(acc, mult[n], shift[n]);
    }
  }
}

/* ---------------- LayerNorm32: layernorm/layernorm_scalar.cpp ---------------- */

/* Division by the width as adds and floor shifts (layernorm_scalar.cpp:14-56).
 * The adds are int32 in the reference; operands stay far from overflow for
 * int15 inputs, and are written modulo 2^32 here. */
static inline int width_code(int64_t h) {
  switch (h) {
    case 384: return 0;
    case 512: return 1;
    case 768: return 2;
    case 1024: return 3;
    case 1280: return 4;
    default: return -1;
  }
}

static inline int32_t norm_reduce(int32_t v, int code) {
  switch (code) {
    case 0: return s32((uint32_t)v + (uint32_t)(v >> 2) + (uint32_t)(v >> 3)) >> 9;
    case 1: return v >> 9;
    case 2: return s32((uint32_t)v + (uint32_t)(v >> 2) + (uint32_t)(v >> 3)) >> 10;
    case 3: return v >> 10;
    default: return s32((uint32_t)v + (uint32_t)(v >> 1)) >> 11;
  }
}

static inline int32_t bit_length(int32_t v) {
  /* bit length of a non-negative value; 0 for 0 */
  return v == 0 ? 0 : 32 - __builtin_clz((uint32_t)v);
}

/* int32 -> fp32 bit pattern with truncated mantissa (layernorm_scalar.cpp:309-343) */
static inline int32_t i2f_bits_trunc(int32_t x) {
  if (x == 0) return 0;
  int32_t e = bit_length(x) - 1;
  uint64_t sig = e <= 23 ? ((uint64_t)(uint32_t)x << (23 - e))
                         : ((uint64_t)(uint32_t)x >> (e - 23));
  uint32_t bits = ((uint32_t)(e + 127) << 23) | ((uint32_t)sig & 0x007FFFFFu);
  return s32(bits);
}

/* fp32 bit pattern -> int32, truncating; negative exponent gives 0
 * (layernorm_scalar.cpp:345-381) */
static inline int32_t f2i_bits_trunc(int32_t bits) {
  uint32_t raw = (uint32_t)bits;
  int32_t e = (int32_t)((raw >> 23) & 0xFFu) - 127;
  uint64_t sig = (uint64_t)((1u << 23) | (raw & 0x007FFFFFu));
  if (e < 0) return 0;
  uint64_t v = e >= 23 ? (sig << (e - 23)) : (sig >> (23 - e));
  return s32((uint32_t)v);
}

/* Integer fast inverse square root with two Newton steps
 * (layernorm_scalar.cpp:383-438). */
int32_t iwo_fisr(int32_t x, uint32_t offset) {
  int32_t i = i2f_bits_trunc(x);
  i = s32(0x5f3759dfu - (uint32_t)(i >> 1));
  int32_t y = f2i_bits_trunc(s32((uint32_t)i + (offset << 23)));
  uint32_t three = 3u << offset;
  for (int it = 0; it < 2; ++it) {
    int32_t xy = s32((uint32_t)x * (uint32_t)y);
    int32_t xs = iwo_rshift(xy, offset);
    uint32_t t = (uint32_t)xs * (uint32_t)y;
    uint32_t corr = three - t;
    int32_t prod = s32((uint32_t)y * corr);
    y = iwo_rshift(prod, offset + 1);
  }
  return y;
}

void iwo_rsqrt(const int32_t *x, int32_t *out, int64_t n, uint32_t offset) {
  for (int64_t i = 0; i < n; ++i) out[i] = iwo_fisr(x[i], offset);
}

typedef struct {
  int32_t mean, var, rshift;
} ln_stats;

static inline ln_stats ln_row_stats(const int16_t *r, int64_t h, int code) {
  ln_stats st;
  uint32_t sum = 0;
  for (int64_t c = 0; c < h; ++c) sum += (uint32_t)(int32_t)r[c];
  st.mean = norm_reduce(s32(sum), code);
  int32_t maxsq = 0;
  for (int64_t c = 0; c < h; ++c) {
    int32_t d = (int32_t)r[c] - st.mean;
    int32_t sq = s32((uint32_t)d * (uint32_t)d);
    if (sq > maxsq) maxsq = sq;
  }
  int32_t rs = bit_length(maxsq) - 16;
  if (rs < 0) rs = 0;
  rs = (rs + 1) & ~1;
  st.rshift = rs;
  uint32_t vs = 0;
  for (int64_t c = 0; c < h; ++c) {
    int32_t d = (int32_t)r[c] - st.mean;
    int32_t sq = s32((uint32_t)d * (uint32_t)d);
    vs += (uint32_t)iwo_rshift(sq, (uint32_t)rs);
  }
  st.var = norm_reduce(s32(vs), code);
  return st;
}

int iwo_layernorm32_stats(const int16_t *x, int32_t *mean, int32_t *var,
                          int32_t *renorm_shift, int64_t rows, int64_t hidden) {
  int code = width_code(hidden);
  if (code < 0) return -1;
  for (int64_t r = 0; r < rows; ++r) {
    ln_stats st = ln_row_stats(x + r * hidden, hidden, code);
    mean[r] = st.mean;
    var[r] = st.var;
    renorm_shift[r] = st.rshift;
  }
  return 0;
}

int iwo_layernorm32(const int16_t *x, const int8_t *gamma, const int32_t *beta,
                    uint8_t ln_mult, int8_t ln_shift, uint32_t out_mult,
                    int8_t out_shift, uint32_t rsqrt_offset, int8_t *out,
                    int64_t rows, int64_t hidden, int has_bias) {
  int code = width_code(hidden);
  if (code < 0) return -1;
  for (int64_t r = 0; r < rows; ++r) {
    const int16_t *xr = x + r * hidden;
    ln_stats st = ln_row_stats(xr, hidden, code);
    int32_t inv = iwo_fisr(st.var, rsqrt_offset);
    /* int8 + int: a negative sum converts to a shift >= 32 (result 0) */
    uint32_t nshift = (uint32_t)((int32_t)ln_shift + (st.rshift >> 1));
    uint32_t oshift = (uint32_t)(int32_t)out_shift;
    for (int64_t c = 0; c < hidden; ++c) {
      int32_t d = (int32_t)xr[c] - st.mean;
      uint32_t v = (uint32_t)d * (uint32_t)inv;
      v *= (uint32_t)ln_mult;
      int32_t t = clampi(iwo_rshift(s32(v), nshift), -16383, 16383);
      uint32_t a = (uint32_t)t * (uint32_t)(int32_t)gamma[c];
      if (has_bias) a += (uint32_t)beta[c];
      int32_t y = iwo_rshift(iwo_mulh(s32(a), out_mult), oshift);
      out[r * hidden + c] = (int8_t)clampi(y, -127, 127);
    }
  }
  return 0;
}

/* ---------------- GeLU: gelu/gelu_scalar.cpp:10-181 ---------------- */

static inline uint32_t clamp_shift(int8_t s) {
  int32_t v = s;
  return (uint32_t)(v < 0 ? 0 : (v > 32 ? 32 : v));
}

void iwo_gelu(const int8_t *x, const uint8_t *lut, const uint8_t *luti_mult,
              const int8_t *luti_shift, const uint8_t *luto_mult,
              const int8_t *luto_shift, int8_t *out, int64_t numel,
              int64_t channels, int64_t luti_count, int64_t luto_count) {
  for (int64_t i = 0; i < numel; ++i) {
    int64_t c = i % channels;
    int64_t a = luti_count == 1 ? 0 : c;
    int64_t b = luto_count == 1 ? 0 : c;
    int32_t xv = x[i];
    int32_t idx = iwo_rshift(xv * (int32_t)luti_mult[a], clamp_shift(luti_shift[a]));
    idx = clampi(idx + 8, 0, 15);
    int32_t v = xv * (int32_t)lut[idx]; /* |v| <= 128*255 */
    v = s32((uint32_t)v * (uint32_t)luto_mult[b]);
    v = iwo_rshift(v, clamp_shift(luto_shift[b]));
    out[i] = (int8_t)clampi(v, -127, 127);
  }
}

/* ---------------- residual15: residual15/residual15_scalar.cpp:9-28 ---------------- */

void iwo_residual15(const int32_t *branch, const int16_t *residual,
                    uint16_t mult, int16_t *out, int64_t numel) {
  for (int64_t i = 0; i < numel; ++i) {
    uint32_t v = (uint32_t)branch[i] + (uint32_t)((int32_t)residual[i] * (int32_t)mult);
    int32_t y = iwo_rshift(s32(v), 15);
    out[i] = (int16_t)clampi(y, -16383, 16383);
  }
}

/* ---------------- add_requant15: add_requant15/add_requant15_scalar.cpp:29-81 ---------------- */

void iwo_add_requant15(const int8_t *x, const int8_t *addend,
                       const uint16_t *mult, const int8_t *shift, int16_t *out,
                       int64_t batch, int64_t positions, int64_t channels,
                       int64_t mult_count, int64_t shift_count) {
  for (int64_t b = 0; b < batch; ++b)
    for (int64_t t = 0; t < positions; ++t)
      for (int64_t c = 0; c < channels; ++c) {
        int64_t i = (b * positions + t) * channels + c;
        int32_t v = (int32_t)x[i] + (int32_t)addend[t * channels + c];
        uint16_t m = mult[mult_count == 1 ? 0 : c];
        int32_t s = shift[shift_count == 1 ? 0 : c];
        int32_t p = s32((uint32_t)v * (uint32_t)m);
        int32_t y = iwo_rshift(p, (uint32_t)(s < 0 ? 0 : s));
        out[i] = (int16_t)clampi(y, -16383, 16383);
      }
}

/* ---------------- conv1d: conv1d/conv1d_scalar.cpp:42-109, 186-288 ---------------- */

void iwo_conv1d(const int8_t *x, const int8_t *w, const int32_t *bias,
                uint32_t mult, int8_t shift, int8_t *out, int64_t batch,
                int64_t cin, int64_t tin, int64_t cout, int64_t ksize,
                int64_t stride, int64_t padding, int has_bias, int nthreads) {
  int64_t tout = (tin + 2 * padding - ksize) / stride + 1;
  uint32_t rs = (uint32_t)((int32_t)shift < 0 ? 0 : (int32_t)shift);
#pragma omp parallel for collapse(2) schedule(static) num_threads(nthr(nthreads))
  for (int64_t b = 0; b < batch; ++b)
    for (int64_t oc = 0; oc < cout; ++oc) {
      const int8_t *xb = x + b * cin * tin;
      const int8_t *wr = w + oc * cin * ksize;
      for (int64_t t = 0; t < tout; ++t) {
        uint32_t acc = has_bias ? (uint32_t)bias[oc] : 0u;
        int64_t o = t * stride - padding;
        for (int64_t ic = 0; ic < cin; ++ic)
          for (int64_t k = 0; k < ksize; ++k) {
            int64_t p = o + k;
            if (p < 0 || p >= tin) continue;
            acc += (uint32_t)((int32_t)xb[ic * tin + p] * (int32_t)wr[ic * ksize + k]);
          }
        int32_t y = iwo_rshift(iwo_mulh(s32(acc), mult), rs);
        out[(b * cout + oc) * tout + t] = (int8_t)clampi(y, -127, 127);
      }
    }
}

/* ---------------- classifier: classifier/classifier_scalar.cpp:91-142 ---------------- */

void iwo_classifier(const int8_t *x, const int8_t *w, uint32_t mult,
                    int8_t shift, int8_t *out, int64_t M, int64_t K, int64_t N,
                    int nthreads) {
  uint32_t rs = (uint32_t)((int32_t)shift < 0 ? 0 : (int32_t)shift);
#pragma omp parallel for collapse(2) schedule(static) num_threads(nthr(nthreads))
  for (int64_t m = 0; m < M; ++m)
    for (int64_t n = 0; n < N; ++n) {
      int32_t y = iwo_rshift(iwo_mulh(s32(dot_s8(x + m * K, w + n * K, K)), mult), rs);
      out[m * N + n] = (int8_t)clampi(y, -127, 127);
    }
}

/* ---------------- attention: attention/attention_scalar.cpp ---------------- */

/* qk_requant_rowmax (attention_scalar.cpp:216-334): masked lanes store -32768
 * and are not part of the row max; rmp1 = row_max + 1 modulo 2^16. */
void iwo_qk_requant_rowmax(const int8_t *q, const int8_t *k,
                           const uint8_t *mask, int16_t *qk, int16_t *rmp1,
                           int64_t batch, int64_t heads, int64_t tq, int64_t tk,
                           int64_t dim, uint8_t mult, int32_t shift,
                           int has_mask, int nthreads) {
  uint32_t rs = (uint32_t)(shift > 0 ? shift : 0);
#pragma omp parallel for collapse(2) schedule(static) num_threads(nthr(nthreads))
  for (int64_t bh = 0; bh < batch * heads; ++bh)
    for (int64_t i = 0; i < tq; ++i) {
      const int8_t *qr = q + (bh * tq + i) * dim;
      int16_t *o = qk + (bh * tq + i) * tk;
      int16_t mx = -32768;
      for (int64_t j = 0; j < tk; ++j) {
        if (has_mask && mask[i * tk + j]) {
          o[j] = -32768;
          continue;
        }
        int32_t acc = s32(dot_s8(qr, k + (bh * tk + j) * dim, dim));
        int32_t v = iwo_rshift(s32((uint32_t)acc * (uint32_t)mult), rs);
        int16_t h = (int16_t)clampi(v, -32768, 32767);
        o[j] = h;
        if (h > mx) mx = h;
      }
      rmp1[bh * tq + i] = s16((uint32_t)(uint16_t)mx + 1u);
    }
}

/* One lane of shift_exp (attention_scalar.cpp:449-554); all int16 adds and
 * subtracts wrap modulo 2^16 as in the torch int16 golden. */
uint8_t iwo_shift_exp_one(int16_t x_sub, int32_t frac_bits) {
  if (x_sub > 0) return 0;
  int16_t half = (int16_t)(x_sub >> 1);
  int16_t sixteenth = (int16_t)(x_sub >> 4);
  int16_t fix = s16((uint32_t)(uint16_t)s16((uint32_t)(uint16_t)x_sub + (uint16_t)half) -
                    (uint32_t)(uint16_t)sixteenth);
  int16_t xi = (int16_t)(fix >> frac_bits);
  int16_t ip = s16((uint32_t)((int32_t)xi * (1 << frac_bits)));
  int16_t frac = s16((uint32_t)((int32_t)fix - (int32_t)ip));
  int16_t num = s16((uint32_t)((1 << frac_bits) + (int32_t)(frac >> 1)));
  int16_t e;
  if (xi > 0) {
    e = 0;
  } else {
    int32_t sh = -(int32_t)xi;
    e = sh >= 16 ? 0 : (int16_t)(num >> sh);
  }
  int32_t o = frac_bits > 7 ? ((int32_t)e >> (frac_bits - 7)) : (int32_t)e;
  return (uint8_t)o;
}

void iwo_shift_exp(const int16_t *qk, const int16_t *rmp1, const uint8_t *mask,
                   uint8_t *p, int32_t *row_sum, int64_t batch, int64_t heads,
                   int64_t tq, int64_t tk, int32_t frac_bits, int has_mask,
                   int nthreads) {
#pragma omp parallel for collapse(2) schedule(static) num_threads(nthr(nthreads))
  for (int64_t bh = 0; bh < batch * heads; ++bh)
    for (int64_t i = 0; i < tq; ++i) {
      int64_t base = (bh * tq + i) * tk;
      int16_t xm = rmp1[bh * tq + i];
      int32_t sum = 0;
      for (int64_t j = 0; j < tk; ++j) {
        if (has_mask && mask[i * tk + j]) {
          p[base + j] = 0;
          continue;
        }
        int16_t xs = s16((uint32_t)(uint16_t)qk[base + j] - (uint32_t)(uint16_t)xm);
        uint8_t v = iwo_shift_exp_one(xs, frac_bits);
        p[base + j] = v;
        sum += v;
      }
      row_sum[bh * tq + i] = sum;
    }
}

/* pv_norm_requant (attention_scalar.cpp:676-814): output layout [B,Tq,H*D]. */
int iwo_pv_norm_requant(const uint8_t *p, const int8_t *v,
                        const int32_t *row_sum, uint8_t av_mult, int8_t av_shift,
                        uint32_t rsqrt_offset, int8_t *out, int64_t batch,
                        int64_t heads, int64_t tq, int64_t tk, int64_t dim,
                        int nthreads) {
  for (int64_t i = 0; i < batch * heads * tq; ++i)
    if (row_sum[i] < 0) return -1;
  int32_t avs = av_shift;
  uint32_t rs = (uint32_t)(avs < 0 ? 0 : (avs > 32 ? 32 : avs));
#pragma omp parallel for collapse(2) schedule(static) num_threads(nthr(nthreads))
  for (int64_t bh = 0; bh < batch * heads; ++bh)
    for (int64_t i = 0; i < tq; ++i) {
      int64_t b = bh / heads, h = bh % heads;
      int32_t inv = iwo_fisr(row_sum[bh * tq + i], rsqrt_offset);
      const uint8_t *pr = p + (bh * tq + i) * tk;
      for (int64_t d = 0; d < dim; ++d) {
        const int8_t *vr = v + (bh * dim + d) * tk;
        uint32_t acc = 0;
        for (int64_t j = 0; j < tk; ++j) acc += (uint32_t)((int32_t)pr[j] * (int32_t)vr[j]);
        int32_t y = iwo_rshift(s32(acc * (uint32_t)inv), rsqrt_offset);
        y = iwo_rshift(s32((uint32_t)y * (uint32_t)inv), rsqrt_offset);
        y = iwo_rshift(s32((uint32_t)y * (uint32_t)av_mult), rs);
        out[(b * tq + i) * heads * dim + h * dim + d] = (int8_t)clampi(y, -127, 127);
      }
    }
  return 0;
}
