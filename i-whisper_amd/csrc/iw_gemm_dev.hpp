// Device helpers shared by the int8 MFMA GEMM kernels: operand chunk loads
// (dense rows, channels-last implicit-GEMM conv rows, byte gathers) and the
// fused integer epilogues with their per-column parameters.
#pragma once

#include "iw_common.hpp"
#include "iw_gemm.hpp"

namespace iw {
namespace gemm {

// Where the A tile comes from.
enum AMode : int {
  A_DENSE16 = 0,    // A[m][k] = a[m*lda + k], K % 16 == 0, 16-byte aligned rows
  A_CONVCL16 = 1,   // channels-last conv input x[b][t][c], C % 16 == 0
  A_GEN_DENSE = 2,  // any K / alignment, byte gathers
  A_GEN_CONVNCT = 3 // conv input in [B][Cin][Tin] layout, byte gathers
};

// Byte-wise 16-byte chunk gather for the generic modes.
__device__ __forceinline__ uint4 gather16(const GemmArgs &g, int amode, bool is_a, int64_t row,
                                          int64_t k0) {
  uint32_t w[4] = {0u, 0u, 0u, 0u};
  for (int i = 0; i < 16; ++i) {
    int64_t k = k0 + i;
    int32_t v = 0;
    if (k < g.K) {
      if (!is_a) {
        if (row < g.N) v = (uint8_t)g.b[row * g.ldb + k];
      } else if (amode == A_GEN_DENSE) {
        if (row < g.M) v = (uint8_t)g.a[row * g.lda + k];
      } else {  // A_GEN_CONVNCT: k = ic * ksize + kk
        if (row < g.M) {
          int64_t bb = row / g.conv_tout, t = row % g.conv_tout;
          int64_t ic = k / g.conv_ksize, kk = k % g.conv_ksize;
          int64_t pos = t * g.conv_stride - g.conv_pad + kk;
          if (pos >= 0 && pos < g.conv_tin)
            v = (uint8_t)g.a[(bb * g.conv_cin + ic) * g.conv_tin + pos];
        }
      }
    }
    w[i >> 2] |= (uint32_t)v << (8 * (i & 3));
  }
  return make_uint4(w[0], w[1], w[2], w[3]);
}

struct RowInfo {
  const int8_t *base;  // address of element k = 0 of this row (may be out of range)
  int32_t pos0;        // conv: first input position t*stride - pad
  bool valid;
};

__device__ __forceinline__ RowInfo a_row_info(const GemmArgs &g, int amode, int64_t m) {
  RowInfo r;
  r.valid = m < g.M;
  r.pos0 = 0;
  r.base = g.a;
  if (amode == A_DENSE16) {
    r.base = g.a + m * g.lda;
  } else if (amode == A_CONVCL16 && r.valid) {
    int64_t bb = m / g.conv_tout, t = m % g.conv_tout;
    r.pos0 = (int32_t)(t * g.conv_stride - g.conv_pad);
    r.base = g.a + (bb * g.conv_tin + r.pos0) * (int64_t)g.conv_cin;
  }
  return r;
}

__device__ __forceinline__ uint4 load_a16(const GemmArgs &g, int amode, const RowInfo &r,
                                          int64_t m, int64_t k) {
  if (amode == A_DENSE16) {
    if (r.valid && k < g.K) return *reinterpret_cast<const uint4 *>(r.base + k);
    return make_uint4(0, 0, 0, 0);
  }
  if (amode == A_CONVCL16) {
    if (r.valid && k < g.K) {
      int32_t pos = r.pos0 + (int32_t)(k / g.conv_cin);
      if (pos >= 0 && pos < g.conv_tin) return *reinterpret_cast<const uint4 *>(r.base + k);
    }
    return make_uint4(0, 0, 0, 0);
  }
  return gather16(g, amode, true, m, k);
}

__device__ __forceinline__ uint4 load_b16(const GemmArgs &g, bool fast, int64_t n, int64_t k) {
  if (fast) {
    if (n < g.N && k < g.K) return *reinterpret_cast<const uint4 *>(g.b + n * g.ldb + k);
    return make_uint4(0, 0, 0, 0);
  }
  return gather16(g, A_GEN_DENSE, false, n, k);
}

__device__ __forceinline__ int32_t sum16(uint4 v) {
  const int ones = 0x01010101;
  int32_t s = __builtin_amdgcn_sdot4((int)v.x, ones, 0, false);
  s = __builtin_amdgcn_sdot4((int)v.y, ones, s, false);
  s = __builtin_amdgcn_sdot4((int)v.z, ones, s, false);
  s = __builtin_amdgcn_sdot4((int)v.w, ones, s, false);
  return s;
}

// Round-half-away-from-zero right shift with the shift decoded once per
// column: rshift(x, s) == (x + half + (sign(x) & neg)) >> sh for s in [0, 31]
// (half = 2^(s-1), neg = -1 when s > 0, both 0 when s == 0), computed modulo 2^32.
struct Shift {
  uint32_t half;
  uint32_t neg;
  uint32_t sh;
};

__device__ __forceinline__ Shift make_shift(uint32_t s) {  // s in [0, 31]
  Shift r;
  r.sh = s;
  r.half = s ? (1u << (s - 1)) : 0u;
  r.neg = s ? 0xffffffffu : 0u;
  return r;
}

__device__ __forceinline__ int32_t apply_shift(int32_t x, const Shift &s) {
  const uint32_t t = (uint32_t)x + s.half + ((uint32_t)(x >> 31) & s.neg);
  return (int32_t)t >> s.sh;
}

// mulh with a uint32 multiplier: high word of the signed 64-bit product.
__device__ __forceinline__ int32_t mulh_su(int32_t a, uint32_t m) {
  return (int32_t)(__umulhi((uint32_t)a, m) - ((uint32_t)(a >> 31) & m));
}

// Per-output-channel epilogue parameters, decoded once per column.
struct ColParams {
  uint32_t wz;    // zero point (as uint32 for the wrap-around product)
  uint32_t bias;
  uint32_t mult;  // 0 when the reference semantics give a zero result
  Shift shift;    // requant shift (Linear8 / per-tensor); Linear32: sh = left shift
  // GeLU
  uint32_t gi_m;
  Shift gi_s;
  uint32_t go_m;
  Shift go_s;
  // positional add_requant15
  uint32_t pe_m;
  Shift pe_s;
};

// The per-column parameter values as stored, before decoding: a kernel can
// request them early and decode them (decode_col) after its main loop, so
// that no wait for them lands in between.
struct ColRaw {
  int32_t wz, bias, s, is, os, ps;
  uint32_t m, im, om, pm;
};

// Fields whose pointer is null stay unset here and are never read by
// decode_col, so no select consumes a loaded value before it is needed.
__device__ __forceinline__ ColRaw load_col_raw(const GemmArgs &g, int64_t n) {
  ColRaw r;
  if (g.wz) r.wz = g.wz[n];
  if (g.bias) r.bias = g.bias[n];
  if (g.mult) r.m = g.mult[g.mult_pc ? n : 0];
  if (g.shift) r.s = g.shift[g.mult_pc ? n : 0];
  if (g.lut) {
    r.is = g.luti_s[g.luti_pc ? n : 0];
    r.os = g.luto_s[g.luto_pc ? n : 0];
    r.im = g.luti_m[g.luti_pc ? n : 0];
    r.om = g.luto_m[g.luto_pc ? n : 0];
  }
  if (g.pe) {
    r.pm = g.pe_mult[g.pe_mpc ? n : 0];
    r.ps = g.pe_shift[g.pe_spc ? n : 0];
  }
  return r;
}

template <int EPI>
__device__ __forceinline__ ColParams decode_col(const GemmArgs &g, const ColRaw &r) {
  ColParams c;
  c.wz = g.wz ? (uint32_t)r.wz : 0u;
  c.bias = g.bias ? (uint32_t)r.bias : 0u;
  uint32_t m = g.mult ? r.m : g.scalar_mult;
  int32_t s = g.shift ? r.s : g.scalar_shift;
  if (EPI == EPI_L8) {
    // linear8_scalar.cpp:71-74: a shift outside [0, 31] gives 0
    if (s < 0 || s >= 32) m = 0, s = 0;
  } else if (EPI == EPI_S8) {
    // classifier / conv: shift clamped at 0; >= 32 gives 0
    if (s < 0) s = 0;
    if (s >= 32) m = 0, s = 0;
  } else {
    // Linear32: (mulh << s), 0 outside [0, 31]
    if (s < 0 || s >= 32) m = 0, s = 0;
  }
  c.mult = m;
  c.shift = make_shift((uint32_t)s);
  if (EPI == EPI_L32 || EPI == EPI_L32RES) c.shift.sh = (uint32_t)s;
  c.gi_m = c.go_m = c.pe_m = 0;
  c.gi_s = c.go_s = c.pe_s = make_shift(0);
  if (g.lut) {
    int32_t is = r.is < 0 ? 0 : r.is;  // gelu_scalar.cpp: shifts clamped to [0, 32]
    int32_t os = r.os < 0 ? 0 : r.os;
    uint32_t im = r.im, om = r.om;
    if (is >= 32) im = 0, is = 0;
    if (os >= 32) om = 0, os = 0;
    c.gi_m = im;
    c.gi_s = make_shift((uint32_t)is);
    c.go_m = om;
    c.go_s = make_shift((uint32_t)os);
  }
  if (g.pe) {
    uint32_t pm = r.pm;
    int32_t ps = r.ps < 0 ? 0 : r.ps;
    if (ps >= 32) pm = 0, ps = 0;
    c.pe_m = pm;
    c.pe_s = make_shift((uint32_t)ps);
  }
  return c;
}

template <int EPI>
__device__ __forceinline__ ColParams load_col(const GemmArgs &g, int64_t n) {
  return decode_col<EPI>(g, load_col_raw(g, n));
}

// Integer GeLU on a clamped int8 value with decoded parameters
// (gelu/gelu_scalar.cpp:29-180). |y| <= 127 and the multipliers are 8-bit, so
// every product fits the 24-bit multiplier exactly (|y*lut*luto_m| < 2^23).
__device__ __forceinline__ int32_t gelu_dec(int32_t y, const uint8_t *lut, const ColParams &c) {
  int32_t idx = apply_shift(__mul24(y, (int32_t)c.gi_m), c.gi_s) + 8;
  idx = clampi(idx, 0, 15);
  const int32_t v = __mul24(__mul24(y, (int32_t)lut[idx]), (int32_t)c.go_m);
  return clampi(apply_shift(v, c.go_s), -127, 127);
}

// The accumulator after the zero-point and bias terms, modulo 2^32.
__device__ __forceinline__ uint32_t corrected(int32_t acc, int32_t xsum, const ColParams &c) {
  return (uint32_t)acc - c.wz * (uint32_t)xsum + c.bias;
}

// The same for K <= 32768: the zero point is an int8 and |row sum| <= 128 K
// <= 2^22, so the product is exact in the 24-bit multiplier.
__device__ __forceinline__ uint32_t corrected_k32k(int32_t acc, int32_t xsum, const ColParams &c) {
  return (uint32_t)acc - (uint32_t)__mul24((int32_t)c.wz, xsum) + c.bias;
}

// Epilogue of one output element of the decode GEMMs: `a` is the
// accumulator after the zero-point and bias terms, m / n its row and column,
// `res` the residual input of Linear32 + residual15.
template <int EPI, bool GELU, bool SCATTER, bool OUT_FRAG = false>
__device__ __forceinline__ void skinny_store(const GemmArgs &g, const SkinnyScatter &sc,
                                             const ColParams &c, const uint8_t *lut, int pos, int m,
                                             int n, uint32_t a, int32_t res) {
  if (EPI == EPI_L8 || EPI == EPI_S8) {
    int32_t y = clampi(apply_shift(mulh_su((int32_t)a, c.mult), c.shift), -127, 127);
    if (GELU) y = gelu_dec(y, lut, c);
    if (SCATTER) {
      // columns [0, C): Q; [C, 2C): K appended at position pos + (m % T)
      // of the [B, H, T_cache, D] cache; [2C, 3C): V appended to the V
      // cache, transposed [B, H, D, T_cache] or in key quads
      // [B, H, T_cache / 4, D, 4]
      const int b = m / sc.T, t = pos + m % sc.T;
      if (n < sc.C) {
        sc.q[(int64_t)m * sc.ldq + n] = (int8_t)y;
      } else if (t < 0 || t >= sc.t_cap) {
        // position outside the cache: nothing is appended
      } else if (n < 2 * sc.C) {
        const int h = (n - sc.C) / sc.D, d = (n - sc.C) % sc.D;
        sc.k[(int64_t)b * sc.k_sb + (int64_t)h * sc.k_sh + (int64_t)t * sc.k_st + d] = (int8_t)y;
      } else {
        const int h = (n - 2 * sc.C) / sc.D, d = (n - 2 * sc.C) % sc.D;
        sc.v[(int64_t)b * sc.v_sb + (int64_t)h * sc.v_sh + (int64_t)d * sc.v_sd + (int64_t)(t >> 2) * sc.v_sq +
             (t & 3)] = (int8_t)y;
      }
    } else if (OUT_FRAG) {
      // fragment-major output: g.ldc is its padded K
      reinterpret_cast<int8_t *>(g.out)[frag_offset(m, n, g.ldc)] = (int8_t)y;
    } else {
      reinterpret_cast<int8_t *>(g.out)[(int64_t)m * g.ldc + n] = (int8_t)y;
    }
  } else {
    const int32_t br = (int32_t)((uint32_t)mulh_su((int32_t)a, c.mult) << c.shift.sh);
    if (EPI == EPI_L32) {
      reinterpret_cast<int32_t *>(g.out)[(int64_t)m * g.ldc + n] = br;
    } else {
      const uint32_t v = (uint32_t)br + (uint32_t)(res * (int32_t)g.res_mult);
      const int32_t y = clampi(rshift_pos((int32_t)v, 15), -16383, 16383);
      reinterpret_cast<int16_t *>(g.out)[(int64_t)m * g.ldc + n] = (int16_t)y;
    }
  }
}

__device__ __forceinline__ int32_t sum16v(v4i v, int32_t acc) {
  const int ones = 0x01010101;
  acc = __builtin_amdgcn_sdot4(v[0], ones, acc, false);
  acc = __builtin_amdgcn_sdot4(v[1], ones, acc, false);
  acc = __builtin_amdgcn_sdot4(v[2], ones, acc, false);
  return __builtin_amdgcn_sdot4(v[3], ones, acc, false);
}

// Round-half-away-from-zero right shift (the Shift rule) in three operations:
// the sign term is a one-bit field extract whose width is 0 for a zero shift.
struct EpiShift {
  uint32_t half, sh, w;
  __device__ __forceinline__ void set(uint32_t h, uint32_t s) { half = h, sh = s, w = min(s, 1u); }
  __device__ __forceinline__ int32_t apply(uint32_t x) const {
    const uint32_t sgn = (uint32_t)__builtin_amdgcn_sbfe((int32_t)x, 31, w);
    return (int32_t)(x + half + sgn) >> sh;
  }
};

// Per-column requantization operands for one output column.
struct EpiCol {
  int32_t m;      // multiplier as int32 (mneg restores the unsigned value)
  uint32_t mneg;  // all ones when the multiplier is >= 2^31
  uint32_t half, sh;
  int32_t nz;     // negated zero point
  uint32_t b;
  __device__ __forceinline__ void set(uint32_t mult, uint32_t shift, uint32_t nzp, uint32_t bias) {
    m = (int32_t)mult, mneg = (uint32_t)((int32_t)mult >> 31), sh = shift, nz = (int32_t)nzp, b = bias;
  }
  // acc - wz * rowsum + bias, modulo 2^32 (|wz * rowsum| < 2^31 for K <= 32768)
  __device__ __forceinline__ uint32_t corrected(int32_t acc, int32_t xsum) const {
    return (uint32_t)__mul24(nz, xsum) + (uint32_t)acc + b;
  }
  // high word of the signed x unsigned 64-bit product
  __device__ __forceinline__ int32_t mulh(uint32_t x) const {
    return (int32_t)((uint32_t)__mulhi((int32_t)x, m) + (x & mneg));
  }
  // Linear8 / per-tensor int8: clamp(rshift(mulh(corrected), s), -127, 127)
  __device__ __forceinline__ int32_t requant8(int32_t acc, int32_t xsum) const {
    const uint32_t hi = (uint32_t)mulh(corrected(acc, xsum));
    const uint32_t sgn = (uint32_t)__builtin_amdgcn_sbfe((int32_t)hi, 31, min(sh, 1u));
    return clampi((int32_t)(hi + half + sgn) >> sh, -127, 127);
  }
  // Linear32: mulh(corrected) << s
  __device__ __forceinline__ uint32_t pre_residual(int32_t acc, int32_t xsum) const {
    return (uint32_t)mulh(corrected(acc, xsum)) << sh;
  }
};

}  // namespace gemm
}  // namespace iw
