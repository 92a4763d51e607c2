// Row-wise and element-wise integer kernels: LayerNorm32, FISR, GeLU,
// residual15, add_requant15, token-embedding gather, log-mel quantization and
// the greedy argmax. All are HBM-bound; each reads and writes its operands
// once.
#include "iw_common.hpp"
#include "iw_gemm.hpp"
#include "iw_kernels.hpp"

namespace iw {

namespace {

__device__ __forceinline__ uint32_t wave_sum_u32(uint32_t v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += (uint32_t)__shfl_xor((int)v, o);
  return v;
}

__device__ __forceinline__ int32_t wave_max_i32(int32_t v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = max(v, __shfl_xor(v, o));
  return v;
}

typedef short s16x2 __attribute__((ext_vector_type(2)));

// LayerNorm32 (layernorm/layernorm_scalar.cpp:464-624), one wave per row.
// The row lives in registers: lane l owns 4-element chunks l, l + 64, ...
// The waves are persistent: each loads its lanes' gamma / beta once, then
// walks the rows wave_id, wave_id + waves, ..., requesting the next row
// before reducing the current one.
//
// The integer steps are the reference's; their arithmetic is arranged for
// the VALU, which bounds this kernel at encoder sizes:
// * one pass over the raw int16 pairs gives the sum (v_dot2 with ones) and
//   the row's largest and smallest value (packed max / min), reduced
//   together with DPP moves;
// * max_e int32(d_e^2), d = x - mean, is max(xmax - mean, mean - xmin)^2
//   whenever every |d| <= 46340 (then no d^2 wraps, and d^2 grows with |d|);
//   a row outside that range takes the per-element form;
// * d^2 and the (non-negative) rounding shift of the variance sum use 24-bit
//   multiply-adds; d * inv * ln_m is d * K with K = inv * ln_m (mod 2^32)
//   formed once per row (written as two 24-bit products, which the compiler
//   may fuse back into one 32-bit multiply), and mulh is a signed high
//   multiply with a mask correction for multipliers >= 2^31.
constexpr int LN_MAX_CHUNKS = 5;  // 1280 / 4 / 64

__global__ __launch_bounds__(256) void layernorm32_kernel(
    const int16_t *__restrict__ x, const int8_t *__restrict__ gamma,
    const int32_t *__restrict__ beta, uint32_t ln_m, int32_t ln_s, uint32_t out_m,
    int32_t out_s, uint32_t rsqrt_off, int8_t *__restrict__ out, int64_t rows, int hidden,
    int code) {
  const int lane = threadIdx.x & 63;
  const int64_t wave_id = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  const int64_t waves = (int64_t)gridDim.x * (blockDim.x >> 6);
  if (wave_id >= rows) return;
  const int nch = hidden >> 2;  // >= 96: every lane owns chunk 0
  auto load_row = [&](int64_t r, uint2 *w) {
    const int16_t *xr = x + r * hidden;
#pragma unroll
    for (int c = 0; c < LN_MAX_CHUNKS; ++c) {
      const int ch = lane + 64 * c;
      w[c] = ch < nch ? *reinterpret_cast<const uint2 *>(xr + ch * 4) : make_uint2(0, 0);
    }
  };
  uint2 xa[LN_MAX_CHUNKS];
  load_row(wave_id, xa);
  const bool g_al = (reinterpret_cast<uintptr_t>(gamma) & 3) == 0;
  const bool b_al = beta && (reinterpret_cast<uintptr_t>(beta) & 15) == 0;
  uint32_t gw[LN_MAX_CHUNKS];
  uint4 bw[LN_MAX_CHUNKS];
#pragma unroll
  for (int c = 0; c < LN_MAX_CHUNKS; ++c) {
    const int ch = lane + 64 * c;
    gw[c] = 0;
    bw[c] = make_uint4(0, 0, 0, 0);
    if (ch < nch) {
      if (g_al) {
        gw[c] = *reinterpret_cast<const uint32_t *>(gamma + ch * 4);
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) gw[c] |= (uint32_t)(uint8_t)gamma[ch * 4 + e] << (8 * e);
      }
      if (b_al) {
        bw[c] = *reinterpret_cast<const uint4 *>(beta + ch * 4);
      } else if (beta) {
        bw[c] = make_uint4((uint32_t)beta[ch * 4], (uint32_t)beta[ch * 4 + 1],
                           (uint32_t)beta[ch * 4 + 2], (uint32_t)beta[ch * 4 + 3]);
      }
    }
  }
  // rshift by out_s: a shift >= 32 (or negative) gives 0, as a zero multiplier does
  const bool out_zero = (uint32_t)out_s >= 32;
  const uint32_t om = out_zero ? 0u : out_m;
  const uint32_t osh = out_zero ? 0u : (uint32_t)out_s;
  const uint32_t omneg = (uint32_t)((int32_t)om >> 31);
  const s16x2 ones = {1, 1};
  // one row: xw holds its raw values on entry and is refilled with row
  // `next` (if any) as soon as they are unpacked
  auto process = [&](int64_t row, uint2 *xw, int64_t next) {
    int32_t sum = 0;
    s16x2 mx2 = {-32768, -32768}, mn2 = {32767, 32767};
#pragma unroll
    for (int c = 0; c < LN_MAX_CHUNKS; ++c) {
      if (lane + 64 * c < nch) {
        const s16x2 p0 = __builtin_bit_cast(s16x2, xw[c].x), p1 = __builtin_bit_cast(s16x2, xw[c].y);
        sum = __builtin_amdgcn_sdot2(p0, ones, sum, false);
        sum = __builtin_amdgcn_sdot2(p1, ones, sum, false);
        mx2 = __builtin_elementwise_max(mx2, __builtin_elementwise_max(p0, p1));
        mn2 = __builtin_elementwise_min(mn2, __builtin_elementwise_min(p0, p1));
      }
    }
    int32_t v[LN_MAX_CHUNKS][4];
#pragma unroll
    for (int c = 0; c < LN_MAX_CHUNKS; ++c) {
      v[c][0] = (int16_t)(xw[c].x & 0xffff);
      v[c][1] = (int16_t)(xw[c].x >> 16);
      v[c][2] = (int16_t)(xw[c].y & 0xffff);
      v[c][3] = (int16_t)(xw[c].y >> 16);
    }
    if (next < rows) load_row(next, xw);
    const int32_t total = (int32_t)wave_sum_dpp((uint32_t)sum);
    const int32_t xmax = wave_max_dpp(max((int32_t)mx2.x, (int32_t)mx2.y));
    const int32_t xmin = -wave_max_dpp(-min((int32_t)mn2.x, (int32_t)mn2.y));
    const int32_t mean = norm_reduce(total, code);
#pragma unroll
    for (int c = 0; c < LN_MAX_CHUNKS; ++c)
#pragma unroll
      for (int e = 0; e < 4; ++e) v[c][e] -= mean;  // d
    const int32_t maxabs = max(xmax - mean, mean - xmin);
    const bool fast = maxabs <= 46340;  // wave-uniform
    int32_t maxsq;
    if (fast) {
      maxsq = maxabs * maxabs;
    } else {
      maxsq = 0;
#pragma unroll
      for (int c = 0; c < LN_MAX_CHUNKS; ++c)
        if (lane + 64 * c < nch)
#pragma unroll
          for (int e = 0; e < 4; ++e) maxsq = max(maxsq, (int32_t)((uint32_t)v[c][e] * (uint32_t)v[c][e]));
      maxsq = wave_max_dpp(maxsq);
    }
    int32_t rs = bitlen(maxsq) - 16;
    rs = rs < 0 ? 0 : rs;
    rs = (rs + 1) & ~1;
    uint32_t vs = 0;
    if (fast) {
      // d^2 < 2^31 and rs <= 16: rshift of a non-negative value, no wrap
      const int32_t half = rs ? 1 << (rs - 1) : 0;
#pragma unroll
      for (int c = 0; c < LN_MAX_CHUNKS; ++c)
        if (lane + 64 * c < nch)
#pragma unroll
          for (int e = 0; e < 4; ++e) vs += (uint32_t)(__mul24(v[c][e], v[c][e]) + half) >> rs;
    } else {
#pragma unroll
      for (int c = 0; c < LN_MAX_CHUNKS; ++c)
        if (lane + 64 * c < nch)
#pragma unroll
          for (int e = 0; e < 4; ++e)
            vs += (uint32_t)rshift((int32_t)((uint32_t)v[c][e] * (uint32_t)v[c][e]), (uint32_t)rs);
    }
    const int32_t var = norm_reduce((int32_t)wave_sum_dpp(vs), code);
    const int32_t inv = fisr(var, rsqrt_off);
    // t = d * inv * ln_m modulo 2^32 = d * K; a shift >= 32 gives 0 (K = 0)
    uint32_t nshift = (uint32_t)(ln_s + (rs >> 1));
    uint32_t K = (uint32_t)inv * ln_m;
    if (nshift >= 32) K = 0, nshift = 0;
    const int32_t klo = (int32_t)(K & 0xffffu), khi = (int32_t)(K >> 16);
    const uint32_t nhalf = nshift ? 1u << (nshift - 1) : 0u, nw = min(nshift, 1u);
    const uint32_t ohalf = osh ? 1u << (osh - 1) : 0u, ow = min(osh, 1u);
    int8_t *orow = out + row * hidden;
#pragma unroll
    for (int c = 0; c < LN_MAX_CHUNKS; ++c) {
      const int ch = lane + 64 * c;
      if (ch < nch) {
        uint32_t packed = 0;
        const uint32_t bv[4] = {bw[c].x, bw[c].y, bw[c].z, bw[c].w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int32_t d = v[c][e];  // |d| < 2^17: exact in the 24-bit multiplier
          const uint32_t t = (uint32_t)__mul24(d, klo) + ((uint32_t)__mul24(d, khi) << 16);
          const uint32_t ts = (uint32_t)__builtin_amdgcn_sbfe((int32_t)t, 31, nw);
          const int32_t y = clampi((int32_t)(t + nhalf + ts) >> nshift, -16383, 16383);
          const uint32_t a = (uint32_t)__mul24(y, (int32_t)(int8_t)(gw[c] >> (8 * e))) + bv[e];
          // mulh(a, om): signed high word, plus a when om >= 2^31
          const uint32_t hi = (uint32_t)__mulhi((int32_t)a, (int32_t)om) + (a & omneg);
          const uint32_t hs = (uint32_t)__builtin_amdgcn_sbfe((int32_t)hi, 31, ow);
          const int32_t o = clampi((int32_t)(hi + ohalf + hs) >> osh, -127, 127);
          packed |= ((uint32_t)(uint8_t)(int8_t)o) << (8 * e);
        }
        *reinterpret_cast<uint32_t *>(orow + ch * 4) = packed;
      }
    }
  };
  // rows wave_id + k * waves, the next one in flight
  for (int64_t row = wave_id; row < rows; row += waves) process(row, xa, row + waves);
}

// LayerNorm32 for few rows (a decode step): one row per block of 256 threads,
// thread t owning elements t, t + 256, ... so that each row's arithmetic is
// spread over four SIMDs. Same integer steps as layernorm32_kernel. With
// pf.w set, the blocks also read the next decode GEMM's weight tiles into
// their XCDs' L2 (behind the row's own loads).
constexpr int LNR_MAX = 5;  // 1280 / 256
__global__ __launch_bounds__(256) void layernorm32_row_kernel(
    const int16_t *__restrict__ x, const int8_t *__restrict__ gamma,
    const int32_t *__restrict__ beta, uint32_t ln_m, int32_t ln_s, uint32_t out_m,
    int32_t out_s, uint32_t rsqrt_off, int8_t *__restrict__ out, int hidden, int code,
    int64_t out_frag_kp, FragPrefetch pf) {
  __shared__ uint32_t sA[4], sB[4], sC[4];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t row = blockIdx.x;
  const int16_t *xr = x + row * hidden;
  int32_t v[LNR_MAX], gm[LNR_MAX], bt[LNR_MAX];
  uint32_t sum = 0;
#pragma unroll
  for (int j = 0; j < LNR_MAX; ++j) {
    const int e = tid + 256 * j;
    const bool ok = e < hidden;
    v[j] = ok ? xr[e] : 0;
    gm[j] = ok ? gamma[e] : 0;
    bt[j] = (ok && beta) ? beta[e] : 0;
  }
  // 4 lines per thread: 1 MB per XCD at 128 rows, more than any decode
  // GEMM's weight share (FC1's is 0.8 MB at Whisper-large)
  uint32_t pfv[4];
  frag_prefetch_issue(pf, xr, pfv);
#pragma unroll
  for (int j = 0; j < LNR_MAX; ++j) sum += (uint32_t)v[j];
  sum = wave_sum_dpp(sum);
  if (lane == 0) sA[wave] = sum;
  __syncthreads();
  const int32_t mean = norm_reduce((int32_t)(sA[0] + sA[1] + sA[2] + sA[3]), code);
  int32_t maxsq = 0;
#pragma unroll
  for (int j = 0; j < LNR_MAX; ++j) {
    if (tid + 256 * j < hidden) {
      const int32_t d = v[j] - mean;
      maxsq = max(maxsq, (int32_t)((uint32_t)d * (uint32_t)d));
    }
  }
  maxsq = wave_max_dpp(maxsq);
  if (lane == 0) sB[wave] = (uint32_t)maxsq;
  __syncthreads();
  maxsq = max(max((int32_t)sB[0], (int32_t)sB[1]), max((int32_t)sB[2], (int32_t)sB[3]));
  int32_t rs = bitlen(maxsq) - 16;
  rs = rs < 0 ? 0 : rs;
  rs = (rs + 1) & ~1;
  uint32_t vs = 0;
#pragma unroll
  for (int j = 0; j < LNR_MAX; ++j) {
    if (tid + 256 * j < hidden) {
      const int32_t d = v[j] - mean;
      vs += (uint32_t)rshift((int32_t)((uint32_t)d * (uint32_t)d), (uint32_t)rs);
    }
  }
  vs = wave_sum_dpp(vs);
  if (lane == 0) sC[wave] = vs;
  __syncthreads();
  const int32_t var = norm_reduce((int32_t)(sC[0] + sC[1] + sC[2] + sC[3]), code);
  const int32_t inv = fisr(var, rsqrt_off);
  const uint32_t nshift = (uint32_t)(ln_s + (rs >> 1));
  int8_t *orow = out + row * hidden;
#pragma unroll
  for (int j = 0; j < LNR_MAX; ++j) {
    const int e = tid + 256 * j;
    if (e < hidden) {
      const int32_t d = v[j] - mean;
      const uint32_t t = (uint32_t)d * (uint32_t)inv * ln_m;
      const int32_t y = clampi(rshift((int32_t)t, nshift), -16383, 16383);
      const uint32_t a = (uint32_t)y * (uint32_t)gm[j] + (uint32_t)bt[j];
      const int8_t yo = (int8_t)clampi(rshift(mulh((int32_t)a, out_m), (uint32_t)out_s), -127, 127);
      // row-major, or the fragment-major operand image of a decode GEMM
      if (out_frag_kp)
        out[frag_offset(row, e, out_frag_kp)] = yo;
      else
        orow[e] = yo;
    }
  }
  frag_prefetch_keep(pfv);
}

__global__ void rsqrt_kernel(const int32_t *x, int32_t *out, int64_t n, uint32_t off) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) out[i] = fisr(x[i], off);
}

__global__ void gelu_kernel(const int8_t *__restrict__ x, const uint8_t *__restrict__ lut,
                            const uint8_t *luti_m, const int8_t *luti_s, const uint8_t *luto_m,
                            const int8_t *luto_s, int8_t *__restrict__ out, int64_t numel,
                            int64_t channels, int luti_pc, int luto_pc) {
  __shared__ uint8_t sl[16];
  if (threadIdx.x < 16) sl[threadIdx.x] = lut[threadIdx.x];
  __syncthreads();
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < numel; i += stride) {
    const int64_t c = i % channels;
    const int64_t a = luti_pc ? c : 0, b = luto_pc ? c : 0;
    out[i] = gelu_one(x[i], sl, luti_m[a], luti_s[a], luto_m[b], luto_s[b]);
  }
}

__global__ void residual15_kernel(const int32_t *__restrict__ br, const int16_t *__restrict__ res,
                                  uint32_t m, int16_t *__restrict__ out, int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    uint32_t v = (uint32_t)br[i] + (uint32_t)((int32_t)res[i] * (int32_t)m);
    out[i] = (int16_t)clampi(rshift_pos((int32_t)v, 15), -16383, 16383);
  }
}

// add_requant15 (add_requant15/add_requant15_scalar.cpp:29-81). When tokens is
// set, the int8 input row is gathered from the token embedding table first
// (TextDecoder_int input, model_int.py:1411-1439).
__global__ void add_requant15_kernel(const int8_t *__restrict__ x, const int64_t *__restrict__ tokens,
                                     const int8_t *__restrict__ addend,
                                     const uint16_t *__restrict__ mult,
                                     const int8_t *__restrict__ shift, int16_t *__restrict__ out,
                                     int64_t positions, int64_t channels, int64_t total, int mpc,
                                     int spc, const int32_t *__restrict__ pos, int64_t addend_rows) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  // with pos, addend rows start at the device-side position (clamped to the table)
  const int64_t p0 = pos ? min(max((int64_t)*pos, (int64_t)0), addend_rows - positions) : 0;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    const int64_t c = i % channels;
    const int64_t bt = i / channels;
    const int64_t t = bt % positions + p0;
    const int32_t xv = tokens ? (int32_t)x[tokens[bt] * channels + c] : (int32_t)x[i];
    const int32_t v = xv + (int32_t)addend[t * channels + c];
    const int32_t p = (int32_t)((uint32_t)v * (uint32_t)mult[mpc ? c : 0]);
    const int32_t s = shift[spc ? c : 0];
    out[i] = (int16_t)clampi(rshift(p, (uint32_t)(s < 0 ? 0 : s)), -16383, 16383);
  }
}

// Vector forms of the two elementwise kernels above for rows of a multiple
// of 16 channels and 16-byte aligned operands: each thread takes 16
// consecutive elements of one row (16-byte loads and stores), reads the
// per-channel parameters as 16-channel vectors, and walks the grid with
// running (row, channel) counters instead of a division per element.
struct PieceWalk {
  int64_t p, row;
  uint32_t c;  // piece within the row
  int64_t drow;
  uint32_t dc, cp;
  __device__ PieceWalk(int64_t start, int64_t stride, uint32_t cpieces) {
    p = start;
    row = start / cpieces;
    c = (uint32_t)(start % cpieces);
    drow = stride / cpieces;
    dc = (uint32_t)(stride % cpieces);
    cp = cpieces;
  }
  // returns the number of rows advanced
  __device__ int64_t next(int64_t stride) {
    p += stride;
    c += dc;
    int64_t adv = drow;
    if (c >= cp) c -= cp, ++adv;
    row += adv;
    return adv;
  }
};

__device__ __forceinline__ uint32_t byte_of(const uint4 &v, int i) {
  const uint32_t w = i < 4 ? v.x : (i < 8 ? v.y : (i < 12 ? v.z : v.w));
  return (w >> (8 * (i & 3))) & 0xffu;
}

__global__ __launch_bounds__(256) void gelu16_kernel(const int8_t *__restrict__ x, const uint8_t *__restrict__ lut,
                                                     const uint8_t *__restrict__ luti_m,
                                                     const int8_t *__restrict__ luti_s,
                                                     const uint8_t *__restrict__ luto_m,
                                                     const int8_t *__restrict__ luto_s, int8_t *__restrict__ out,
                                                     int64_t pieces, uint32_t cpieces, int luti_pc, int luto_pc) {
  __shared__ uint8_t sl[16];
  if (threadIdx.x < 16) sl[threadIdx.x] = lut[threadIdx.x];
  __syncthreads();
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  const int64_t start = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (start >= pieces) return;
  // per-tensor parameters as broadcast vectors
  const uint4 bim = make_uint4(luti_m[0] * 0x01010101u, 0, 0, 0), bis = make_uint4((uint8_t)luti_s[0] * 0x01010101u, 0, 0, 0);
  const uint4 bom = make_uint4(luto_m[0] * 0x01010101u, 0, 0, 0), bos = make_uint4((uint8_t)luto_s[0] * 0x01010101u, 0, 0, 0);
  for (PieceWalk w(start, stride, cpieces); w.p < pieces; w.next(stride)) {
    const uint4 xv = *reinterpret_cast<const uint4 *>(x + w.p * 16);
    const int64_t c0 = (int64_t)w.c * 16;
    const uint4 im = luti_pc ? *reinterpret_cast<const uint4 *>(luti_m + c0) : bim;
    const uint4 is = luti_pc ? *reinterpret_cast<const uint4 *>(luti_s + c0) : bis;
    const uint4 om = luto_pc ? *reinterpret_cast<const uint4 *>(luto_m + c0) : bom;
    const uint4 os = luto_pc ? *reinterpret_cast<const uint4 *>(luto_s + c0) : bos;
    uint32_t o[4] = {0, 0, 0, 0};
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int pi = luti_pc ? i : 0, po = luto_pc ? i : 0;
      const int8_t y = gelu_one((int8_t)byte_of(xv, i), sl, byte_of(im, pi), (int8_t)byte_of(is, pi),
                                byte_of(om, po), (int8_t)byte_of(os, po));
      o[i >> 2] |= (uint32_t)(uint8_t)y << (8 * (i & 3));
    }
    *reinterpret_cast<uint4 *>(out + w.p * 16) = make_uint4(o[0], o[1], o[2], o[3]);
  }
}

__global__ __launch_bounds__(256) void add_requant15_16_kernel(
    const int8_t *__restrict__ x, const int64_t *__restrict__ tokens, const int8_t *__restrict__ addend,
    const uint16_t *__restrict__ mult, const int8_t *__restrict__ shift, int16_t *__restrict__ out,
    int64_t positions, int64_t channels, int64_t pieces, int mpc, int spc, const int32_t *__restrict__ pos,
    int64_t addend_rows) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  const int64_t start = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (start >= pieces) return;
  const int64_t p0 = pos ? min(max((int64_t)*pos, (int64_t)0), addend_rows - positions) : 0;
  const uint32_t cpieces = (uint32_t)(channels / 16);
  const uint32_t m0 = mult[0];
  const int32_t s0 = shift[0];
  PieceWalk w(start, stride, cpieces);
  // t = row % positions, kept as a running counter too
  int64_t t = w.row % positions;
  const int64_t dt = w.drow % positions;
  for (; w.p < pieces;) {
    const int64_t c0 = (int64_t)w.c * 16;
    const int8_t *xr = tokens ? x + tokens[w.row] * channels + c0 : x + w.p * 16;
    const uint4 xv = *reinterpret_cast<const uint4 *>(xr);
    const uint4 av = *reinterpret_cast<const uint4 *>(addend + (t + p0) * channels + c0);
    uint4 mv0 = make_uint4(0, 0, 0, 0), mv1 = mv0, sv = mv0;
    if (mpc) {
      mv0 = *reinterpret_cast<const uint4 *>(mult + c0);
      mv1 = *reinterpret_cast<const uint4 *>(mult + c0 + 8);
    }
    if (spc) sv = *reinterpret_cast<const uint4 *>(shift + c0);
    uint32_t o[8];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int32_t v = (int32_t)(int8_t)byte_of(xv, i) + (int32_t)(int8_t)byte_of(av, i);
      uint32_t m = m0;
      if (mpc) {
        const uint4 &mv = i < 8 ? mv0 : mv1;
        const int j = i & 7;
        const uint32_t ww = j < 2 ? mv.x : (j < 4 ? mv.y : (j < 6 ? mv.z : mv.w));
        m = (ww >> (16 * (j & 1))) & 0xffffu;
      }
      const int32_t sh = spc ? (int32_t)(int8_t)byte_of(sv, i) : s0;
      const int32_t pr = (int32_t)((uint32_t)v * m);
      const uint32_t r = (uint32_t)(uint16_t)(int16_t)clampi(rshift(pr, (uint32_t)(sh < 0 ? 0 : sh)), -16383, 16383);
      if (i & 1)
        o[i >> 1] |= r << 16;
      else
        o[i >> 1] = r;
    }
    uint4 *op = reinterpret_cast<uint4 *>(out + w.p * 16);
    op[0] = make_uint4(o[0], o[1], o[2], o[3]);
    op[1] = make_uint4(o[4], o[5], o[6], o[7]);
    const int64_t adv = w.next(stride);
    t += dt + (adv - w.drow);  // adv is drow or drow + 1
    if (t >= positions) t -= positions;
  }
}

// Encoder input quantization round(mel * alpha) clamped to +-127
// (model_int.py:1265-1267; round half to even as torch.round), written
// channels-last [B][T][n_mels] for the implicit-GEMM conv.
__global__ void quantize_mel_kernel(const float *__restrict__ mel, float alpha,
                                    int8_t *__restrict__ out, int64_t nb, int64_t nm, int64_t nt) {
  const int64_t total = nb * nm * nt;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    // i indexes the output [b][t][m]
    const int64_t m = i % nm;
    const int64_t bt = i / nm;
    const int64_t t = bt % nt, b = bt / nt;
    const float v = __fmul_rn(mel[(b * nm + m) * nt + t], alpha);
    float r = rintf(v);
    r = fminf(fmaxf(r, -127.0f), 127.0f);
    out[i] = (int8_t)(int)r;
  }
}

// First index of the row maximum (torch.argmax tie rule) over int8 logits,
// one block per row. The row is read in 16-byte pieces from its first
// 16-byte boundary (the bytes before it and after the last whole piece one
// at a time); each thread visits its indices in increasing order, keeping
// the first maximum, and the block reduces keys (value + 128) << 23 |
// (2^23 - 1 - index), whose maximum is the first maximal element. When
// `step` is given, the index is also recorded in history[row][*step] (if
// *step < hist_cols).
__global__ __launch_bounds__(256) void argmax_rows_kernel(const int8_t *__restrict__ x,
                                                          int64_t cols, int64_t ld,
                                                          int64_t *__restrict__ out,
                                                          int64_t *__restrict__ history,
                                                          int64_t hist_ld, int64_t hist_cols,
                                                          const int32_t *step) {
  __shared__ int32_t sk[4];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t row = blockIdx.x;
  const int8_t *xr = x + row * ld;
  const int n = (int)cols;
  const int head = min((int)((16 - (reinterpret_cast<uintptr_t>(xr) & 15)) & 15), n);
  const int pieces = (n - head) >> 4;
  const int tail0 = head + (pieces << 4);
  int32_t best = -1000, bi = 0;
  if (tid < head) {
    best = xr[tid];
    bi = tid;
  }
  const uint4 *xa = reinterpret_cast<const uint4 *>(xr + head);
  for (int c = tid; c < pieces; c += 256) {
    const uint4 w = xa[c];
    const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int32_t v = (int32_t)(int8_t)(ws[e >> 2] >> (8 * (e & 3)));
      if (v > best) {
        best = v;
        bi = head + (c << 4) + e;
      }
    }
  }
  if (tail0 + tid < n) {
    const int32_t v = xr[tail0 + tid];
    if (v > best) {
      best = v;
      bi = tail0 + tid;
    }
  }
  int32_t key = best < -128 ? 0 : (((best + 128) << 23) | (0x7FFFFF - bi));
  key = wave_max_dpp(key);
  if (lane == 0) sk[wave] = key;
  __syncthreads();
  if (tid == 0) {
    key = max(max(sk[0], sk[1]), max(sk[2], sk[3]));
    const int64_t idx = 0x7FFFFF - (key & 0x7FFFFF);
    out[row] = idx;
    if (history) {
      const int32_t st = *step;
      if (st >= 0 && st < hist_cols) history[row * hist_ld + st] = idx;
    }
  }
}

// Greedy token choice with the reference's logit filters applied on the
// device (decoding.py:410-509 and GreedyDecoder.update, :275-296), one block
// per row. The filters only remove candidates, so the argmax runs over the
// allowed set of the int8 logits directly:
//  * point masks (SuppressTokens, plus SuppressBlank's ids on the first
//    sampled step and <|notimestamps|> under the timestamp rules) come as
//    bitmasks over the vocabulary;
//  * the timestamp rules (ApplyTimestampRules) leave the allowed set as
//    [text_lo, ts_begin) + [ts_lo, ts_hi), derived from the sampled tokens
//    history[row][0 .. *step);
//  * their last rule ("sample a timestamp if the timestamp tokens' total
//    probability exceeds every text token's") compares, in fp32 over the
//    dequantised logits, logsumexp over the allowed timestamps with the
//    largest allowed text logit (the log-softmax normaliser cancels);
//  * a sequence whose previous token is EOT keeps emitting EOT.
// With nothing allowed the result is index 0 (torch.argmax over all -inf).
struct GreedyFilter {
  const uint32_t *mask;        // suppressed at every step, or null
  const uint32_t *mask_first;  // suppressed at the first sampled step, or null
  const int64_t *prev0;        // per row: the token before the first sampled one, or null
  int32_t eot;                 // < 0: no EOT freeze and no timestamp rules
  int32_t ts_begin;            // < 0: no timestamp rules
  int32_t max_init;            // max_initial_timestamp_index, < 0: none
  float scale;                 // logit dequantisation scale (> 0)
  float *sum_logprobs;         // per row, or null: += log_softmax of the filtered logits at the token
  int32_t *eot_count;          // [hist_cols], or null: rows whose new token is EOT, per step
};

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = max(v, (uint32_t)__shfl_xor((int)v, o));
  return v;
}

__global__ __launch_bounds__(256) void greedy_filtered_kernel(const int8_t *__restrict__ x, int64_t cols,
                                                              int64_t ld, int64_t *__restrict__ out,
                                                              int64_t *__restrict__ history, int64_t hist_ld,
                                                              int64_t hist_cols, const int32_t *step,
                                                              GreedyFilter f) {
  __shared__ uint32_t s_kt[4], s_ks[4];
  __shared__ int32_t s_m[4], s_i[4], s_mx[4];
  __shared__ float s_s[4], s_sx[4];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t row = blockIdx.x;
  const int n = (int)cols;
  const int st = *step;
  const int64_t *h = history + row * hist_ld;
  const int nh = min(st, (int)hist_cols);  // sampled tokens held in the history

  // ---- allowed set ----
  int text_lo = 0, ts_b = n, ts_lo = n, ts_hi = n;
  const bool rules = f.eot >= 0 && f.ts_begin >= 0;
  if (rules) {
    ts_b = min(f.ts_begin, n);
    ts_lo = ts_b;
    const int64_t last = nh >= 1 ? h[nh - 1] : -1, pen = nh >= 2 ? h[nh - 2] : -1;
    const bool last_ts = nh >= 1 && last >= f.ts_begin;
    const bool pen_ts = nh < 2 || pen >= f.ts_begin;
    if (last_ts) {
      if (pen_ts)
        ts_hi = ts_lo;  // has to be a non-timestamp
      else
        text_lo = min(max(f.eot, 0), ts_b);  // cannot be normal text
    }
    // the last timestamp sampled so far
    int im = -1;
    for (int i = tid; i < nh; i += 256)
      if (h[i] >= f.ts_begin) im = i;
    im = wave_max_i32(im);
    if (lane == 0) s_i[wave] = im;
    __syncthreads();
    im = max(max(s_i[0], s_i[1]), max(s_i[2], s_i[3]));
    if (im >= 0) {
      const int64_t tl = h[im] + ((last_ts && !pen_ts) ? 0 : 1);  // non-decreasing, nonzero segments
      ts_lo = (int)min(max((int64_t)ts_lo, tl), (int64_t)n);
    }
    if (nh == 0) {
      text_lo = ts_b;  // the first sampled token is a timestamp
      if (f.max_init >= 0) ts_hi = (int)min((int64_t)ts_hi, (int64_t)f.ts_begin + f.max_init + 1);
    }
    ts_hi = max(ts_hi, ts_lo);
  }
  const uint32_t *mk = (st == 0 && f.mask_first) ? f.mask_first : f.mask;
  const int nw = (n + 31) >> 5;

  // ---- one pass: text argmax key, timestamp argmax key, timestamp (max, sum exp),
  // and with sum_logprobs the text tokens' (max, sum exp) ----
  const bool lps = f.sum_logprobs != nullptr;
  uint32_t kt = 0, ks = 0;
  int32_t m = -1000, mx = -1000;
  float sum = 0.f, sumx = 0.f;
  const int8_t *xr = x + row * ld;
  for (int i0 = tid * 16; i0 < n; i0 += 256 * 16) {
    uint32_t bits = 0;
    if (mk) {
      const int w = i0 >> 5, sh = i0 & 31;
      uint64_t pair = mk[w];
      if (w + 1 < nw) pair |= (uint64_t)mk[w + 1] << 32;
      bits = (uint32_t)(pair >> sh) & 0xffffu;
    }
#pragma unroll 4
    for (int e = 0; e < 16; ++e) {
      const int i = i0 + e;
      if (i >= n || ((bits >> e) & 1)) continue;
      const int32_t v = xr[i];
      const uint32_t key = ((uint32_t)(v + 129) << 23) | (uint32_t)(0x7FFFFF - i);
      if (i >= text_lo && i < ts_b) {
        kt = max(kt, key);
        if (lps) {
          if (v > mx) {
            sumx = sumx * expf((float)(mx - v) * f.scale) + 1.f;
            mx = v;
          } else {
            sumx += expf((float)(v - mx) * f.scale);
          }
        }
      } else if (i >= ts_lo && i < ts_hi) {
        ks = max(ks, key);
        if (v > m) {
          sum = sum * expf((float)(m - v) * f.scale) + 1.f;
          m = v;
        } else {
          sum += expf((float)(v - m) * f.scale);
        }
      }
    }
  }
  kt = wave_max_u32(kt);
  ks = wave_max_u32(ks);
  int32_t mw = wave_max_i32(m);
  float sw = sum * expf((float)(m - mw) * f.scale);
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) sw += __shfl_xor(sw, o);
  if (lane == 0) s_kt[wave] = kt, s_ks[wave] = ks, s_m[wave] = mw, s_s[wave] = sw;
  if (lps) {
    const int32_t mxw = wave_max_i32(mx);
    float sxw = sumx * expf((float)(mx - mxw) * f.scale);
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) sxw += __shfl_xor(sxw, o);
    if (lane == 0) s_mx[wave] = mxw, s_sx[wave] = sxw;
  }
  __syncthreads();
  if (tid == 0) {
    kt = max(max(s_kt[0], s_kt[1]), max(s_kt[2], s_kt[3]));
    ks = max(max(s_ks[0], s_ks[1]), max(s_ks[2], s_ks[3]));
    uint32_t key = max(kt, ks);
    // the timestamps' (max, sum exp) over the allowed timestamps
    const int32_t mt = max(max(s_m[0], s_m[1]), max(s_m[2], s_m[3]));
    float st_sum = 0.f;
    for (int w = 0; w < 4; ++w) st_sum += s_s[w] * expf((float)(s_m[w] - mt) * f.scale);
    bool ts_wins = false;
    if (rules && ks != 0) {
      const float lse_ts = (float)mt * f.scale + logf(st_sum);
      ts_wins = kt == 0 || lse_ts > (float)((int32_t)(kt >> 23) - 129) * f.scale;
      if (ts_wins) key = ks;
    }
    int64_t idx = key == 0 ? 0 : (int64_t)(0x7FFFFF - (key & 0x7FFFFF));
    bool after_eot = false;
    if (f.eot >= 0) {
      const int64_t prev = nh >= 1 ? h[nh - 1] : (f.prev0 ? f.prev0[row] : -1);
      after_eot = prev == f.eot;
    }
    if (lps) {
      // log_softmax of the filtered logits at the chosen token: the chosen
      // value is the maximum of the allowed set, which is the timestamps alone
      // when they win (the text logits are then -inf) and text + timestamps
      // otherwise; nothing allowed gives NaN, as log_softmax over all -inf
      float lp;
      if (key == 0) {
        lp = __builtin_nanf("");
      } else if (ts_wins || kt == 0) {
        lp = -logf(st_sum);
      } else {
        const int32_t mxt = max(max(s_mx[0], s_mx[1]), max(s_mx[2], s_mx[3]));
        float sx = 0.f;
        for (int w = 0; w < 4; ++w) sx += s_sx[w] * expf((float)(s_mx[w] - mxt) * f.scale);
        const int32_t top = (int32_t)(key >> 23) - 129;  // the chosen value
        float total = sx * expf((float)(mxt - top) * f.scale);
        if (ks != 0) total += st_sum * expf((float)(mt - top) * f.scale);
        lp = -logf(total);
      }
      // the reference adds lp * (previous token != EOT)
      f.sum_logprobs[row] += after_eot ? lp * 0.f : lp;
    }
    if (after_eot) idx = f.eot;
    out[row] = idx;
    if (st >= 0 && st < hist_cols) {
      history[row * hist_ld + st] = idx;
      if (f.eot_count && f.eot >= 0 && idx == f.eot) atomicAdd(f.eot_count + st, 1);
    }
  }
}

// The sum of e[x + 128] over the int8 values x of one row (NT threads, the
// row read in 16-byte pieces from its first 16-byte boundary), in float32.
template <int NT = 256>
__device__ __forceinline__ float row_table_sum(const int8_t *xr, int n, const float *e) {
  const int tid = threadIdx.x;
  const int head = min((int)((16 - (reinterpret_cast<uintptr_t>(xr) & 15)) & 15), n);
  const int pieces = (n - head) >> 4;
  const int tail0 = head + (pieces << 4);
  float s = 0.f;
  if (tid < head) s += e[xr[tid] + 128];
  const uint4 *xa = reinterpret_cast<const uint4 *>(xr + head);
  for (int c = tid; c < pieces; c += NT) {
    const uint4 w = xa[c];
    const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int q = 0; q < 16; ++q) s += e[(int32_t)(int8_t)(ws[q >> 2] >> (8 * (q & 3))) + 128];
  }
  if (tail0 + tid < n) s += e[xr[tail0 + tid] + 128];
  return s;
}

// Block sum of NT threads' values: wave sums, then the waves' sums added in
// adjacent pairs ((w0 + w1) + (w2 + w3), ...).
template <int NT = 256>
__device__ __forceinline__ float block_sum_f32(float v, float *sh) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
  const int tid = threadIdx.x;
  __syncthreads();
  if ((tid & 63) == 0) sh[tid >> 6] = v;
  __syncthreads();
  float t[NT / 64];
#pragma unroll
  for (int w = 0; w < NT / 64; ++w) t[w] = sh[w];
#pragma unroll
  for (int n = NT / 128; n >= 1; n >>= 1)
#pragma unroll
    for (int i = 0; i < n; ++i) t[i] = t[2 * i] + t[2 * i + 1];
  return t[0];
}

// One step of GreedyDecoder.update (decoding.py:280-296) at temperature 0,
// one block per row:
//  * next token = first index of the row maximum of the int8 logits, from the
//    classifier's per-32-column-tile maxima (amax, tiles per row) or, without
//    them, from the logits row itself;
//  * sum_logprobs[row] += log_softmax(logits * scale)[next], added only when
//    the previous token is not EOT (:287-289): for the row maximum v that is
//    -log(sum_i exp((x_i - v) * scale)), the sum taken through a 256-entry
//    table of exp((x - v) * scale) over the int8 values x;
//  * a row whose previous token is EOT emits EOT (:291); the number of rows
//    whose new token is EOT is added to eot_count[*step] (completed = that
//    count equals the batch, :293);
//  * history[row][*step] = next_tokens[row] = the token; then the last block to
//    finish advances *step by 1 and *pos by pos_inc (every block has read
//    *step by then: each one's arrival on `arrive` comes after its read).
struct GreedyUpdate {
  const uint16_t *amax = nullptr;
  int64_t tiles = 0;
  const int8_t *logits = nullptr;
  int64_t ld = 0;
  int cols = 0;
  int64_t *next = nullptr;
  int64_t *history = nullptr;
  int64_t hist_ld = 0, hist_cols = 0;
  int32_t *step = nullptr, *pos = nullptr;
  int32_t pos_inc = 0;
  int32_t eot = -1;
  const int64_t *prev0 = nullptr;
  float *sum_logprobs = nullptr;
  float scale = 1.f;
  int32_t *eot_count = nullptr;
  uint32_t *arrive = nullptr;
};

// 1024 threads per row: the row's 51865 table lookups (Whisper) spread over
// four waves per SIMD rather than one
constexpr int GU_NT = 1024;

__global__ __launch_bounds__(GU_NT) void greedy_update_kernel(GreedyUpdate p) {
  constexpr int NW = GU_NT / 64;
  __shared__ int32_t s_st;
  __shared__ uint32_t s_k[NW];
  __shared__ float s_f[NW];
  __shared__ float s_e[256];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t row = blockIdx.x;
  if (tid == 0) s_st = *p.step;
  // first maximum: key (v + 128) << 23 | (2^23 - 1 - index)
  uint32_t key = 0;
  if (p.amax) {
    const uint16_t *ar = p.amax + row * p.tiles;
    for (int64_t t = tid; t < p.tiles; t += GU_NT) {
      const uint32_t q = ar[t];
      if (q) {
        const uint32_t i = (uint32_t)t * 32u + (31u - (q & 31u));
        key = max(key, ((q >> 5) << 23) | (0x7FFFFFu - i));
      }
    }
  } else {
    const int8_t *xr = p.logits + row * p.ld;
    for (int i = tid; i < p.cols; i += GU_NT)
      key = max(key, ((uint32_t)(xr[i] + 128) << 23) | (uint32_t)(0x7FFFFF - i));
  }
  key = (uint32_t)wave_max_dpp((int32_t)key);  // keys < 2^31
  if (lane == 0) s_k[wave] = key;
  __syncthreads();  // s_st, s_k
  key = s_k[0];
#pragma unroll
  for (int w = 1; w < NW; ++w) key = max(key, s_k[w]);
  const int st = s_st;
  const int32_t vmax = (int32_t)(key >> 23) - 128;
  const int64_t idx = (int64_t)(0x7FFFFF - (key & 0x7FFFFF));
  float lp = 0.f;
  if (p.sum_logprobs) {
    if (tid < 256) s_e[tid] = expf((float)(tid - 128 - vmax) * p.scale);
    __syncthreads();
    lp = -logf(block_sum_f32<GU_NT>(row_table_sum<GU_NT>(p.logits + row * p.ld, p.cols, s_e), s_f));
  }
  if (tid == 0) {
    const int64_t prev = st >= 1 ? (st - 1 < p.hist_cols ? p.history[row * p.hist_ld + st - 1] : -1)
                                 : (p.prev0 ? p.prev0[row] : -1);
    const bool after_eot = p.eot >= 0 && prev == p.eot;
    const int64_t tok = after_eot ? p.eot : idx;
    p.next[row] = tok;
    if (st >= 0 && st < p.hist_cols) {
      p.history[row * p.hist_ld + st] = tok;
      if (p.eot_count && p.eot >= 0 && tok == p.eot) atomicAdd(p.eot_count + st, 1);
    }
    // the reference adds lp * (previous token != EOT)
    if (p.sum_logprobs) p.sum_logprobs[row] += after_eot ? lp * 0.f : lp;
    // this block has read *step (s_st, above a barrier): arrive
    if (atomicAdd(p.arrive, 1u) == gridDim.x - 1) {
      *p.step = st + 1;
      *p.pos += p.pos_inc;
      *p.arrive = 0;
    }
  }
}

// softmax(logits * scale)[token] of each row in float32 (the no-speech
// probability at the start-of-transcript position, decoding.py:690-695):
// exp((x_token - v) * scale) / sum_i exp((x_i - v) * scale), v the row maximum.
__global__ __launch_bounds__(256) void token_prob_kernel(const int8_t *__restrict__ x, int64_t ld, int cols,
                                                         int64_t token, float scale, float *__restrict__ out) {
  __shared__ int32_t s_m[4];
  __shared__ float s_f[4];
  __shared__ float s_e[256];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int8_t *xr = x + blockIdx.x * ld;
  int32_t m = -128;
  for (int i = tid; i < cols; i += 256) m = max(m, (int32_t)xr[i]);
  m = wave_max_i32(m);
  if (lane == 0) s_m[wave] = m;
  __syncthreads();
  m = max(max(s_m[0], s_m[1]), max(s_m[2], s_m[3]));
  s_e[tid] = expf((float)(tid - 128 - m) * scale);
  __syncthreads();
  const float sum = block_sum_f32(row_table_sum(xr, cols, s_e), s_f);
  if (tid == 0) out[blockIdx.x] = s_e[xr[token] + 128] / sum;
}

// Greedy step bookkeeping after argmax_rows wrote next[]: record the tokens
// in column *step of the history and advance the device-side counters.
__global__ void greedy_advance_kernel(int32_t *step, int32_t *pos, int32_t pos_inc) {
  if (threadIdx.x == 0) {
    *step += 1;
    *pos += pos_inc;
  }
}

// Per-head transpose of a [B, T, H*D] operand slice into a V cache: with
// p = t_off + t, dst[b*dst_sb + h*dst_sh + d*dst_sd + (p/4)*dst_sq + p%4] =
// src[b*src_sb + t*src_st + h*D + d] (dst_sq = 4: V^T rows [b][h][d][p]).
// Tiles of 64 positions x 64 feature columns go through LDS so that both the
// reads (along features) and the V^T writes (along positions) are contiguous.
__global__ __launch_bounds__(256) void transpose_heads_kernel(
    const int8_t *__restrict__ src, int64_t src_sb, int64_t src_st, int8_t *__restrict__ dst,
    int64_t dst_sb, int64_t dst_sh, int64_t dst_sd, int64_t dst_sq, int64_t t_off, int64_t T, int64_t H,
    int64_t D) {
  __shared__ int8_t tile[64][65];
  const int64_t b = blockIdx.z;
  const int64_t t0 = (int64_t)blockIdx.x * 64;
  const int64_t c0 = (int64_t)blockIdx.y * 64;  // feature column h*D + d
  const int64_t C = H * D;
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  for (int r = ty; r < 64; r += 4) {
    const int64_t t = t0 + r, c = c0 + tx;
    tile[r][tx] = (t < T && c < C) ? src[b * src_sb + t * src_st + c] : (int8_t)0;
  }
  __syncthreads();
  for (int r = ty; r < 64; r += 4) {
    const int64_t c = c0 + r, t = t0 + tx;
    if (t < T && c < C) {
      const int64_t h = c / D, d = c % D;
      const int64_t p = t_off + t;  // cache position
      dst[b * dst_sb + h * dst_sh + d * dst_sd + (p >> 2) * dst_sq + (p & 3)] = tile[tx][r];
    }
  }
}

// transpose_heads_kernel with 16-byte accesses (row strides, offsets and
// H * D multiples of 16): a 64 x 64 tile is read as 16-byte row pieces into
// LDS, and each thread writes 16 consecutive positions t of one feature
// column (a byte gather down the tile); positions past T are not written.
__global__ __launch_bounds__(256) void transpose_heads16_kernel(
    const int8_t *__restrict__ src, int64_t src_sb, int64_t src_st, int8_t *__restrict__ dst,
    int64_t dst_sb, int64_t dst_sh, int64_t dst_sd, int64_t t_off, int64_t T, int64_t H,
    int64_t D) {
  __shared__ __attribute__((aligned(16))) uint8_t tile[64][64 + 16];
  const int64_t b = blockIdx.z;
  const int64_t t0 = (int64_t)blockIdx.x * 64;
  const int64_t c0 = (int64_t)blockIdx.y * 64;  // feature column h*D + d
  const int64_t C = H * D;
  const int tid = threadIdx.x, r = tid >> 2, q = (tid & 3) * 16;
  uint4 v = make_uint4(0, 0, 0, 0);
  if (t0 + r < T && c0 + q < C) v = *reinterpret_cast<const uint4 *>(src + b * src_sb + (t0 + r) * src_st + c0 + q);
  *reinterpret_cast<uint4 *>(&tile[r][q]) = v;
  __syncthreads();
  const int64_t c = c0 + r, t = t0 + q;
  if (c >= C || t >= T) return;
  uint32_t w[4];
#pragma unroll
  for (int k = 0; k < 4; ++k)
    w[k] = (uint32_t)tile[q + 4 * k][r] | ((uint32_t)tile[q + 4 * k + 1][r] << 8) |
           ((uint32_t)tile[q + 4 * k + 2][r] << 16) | ((uint32_t)tile[q + 4 * k + 3][r] << 24);
  const int32_t h = (int32_t)c / (int32_t)D, d = (int32_t)c - h * (int32_t)D;
  int8_t *o = dst + b * dst_sb + (int64_t)h * dst_sh + (int64_t)d * dst_sd + t_off + t;
  if (t + 16 <= T) {
    *reinterpret_cast<uint4 *>(o) = make_uint4(w[0], w[1], w[2], w[3]);
  } else {
    for (int i = 0; i < 16 && t + i < T; ++i) o[i] = (int8_t)(w[i >> 2] >> (8 * (i & 3)));
  }
}

// Per-head gather of a [B, T, H*D] operand slice into a [B, H, T_cap, D]
// cache at positions [t_off, t_off + T): dst[b*dst_sb + h*dst_sh + (t_off+t)*dst_st + d]
// = src[b*src_sb + t*src_st + h*D + d], 16 bytes per thread (D % 16 == 0).
__global__ void gather_heads_kernel(const int8_t *__restrict__ src, int64_t src_sb, int64_t src_st,
                                    int8_t *__restrict__ dst, int64_t dst_sb, int64_t dst_sh,
                                    int64_t dst_st, int64_t t_off, int64_t B, int64_t T, int64_t H,
                                    int64_t D) {
  const int64_t cpr = H * D / 16;  // 16-byte chunks per source row
  const int64_t total = B * T * cpr;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    const int64_t c = i % cpr, bt = i / cpr;
    const int64_t t = bt % T, b = bt / T;
    const int64_t h = (c * 16) / D, d = (c * 16) % D;
    *reinterpret_cast<uint4 *>(dst + b * dst_sb + h * dst_sh + (t_off + t) * dst_st + d) =
        *reinterpret_cast<const uint4 *>(src + b * src_sb + t * src_st + c * 16);
  }
}

// Copy rows of a [B, T, ld] operand slice (C features) into a [B, Tmax, C]
// cache at positions [t_off, t_off + T).
__global__ void copy_rows_kernel(const int8_t *__restrict__ src, int64_t src_sb, int64_t src_st,
                                 int8_t *__restrict__ dst, int64_t dst_sb, int64_t dst_st,
                                 int64_t t_off, int64_t B, int64_t T, int64_t C) {
  const int64_t total = B * T * C;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    const int64_t c = i % C, bt = i / C;
    const int64_t t = bt % T, b = bt / T;
    dst[b * dst_sb + (t_off + t) * dst_st + c] = src[b * src_sb + t * src_st + c];
  }
}

int grid_for(int64_t n, int threads) {
  int64_t b = (n + threads - 1) / threads;
  if (b > 65536) b = 65536;
  return (int)(b < 1 ? 1 : b);
}

}  // namespace

// row counts up to which each row gets a block of its own
constexpr int64_t kLnRowBlockMaxRows = 2048;

// Blocks of layernorm32_kernel resident on the whole device at once (its
// persistent grid): CUs x blocks per CU at the kernel's register use.
int64_t ln_persistent_blocks() {
  static const int64_t blocks = [] {
    int dev = 0, cus = 0, per_cu = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, layernorm32_kernel, 256, 0) != hipSuccess ||
        cus <= 0 || per_cu <= 0) {
      (void)hipGetLastError();
      return (int64_t)256 * 4;
    }
    return (int64_t)cus * per_cu;
  }();
  return blocks;
}

int layernorm_width_code(int64_t h) {
  switch (h) {
    case 384: return 0;
    case 512: return 1;
    case 768: return 2;
    case 1024: return 3;
    case 1280: return 4;
    default: return -1;
  }
}

int launch_layernorm32(const int16_t *x, const int8_t *gamma, const int32_t *beta, uint8_t ln_m,
                       int8_t ln_s, uint32_t out_m, int8_t out_s, uint32_t rsqrt_off, int8_t *out,
                       int64_t rows, int64_t hidden, hipStream_t s, bool out_frag, const FragPrefetch *pf) {
  const int code = layernorm_width_code(hidden);
  if (code < 0) return fail("unsupported LayerNorm hidden size: " + std::to_string(hidden));
  if (rows == 0) return 0;
  if (out_frag && rows > kSkinnyMaxRows) return fail("a fragment-major LayerNorm output takes at most 128 rows");
  if (rows <= kLnRowBlockMaxRows) {
    // few rows (a decode step): a block of 256 threads per row
    FragPrefetch pfl = pf ? *pf : FragPrefetch();
    frag_prefetch_launch(pfl, rows, 256);
    hipLaunchKernelGGL(layernorm32_row_kernel, dim3((unsigned)rows), dim3(256), 0, s, x, gamma, beta,
                       (uint32_t)ln_m, (int32_t)ln_s, out_m, (int32_t)out_s, rsqrt_off, out, (int)hidden,
                       code, out_frag ? frag_kpad(hidden) : (int64_t)0, pfl);
    return check_launch("layernorm32_row_kernel");
  }
  // one row per wave at a time, four waves per block; persistent waves, as
  // many blocks as the device holds at once
  const int64_t blocks = std::min<int64_t>((rows + 3) / 4, ln_persistent_blocks());
  hipLaunchKernelGGL(layernorm32_kernel, dim3((unsigned)blocks), dim3(256), 0, s, x, gamma, beta,
                     (uint32_t)ln_m, (int32_t)ln_s, out_m, (int32_t)out_s, rsqrt_off, out, rows,
                     (int)hidden, code);
  return check_launch("layernorm32_kernel");
}

int launch_rsqrt(const int32_t *x, int32_t *out, int64_t n, uint32_t off, hipStream_t s) {
  if (n == 0) return 0;
  hipLaunchKernelGGL(rsqrt_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, x, out, n,
                     off);
  return check_launch("rsqrt_kernel");
}

int launch_gelu(const int8_t *x, const uint8_t *lut, const uint8_t *luti_m, const int8_t *luti_s,
                const uint8_t *luto_m, const int8_t *luto_s, int8_t *out, int64_t numel,
                int64_t channels, int luti_pc, int luto_pc, hipStream_t s) {
  if (numel == 0) return 0;
  const uintptr_t al = reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(out) |
                       (luti_pc ? reinterpret_cast<uintptr_t>(luti_m) | reinterpret_cast<uintptr_t>(luti_s) : 0) |
                       (luto_pc ? reinterpret_cast<uintptr_t>(luto_m) | reinterpret_cast<uintptr_t>(luto_s) : 0);
  if (channels % 16 == 0 && numel % channels == 0 && (al & 15) == 0 && channels / 16 <= 0xffffffffLL) {
    const int64_t pieces = numel / 16;
    hipLaunchKernelGGL(gelu16_kernel, dim3(grid_for(pieces, 256)), dim3(256), 0, s, x, lut, luti_m, luti_s,
                       luto_m, luto_s, out, pieces, (uint32_t)(channels / 16), luti_pc, luto_pc);
    return check_launch("gelu16_kernel");
  }
  hipLaunchKernelGGL(gelu_kernel, dim3(grid_for(numel, 256)), dim3(256), 0, s, x, lut, luti_m,
                     luti_s, luto_m, luto_s, out, numel, channels, luti_pc, luto_pc);
  return check_launch("gelu_kernel");
}

int launch_residual15(const int32_t *br, const int16_t *res, uint16_t m, int16_t *out, int64_t n,
                      hipStream_t s) {
  if (n == 0) return 0;
  hipLaunchKernelGGL(residual15_kernel, dim3(grid_for(n, 256)), dim3(256), 0, s, br, res,
                     (uint32_t)m, out, n);
  return check_launch("residual15_kernel");
}

int launch_add_requant15(const int8_t *x, const int64_t *tokens, const int8_t *addend,
                         const uint16_t *mult, const int8_t *shift, int16_t *out, int64_t batch,
                         int64_t positions, int64_t channels, int mpc, int spc, hipStream_t s,
                         const int32_t *pos, int64_t addend_rows) {
  const int64_t total = batch * positions * channels;
  if (total == 0) return 0;
  const uintptr_t al = reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(addend) |
                       reinterpret_cast<uintptr_t>(out) | (mpc ? reinterpret_cast<uintptr_t>(mult) : 0) |
                       (spc ? reinterpret_cast<uintptr_t>(shift) : 0);
  if (channels % 16 == 0 && (al & 15) == 0 && channels / 16 <= 0xffffffffLL) {
    const int64_t pieces = total / 16;
    hipLaunchKernelGGL(add_requant15_16_kernel, dim3(grid_for(pieces, 256)), dim3(256), 0, s, x, tokens, addend,
                       mult, shift, out, positions, channels, pieces, mpc, spc, pos, addend_rows);
    return check_launch("add_requant15_16_kernel");
  }
  hipLaunchKernelGGL(add_requant15_kernel, dim3(grid_for(total, 256)), dim3(256), 0, s, x, tokens,
                     addend, mult, shift, out, positions, channels, total, mpc, spc, pos, addend_rows);
  return check_launch("add_requant15_kernel");
}

int launch_quantize_mel(const float *mel, float alpha, int8_t *out, int64_t b, int64_t m,
                        int64_t t, hipStream_t s) {
  const int64_t total = b * m * t;
  if (total == 0) return 0;
  hipLaunchKernelGGL(quantize_mel_kernel, dim3(grid_for(total, 256)), dim3(256), 0, s, mel, alpha,
                     out, b, m, t);
  return check_launch("quantize_mel_kernel");
}

int launch_transpose_heads(const int8_t *src, int64_t src_sb, int64_t src_st, int8_t *dst,
                           int64_t dst_sb, int64_t dst_sh, int64_t dst_sd, int64_t dst_sq, int64_t t_off,
                           int64_t B, int64_t T, int64_t H, int64_t D, hipStream_t s) {
  if (B * T * H * D == 0) return 0;
  const dim3 grid((unsigned)((T + 63) / 64), (unsigned)((H * D + 63) / 64), (unsigned)B);
  const uintptr_t al = reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst) | (uintptr_t)src_sb |
                       (uintptr_t)src_st | (uintptr_t)dst_sb | (uintptr_t)dst_sh | (uintptr_t)dst_sd |
                       (uintptr_t)t_off | (uintptr_t)(H * D);
  if (dst_sq == 4 && (al & 15) == 0 && H * D <= 0x7fffffff) {
    hipLaunchKernelGGL(transpose_heads16_kernel, grid, dim3(256), 0, s, src, src_sb, src_st, dst, dst_sb, dst_sh,
                       dst_sd, t_off, T, H, D);
    return check_launch("transpose_heads16_kernel");
  }
  hipLaunchKernelGGL(transpose_heads_kernel, grid, dim3(256), 0, s, src, src_sb, src_st, dst,
                     dst_sb, dst_sh, dst_sd, dst_sq, t_off, T, H, D);
  return check_launch("transpose_heads_kernel");
}

int launch_gather_heads(const int8_t *src, int64_t src_sb, int64_t src_st, int8_t *dst,
                        int64_t dst_sb, int64_t dst_sh, int64_t dst_st, int64_t t_off, int64_t B,
                        int64_t T, int64_t H, int64_t D, hipStream_t s) {
  const int64_t total = B * T * H * D / 16;
  if (total == 0) return 0;
  hipLaunchKernelGGL(gather_heads_kernel, dim3(grid_for(total, 256)), dim3(256), 0, s, src, src_sb,
                     src_st, dst, dst_sb, dst_sh, dst_st, t_off, B, T, H, D);
  return check_launch("gather_heads_kernel");
}

int launch_copy_rows(const int8_t *src, int64_t src_sb, int64_t src_st, int8_t *dst,
                     int64_t dst_sb, int64_t dst_st, int64_t t_off, int64_t B, int64_t T,
                     int64_t C, hipStream_t s) {
  const int64_t total = B * T * C;
  if (total == 0) return 0;
  hipLaunchKernelGGL(copy_rows_kernel, dim3(grid_for(total, 256)), dim3(256), 0, s, src, src_sb,
                     src_st, dst, dst_sb, dst_st, t_off, B, T, C);
  return check_launch("copy_rows_kernel");
}

int launch_greedy_step(const int8_t *logits, int64_t rows, int64_t cols, int64_t ld, int64_t *next,
                       int64_t *history, int64_t hist_ld, int64_t hist_cols, int32_t *step,
                       int32_t *pos, int32_t pos_inc, hipStream_t s) {
  if (rows > 0) {
    hipLaunchKernelGGL(argmax_rows_kernel, dim3((unsigned)rows), dim3(256), 0, s, logits, cols, ld, next,
                       history, hist_ld, hist_cols, step);
    int rc = check_launch("argmax_rows_kernel");
    if (rc) return rc;
  }
  hipLaunchKernelGGL(greedy_advance_kernel, dim3(1), dim3(64), 0, s, step, pos, pos_inc);
  return check_launch("greedy_advance_kernel");
}

int launch_greedy_step_filtered(const int8_t *logits, int64_t rows, int64_t cols, int64_t ld, int64_t *next,
                                int64_t *history, int64_t hist_ld, int64_t hist_cols, int32_t *step,
                                int32_t *pos, int32_t pos_inc, const uint32_t *mask, const uint32_t *mask_first,
                                const int64_t *prev0, int32_t eot, int32_t ts_begin, int32_t max_init,
                                float scale, float *sum_logprobs, int32_t *eot_count, hipStream_t s) {
  if (rows > 0) {
    const GreedyFilter f{mask, mask_first, prev0, eot, ts_begin, max_init, scale, sum_logprobs, eot_count};
    hipLaunchKernelGGL(greedy_filtered_kernel, dim3((unsigned)rows), dim3(256), 0, s, logits, cols, ld, next,
                       history, hist_ld, hist_cols, step, f);
    int rc = check_launch("greedy_filtered_kernel");
    if (rc) return rc;
  }
  hipLaunchKernelGGL(greedy_advance_kernel, dim3(1), dim3(64), 0, s, step, pos, pos_inc);
  return check_launch("greedy_advance_kernel");
}

int launch_greedy_update(const uint16_t *amax, int64_t tiles, const int8_t *logits, int64_t ld, int64_t rows,
                         int64_t cols, int64_t *next, int64_t *history, int64_t hist_ld, int64_t hist_cols,
                         int32_t *step, int32_t *pos, int32_t pos_inc, int32_t eot, const int64_t *prev0,
                         float *sum_logprobs, float scale, int32_t *eot_count, uint32_t *arrive, hipStream_t s) {
  GreedyUpdate p;
  p.amax = amax;
  p.tiles = tiles;
  p.logits = logits;
  p.ld = ld;
  p.cols = (int)cols;
  p.next = next;
  p.history = history;
  p.hist_ld = hist_ld;
  p.hist_cols = hist_cols;
  p.step = step;
  p.pos = pos;
  p.pos_inc = pos_inc;
  p.eot = eot;
  p.prev0 = prev0;
  p.sum_logprobs = sum_logprobs;
  p.scale = scale;
  p.eot_count = eot_count;
  p.arrive = arrive;
  hipLaunchKernelGGL(greedy_update_kernel, dim3((unsigned)rows), dim3(GU_NT), 0, s, p);
  return check_launch("greedy_update_kernel");
}

int launch_token_prob(const int8_t *logits, int64_t rows, int64_t cols, int64_t ld, int64_t token, float scale,
                      float *out, hipStream_t s) {
  if (rows == 0) return 0;
  hipLaunchKernelGGL(token_prob_kernel, dim3((unsigned)rows), dim3(256), 0, s, logits, ld, (int)cols, token, scale,
                     out);
  return check_launch("token_prob_kernel");
}

int launch_argmax_rows(const int8_t *x, int64_t rows, int64_t cols, int64_t ld, int64_t *out,
                       hipStream_t s) {
  if (rows == 0) return 0;
  hipLaunchKernelGGL(argmax_rows_kernel, dim3((unsigned)rows), dim3(256), 0, s, x, cols, ld, out,
                     (int64_t *)nullptr, (int64_t)0, (int64_t)0, (const int32_t *)nullptr);
  return check_launch("argmax_rows_kernel");
}

}  // namespace iw
