// Integer attention on gfx950.
//
// Op-level kernels, one per reference op (attention/attention_scalar.cpp):
//   qk_requant_rowmax  :216-334   QK^T, requant to int16, masked row max + 1
//   shift_exp          :388-568   shift-exponential to uint8 P and int32 row sums
//   pv_norm_requant    :676-814   P.V, FISR normalisation, AV requant, [B,Tq,H*D]
//
// Fused kernels used by the layer API (bit-identical to the three ops above):
//   attn_prefill  - MFMA kernel for long query blocks (encoder self-attention,
//                   decoder prompt). Two passes over K: pass 1 takes the row max
//                   of the raw int32 scores (the requant is monotone, so
//                   requant(max) == max(requant)); pass 2 recomputes the scores,
//                   maps them to P through a per-launch shift-exp table in LDS,
//                   and accumulates P.V on MFMA. The int16 score and uint8 P
//                   tensors are never written to memory.
//   attn_decode   - streaming kernel for a few query rows over a KV cache
//                   (decoder self- and cross-attention).
#include "iw_common.hpp"
#include "iw_gemm.hpp"
#include "iw_kernels.hpp"

#include <type_traits>

namespace iw {

namespace {

// Output element (b, c) of the decode kernels over the caches: row-major at
// b * o_sb + c, or the fragment-major image of [B][H*D] feeding the
// out-projection GEMM.
__device__ __forceinline__ int64_t decode_out_index(const AttnArgs &a, int64_t b, int c) {
  return a.o_frag_kp ? frag_offset(b, c, a.o_frag_kp) : b * a.o_sb + c;
}

__device__ __forceinline__ int32_t qk_requant16(int32_t acc, uint32_t m, uint32_t s) {
  // (int32)(acc * m) modulo 2^32, Rshift, saturate to int16
  return clampi(rshift((int32_t)((uint32_t)acc * m), s), -32768, 32767);
}

// ------------------------------------------------------------------------
// Op-level kernels
// ------------------------------------------------------------------------

// One wave per query row; lanes stride over keys.
__global__ __launch_bounds__(256) void qk_requant_rowmax_kernel(
    const int8_t *__restrict__ q, const int8_t *__restrict__ k, const uint8_t *__restrict__ mask,
    int16_t *__restrict__ qk, int16_t *__restrict__ rmp1, int64_t rows, int64_t tq, int64_t tk,
    int64_t dim, uint32_t m, uint32_t s) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int64_t bh = row / tq, i = row % tq;
  const int8_t *qr = q + row * dim;
  const int8_t *kb = k + bh * tk * dim;
  int16_t *o = qk + row * tk;
  int32_t mx = -32768;
  for (int64_t j = lane; j < tk; j += 64) {
    if (mask && mask[i * tk + j]) {
      o[j] = -32768;
      continue;
    }
    const int8_t *kr = kb + j * dim;
    int32_t acc = 0;
    for (int64_t d = 0; d < dim; ++d) acc += (int32_t)qr[d] * (int32_t)kr[d];
    const int32_t h = qk_requant16(acc, m, s);
    o[j] = (int16_t)h;
    mx = max(mx, h);
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) mx = max(mx, __shfl_xor(mx, off));
  if (lane == 0) rmp1[row] = (int16_t)(uint16_t)((uint32_t)(uint16_t)(int16_t)mx + 1u);
}

__global__ __launch_bounds__(256) void shift_exp_kernel(const int16_t *__restrict__ qk,
                                                        const int16_t *__restrict__ rmp1,
                                                        const uint8_t *__restrict__ mask,
                                                        uint8_t *__restrict__ p,
                                                        int32_t *__restrict__ row_sum,
                                                        int64_t rows, int64_t tq, int64_t tk,
                                                        int32_t f) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int64_t i = row % tq;
  const int16_t xm = rmp1[row];
  uint32_t sum = 0;
  for (int64_t j = lane; j < tk; j += 64) {
    uint32_t v = 0;
    if (!(mask && mask[i * tk + j])) {
      const int32_t xs = (int16_t)(uint16_t)((uint32_t)(uint16_t)qk[row * tk + j] - (uint32_t)(uint16_t)xm);
      v = shift_exp_one(xs, f);
    }
    p[row * tk + j] = (uint8_t)v;
    sum += v;
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) sum += (uint32_t)__shfl_xor((int)sum, off);
  if (lane == 0) row_sum[row] = (int32_t)sum;
}

// One block per query row; each wave owns a subset of the head dims.
__global__ __launch_bounds__(256) void pv_norm_requant_kernel(
    const uint8_t *__restrict__ p, const int8_t *__restrict__ v, const int32_t *__restrict__ rsum,
    uint32_t av_m, uint32_t av_s, uint32_t off, int8_t *__restrict__ out, int64_t heads,
    int64_t tq, int64_t tk, int64_t dim) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int64_t row = blockIdx.x;  // (b*H + h)*Tq + i
  const int64_t bh = row / tq, i = row % tq;
  const int64_t b = bh / heads, h = bh % heads;
  const uint8_t *pr = p + row * tk;
  const int32_t inv = fisr(rsum[row], off);
  for (int64_t d = wave; d < dim; d += 4) {
    const int8_t *vr = v + (bh * dim + d) * tk;
    uint32_t acc = 0;
    for (int64_t j = lane; j < tk; j += 64) acc += (uint32_t)((int32_t)pr[j] * (int32_t)vr[j]);
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) acc += (uint32_t)__shfl_xor((int)acc, o);
    if (lane == 0) {
      int32_t y = rshift((int32_t)(acc * (uint32_t)inv), off);
      y = rshift((int32_t)((uint32_t)y * (uint32_t)inv), off);
      y = rshift((int32_t)((uint32_t)y * av_m), av_s);
      out[(b * tq + i) * heads * dim + h * dim + d] = (int8_t)clampi(y, -127, 127);
    }
  }
}

// Shift-exp table for one frac_bits value: lut[i] = P(x_sub = -i) for
// i in [0, 32767]. Every x_sub <= -32767 and every x_sub > 0 maps to 0, so an
// index min((uint16)(rmp1 - qk), 32767) covers all int16 inputs.
__global__ void shift_exp_lut_kernel(uint8_t *lut, int32_t f) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < IW_SEXP_LUT) lut[i] = (uint8_t)shift_exp_one(-i, f);
}

// ------------------------------------------------------------------------
// Fused prefill attention (MFMA)
// ------------------------------------------------------------------------
//
// Block: 4 waves x 32 query rows of one (batch, head); persistent over tiles.
// Scores are computed transposed, S^T = K . Q^T, with MFMA 32x32x32: lane l
// owns query l % 32 and, for register r, the key held in LDS row
// (r/4)*8 + (l/32)*4 + r%4 of the 32-key sub-block. Keys are stored in LDS in
// the order that puts key 16*(l/32) + r in that row, so each lane holds 16
// consecutive keys of its query — exactly the A-operand layout of the P.V
// MFMA, whose B operand is then one 16-byte read of V^T from LDS.

constexpr int PF_KC = 64;  // keys per LDS stage

// Median of three signed ints: clamp of x to [lo, hi] for lo <= hi, in one
// instruction where the bounds are not compile-time constants.
__device__ __forceinline__ int32_t med3i(int32_t x, int32_t lo, int32_t hi) {
  int32_t r;
  asm("v_med3_i32 %0, %1, %2, %3" : "=v"(r) : "v"(x), "v"(lo), "v"(hi));
  return r;
}

__device__ __forceinline__ int key_row(int kk) {
  // LDS row of key kk (0..31) inside a 32-key sub-block
  const int g = kk >> 4, r = kk & 15;
  return (r >> 2) * 8 + g * 4 + (r & 3);
}

// DF: the head dim is exactly 32 KS, so whole-chunk K / V^T copies need no
// bounds tests.
template <int KS, bool HAS_MASK, bool DF>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(KS <= 2 ? 4 : 1)))
void attn_prefill_kernel(AttnArgs a) {
  constexpr int DP = KS * 32;           // padded head dim
  // K and V^T rows of 4 chunks of 16 bytes (head_dim 64) are unpadded, with
  // chunk c of row r stored at position c ^ ((r >> 2) & 3): the 16 rows one
  // 16-lane pass of a fragment read touches then cover the 64 banks once.
  // That keeps a block at 40 KB of LDS (the table, one K and one V^T stage),
  // four blocks per CU. Other head sizes pad each row by 16 bytes instead.
  constexpr bool SWZ = KS == 2;
  constexpr int KLD = SWZ ? DP : DP + 16;           // sK row stride
  constexpr int VLD = SWZ ? PF_KC : PF_KC + 16;     // sVt row stride
  auto kpos = [](int row, int chunk) { return SWZ ? (chunk ^ ((row >> 2) & 3)) : chunk; };
  __shared__ __attribute__((aligned(16))) uint8_t sLut[IW_SEXP_LUT];
  __shared__ __attribute__((aligned(16))) int8_t sK[PF_KC * KLD];
  __shared__ __attribute__((aligned(16))) int8_t sVt[DP * VLD];
  // the per-row reciprocal square roots of a tile go to sK once its last
  // chunk is consumed
  int32_t(*const sInv)[32] = reinterpret_cast<int32_t(*)[32]>(sK);
  static_assert(PF_KC * KLD >= 4 * 32 * 4, "sK holds the tile's 128 row factors");

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 5, ql = lane & 31;

  for (int i = tid; i < IW_SEXP_LUT / 16; i += 256)
    reinterpret_cast<uint4 *>(sLut)[i] = reinterpret_cast<const uint4 *>(a.lut)[i];

  const int qtiles = (a.Tq + 127) / 128;
  const int64_t ntiles = (int64_t)qtiles * a.H * a.B;
  const int nkc = (a.Tk + PF_KC - 1) / PF_KC;
  const int D = a.D;

  // Workgroup x runs on XCD x % 8 (round-robin dispatch). With a grid that
  // is a multiple of 8, each XCD takes one contiguous range of tiles, so the
  // query tiles of one (batch, head) share their K and V^T in that XCD's L2.
  const int64_t G = gridDim.x;
  const bool xcd_map = G % 8 == 0;
  const int64_t per_xcd = xcd_map ? (ntiles + 7) / 8 : ntiles;
  const int64_t t0 = xcd_map ? (int64_t)(blockIdx.x % 8) * per_xcd : 0;
  const int64_t t1 = min(t0 + per_xcd, ntiles);
  const int64_t tstep = xcd_map ? G / 8 : G;
  for (int64_t tile = t0 + (xcd_map ? blockIdx.x / 8 : blockIdx.x); tile < t1; tile += tstep) {
    const int qt = (int)(tile % qtiles);
    const int64_t bh = tile / qtiles;
    const int h = (int)(bh % a.H);
    const int64_t b = bh / a.H;
    const int q = qt * 128 + wave * 32 + ql;  // this lane's query row
    const int8_t *kbase = a.k + b * a.k_sb + (int64_t)h * a.k_sh;
    const int8_t *vbase = a.vt + (b * a.H + h) * (int64_t)D * a.vt_ld;

    v4i qf[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const int d0 = ks * 32 + g * 16;
      if (q < a.Tq && d0 < D)
        qf[ks] = *reinterpret_cast<const v4i *>(a.q + b * a.q_sb + (int64_t)q * a.q_st +
                                                 (int64_t)h * D + d0);
      else
        qf[ks] = v4i{0, 0, 0, 0};
    }

    // K and V^T chunks move global -> registers -> LDS. The next chunk's
    // loads are issued as soon as the current one is in LDS, so their
    // latency passes under the current chunk's MFMAs and softmax.
    constexpr int CPK = DP / 16;                     // 16-byte chunks per key row
    constexpr int KPT = (PF_KC * CPK + 255) / 256;   // K pieces per thread
    constexpr int VPT = (DP * 4 + 255) / 256;        // V^T pieces per thread
    uint4 kv[KPT], vv[VPT];
    // A chunk whose keys are all below Tk (and, with DF, every head dim
    // valid) is copied without per-piece tests: the tests' zero fills and
    // exec-mask branches cost more than the loads, and the branchy form made
    // the compiler wait for the next chunk's loads before this chunk's MFMAs.
    constexpr bool KWHOLE = DF && (PF_KC * CPK) % 256 == 0;
    constexpr bool VWHOLE = DF && (DP * 4) % 256 == 0;
    auto load_k = [&](int kc, auto whole_tag) {
      constexpr bool W = decltype(whole_tag)::value && KWHOLE;
#pragma unroll
      for (int j = 0; j < KPT; ++j) {
        const int c = tid + 256 * j;
        const int kk = c / CPK, part = c % CPK;
        const int key = kc * PF_KC + kk;
        if (W) {
          kv[j] = *reinterpret_cast<const uint4 *>(kbase + (int64_t)key * a.k_st + part * 16);
        } else {
          kv[j] = make_uint4(0, 0, 0, 0);
          if (c < PF_KC * CPK && key < a.Tk && part * 16 < D)
            kv[j] = *reinterpret_cast<const uint4 *>(kbase + (int64_t)key * a.k_st + part * 16);
        }
      }
    };
    auto store_k = [&]() {
#pragma unroll
      for (int j = 0; j < KPT; ++j) {
        const int c = tid + 256 * j;
        if (c < PF_KC * CPK) {
          const int kk = c / CPK, part = c % CPK;
          const int row = (kk & 32) + key_row(kk & 31);
          *reinterpret_cast<uint4 *>(&sK[row * KLD + kpos(row, part) * 16]) = kv[j];
        }
      }
    };
    // V^T chunk: rows d, 64 keys each (4 pieces of 16 bytes)
    auto load_v = [&](int kc, auto whole_tag) {
      constexpr bool W = decltype(whole_tag)::value && VWHOLE;
#pragma unroll
      for (int j = 0; j < VPT; ++j) {
        const int c = tid + 256 * j;
        const int d = c >> 2, part = c & 3;
        const int key0 = kc * PF_KC + part * 16;
        if (W) {
          vv[j] = *reinterpret_cast<const uint4 *>(vbase + (int64_t)d * a.vt_ld + key0);
        } else {
          vv[j] = make_uint4(0, 0, 0, 0);
          if (c < DP * 4 && d < D && key0 < a.vt_ld)
            vv[j] = *reinterpret_cast<const uint4 *>(vbase + (int64_t)d * a.vt_ld + key0);
        }
      }
    };
    auto store_v = [&]() {
#pragma unroll
      for (int j = 0; j < VPT; ++j) {
        const int c = tid + 256 * j;
        if (c < DP * 4) *reinterpret_cast<uint4 *>(&sVt[(c >> 2) * VLD + kpos(c >> 2, c & 3) * 16]) = vv[j];
      }
    };
    auto scores = [&](int sub) {
      v16i s;
#pragma unroll
      for (int r = 0; r < 16; ++r) s[r] = 0;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const v4i ka = *reinterpret_cast<const v4i *>(&sK[(sub * 32 + ql) * KLD + kpos(sub * 32 + ql, ks * 2 + g) * 16]);
        s = __builtin_amdgcn_mfma_i32_32x32x32_i8(ka, qf[ks], s, 0, 0, 0);
      }
      return s;
    };

    // ---- pass 1: row max of the raw scores over unmasked keys ----
    // The chunks whose keys are all below Tk (no mask) take no per-key test
    // and run as a loop of their own, ahead of the rest.
    int32_t mx = INT32_MIN;
    using Yes = std::true_type;
    using No = std::false_type;
    // NEXT_WHOLE: chunk kc + 1 exists and all its keys are below Tk
    auto pass1 = [&](int kc, auto full_tag, auto next_tag) {
      constexpr bool FULL = decltype(full_tag)::value;
      constexpr bool NEXT_WHOLE = decltype(next_tag)::value;
      store_k();
      __syncthreads();
      // next: K chunk kc + 1, or pass 2's first K and V chunks
      if (NEXT_WHOLE) {
        load_k(kc + 1, Yes{});
      } else if (kc + 1 < nkc) {
        load_k(kc + 1, No{});
      } else {
        load_k(0, No{});
        load_v(0, No{});
      }
#pragma unroll
      for (int sub = 0; sub < 2; ++sub) {
        const v16i s = scores(sub);
        if constexpr (FULL) {
#pragma unroll
          for (int r = 0; r < 16; r += 2) mx = max(max(mx, s[r]), s[r + 1]);
        } else {
          const int kbase0 = kc * PF_KC + sub * 32 + g * 16;
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int key = kbase0 + r;
            bool ok = key < a.Tk;
            if (HAS_MASK) ok = ok && q < a.Tq && !a.mask[(int64_t)q * a.Tk + key];
            if (ok) mx = max(mx, s[r]);
          }
        }
      }
      __syncthreads();
    };
    load_k(0, No{});
    // chunks whose keys are all below Tk
    const int nfk = HAS_MASK ? 0 : a.Tk / PF_KC;
    int kc1 = 0;
    for (; kc1 + 1 < nfk; ++kc1) pass1(kc1, Yes{}, Yes{});
    for (; kc1 < nfk; ++kc1) pass1(kc1, Yes{}, No{});
    for (; kc1 < nkc; ++kc1) pass1(kc1, No{}, No{});
    mx = max(mx, __shfl_xor(mx, 32));
    const int32_t rowmax = mx == INT32_MIN ? -32768 : qk_requant16(mx, a.qk_m, a.qk_s);
    const uint32_t rmp1 = (uint32_t)(uint16_t)(rowmax + 1);

    // ---- pass 2: P = E(S - rmp1) and O = P . V ----
    // requant constants (a shift >= 32 gives 0: multiplier 0 instead)
    const int32_t qm24 = a.qk_s >= 32 ? 0 : (int32_t)a.qk_m;
    const uint32_t qsh = a.qk_s >= 32 ? 0u : a.qk_s;
    const uint32_t qhalf = qsh ? 1u << (qsh - 1) : 0u;
    const uint32_t qw = min(qsh, 1u);
    // Keys of a full chunk all count in the row maximum, so with the row
    // maximum below 32767 rowmax + 1 - h16 lies in [1, 65535] and the table
    // index is
    //   min(R - clamp16(h), L) = med3(R - h, min(R - 32767, L), min(R + 32768, L))
    // with R = rowmax + 1 and h the unsaturated shift. R - h itself is one
    // shift: with v = s * m, h = (v + half - [v < 0]) >> sh (floor), and
    //   R - h = (R * 2^sh + 2^sh - 1 - half - v + [v < 0]) >> sh   (floor),
    // which stays inside int32: |v| <= 2^21 * 255 < 2^29 and |R| <= 2^(29 - sh) + 2
    // for sh <= 29. For sh >= 30 every h is 0 (|v| < 2^29 <= half), the same
    // as m = 0 with sh = 0. [v < 0] = [s < 0] when m > 0; when m = 0 the term
    // is below the rounding step either way (2^sh - half <= 2^sh - 1).
    const uint32_t fsh = a.qk_s >= 30 ? 0u : a.qk_s;
    const int32_t fnm = a.qk_s >= 30 ? 0 : -(int32_t)a.qk_m;
    const uint32_t fw = min(fsh, 1u);
    const int32_t fR = rowmax + 1;
    const bool no_sat = !__any(rowmax >= 32767);
    const int32_t fK = (int32_t)(((uint32_t)fR << fsh) + ((1u << fsh) - 1u) - (fsh ? 1u << (fsh - 1) : 0u));
    const int32_t flo = min(fR - 32767, IW_SEXP_LUT - 1), fhi = min(fR + 32768, IW_SEXP_LUT - 1);
    v16i o[KS];
#pragma unroll
    for (int t = 0; t < KS; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) o[t][r] = 0;
    uint32_t psum = 0;
    // Full chunks (all keys below Tk, no mask, no row maximum at 32767) run
    // as a loop of their own with the short table index. There the index is
    // at least 1, where the table holds at most 95 (x_sub <= -1 gives
    // e < 0.75 * 2^f before the final shift to 7 fraction bits), so P fits
    // the signed int8 MFMA operand as it is. The other chunks keep the
    // per-key tests and the split of P = 128 (x_sub = 0 after the int16 wrap
    // of a row maximum at 32767).
    auto pass2 = [&](int kc, auto full_tag, auto next_tag) {
      constexpr bool FULL = decltype(full_tag)::value;
      constexpr bool NEXT_WHOLE = decltype(next_tag)::value;
      store_k();
      store_v();
      __syncthreads();
      if (NEXT_WHOLE) {
        load_k(kc + 1, Yes{});
        load_v(kc + 1, Yes{});
      } else if (kc + 1 < nkc) {
        load_k(kc + 1, No{});
        load_v(kc + 1, No{});
      }
#pragma unroll
      for (int sub = 0; sub < 2; ++sub) {
        const v16i s = scores(sub);
        const int kbase0 = kc * PF_KC + sub * 32 + g * 16;
        // P of the 16 keys: requant (24-bit product: |score| < 2^21 and an
        // 8-bit multiplier), round-half-away shift, int16 saturation, then
        // the table at min((rowmax + 1 - h16) mod 2^16, size - 1)
        // (keys past Tk or masked: P = 0, applied as a byte mask on the
        // loaded value rather than a conditional write)
        uint32_t pb[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          uint32_t idx;
          if constexpr (FULL) {
            const uint32_t y = (uint32_t)(__mul24(s[r], fnm) + fK) -
                               (uint32_t)__builtin_amdgcn_sbfe(s[r], 31, fw);
            idx = (uint32_t)med3i((int32_t)y >> fsh, flo, fhi);
          } else {
            const int32_t v = __mul24(s[r], qm24);
            const uint32_t tr = (uint32_t)v + qhalf + (uint32_t)__builtin_amdgcn_sbfe(v, 31, qw);
            const int32_t h16 = clampi((int32_t)tr >> qsh, -32768, 32767);
            idx = min((rmp1 - (uint32_t)h16) & 0xffffu, (uint32_t)(IW_SEXP_LUT - 1));
          }
          pb[r] = (uint32_t)sLut[idx];
          if constexpr (!FULL) {
            const int key = kbase0 + r;
            bool ok = key < a.Tk;
            if (HAS_MASK) ok = ok && q < a.Tq && !a.mask[(int64_t)q * a.Tk + key];
            pb[r] &= ok ? 0xffu : 0u;
          }
        }
        uint32_t pw[4];
#pragma unroll
        for (int j = 0; j < 4; ++j)
          pw[j] = __builtin_amdgcn_perm(__builtin_amdgcn_perm(pb[4 * j + 3], pb[4 * j + 2], 0x0c0c0400u),
                                        __builtin_amdgcn_perm(pb[4 * j + 1], pb[4 * j], 0x0c0c0400u),
                                        0x05040100u);
        const uint32_t ones = 0x01010101u;
        psum = __builtin_amdgcn_udot4(pw[0], ones, psum, false);
        psum = __builtin_amdgcn_udot4(pw[1], ones, psum, false);
        psum = __builtin_amdgcn_udot4(pw[2], ones, psum, false);
        psum = __builtin_amdgcn_udot4(pw[3], ones, psum, false);
        const v4i pa0 = v4i{(int)pw[0], (int)pw[1], (int)pw[2], (int)pw[3]};
        if constexpr (FULL) {
#pragma unroll
          for (int t = 0; t < KS; ++t) {
            const v4i vb = *reinterpret_cast<const v4i *>(&sVt[(t * 32 + ql) * VLD + kpos(t * 32 + ql, sub * 2 + g) * 16]);
            o[t] = __builtin_amdgcn_mfma_i32_32x32x32_i8(pa0, vb, o[t], 0, 0, 0);
          }
        } else {
          // int8 MFMA is signed: tiles with P = 128 split P = lo + 64 * hi2
          const uint32_t hib = (pw[0] | pw[1] | pw[2] | pw[3]) & 0x80808080u;
          const bool any_hi = __any(hib != 0u);
          v4i pa = pa0, ph;
          if (any_hi) {
            pa = v4i{(int)(pw[0] & 0x7f7f7f7fu), (int)(pw[1] & 0x7f7f7f7fu),
                     (int)(pw[2] & 0x7f7f7f7fu), (int)(pw[3] & 0x7f7f7f7fu)};
            ph = v4i{(int)((pw[0] >> 1) & 0x40404040u), (int)((pw[1] >> 1) & 0x40404040u),
                     (int)((pw[2] >> 1) & 0x40404040u), (int)((pw[3] >> 1) & 0x40404040u)};
          }
#pragma unroll
          for (int t = 0; t < KS; ++t) {
            const v4i vb = *reinterpret_cast<const v4i *>(&sVt[(t * 32 + ql) * VLD + kpos(t * 32 + ql, sub * 2 + g) * 16]);
            o[t] = __builtin_amdgcn_mfma_i32_32x32x32_i8(pa, vb, o[t], 0, 0, 0);
            if (any_hi) {
              // 128 * hi = 64 * hi + 64 * hi
              o[t] = __builtin_amdgcn_mfma_i32_32x32x32_i8(ph, vb, o[t], 0, 0, 0);
              o[t] = __builtin_amdgcn_mfma_i32_32x32x32_i8(ph, vb, o[t], 0, 0, 0);
            }
          }
        }
      }
      __syncthreads();
    };
    // the split point is uniform over the wave; every wave of the block runs
    // nkc iterations, so the barriers pair up
    const int nfull2 = no_sat ? nfk : 0;
    int kc2 = 0;
    for (; kc2 + 1 < nfull2; ++kc2) pass2(kc2, Yes{}, Yes{});
    for (; kc2 < nfull2; ++kc2) pass2(kc2, Yes{}, No{});
    for (; kc2 < nkc; ++kc2) pass2(kc2, No{}, No{});
    psum += (uint32_t)__shfl_xor((int)psum, 32);
    if (g == 0) sInv[wave][ql] = fisr((int32_t)psum, a.rsqrt_off);
    __syncthreads();

    // ---- epilogue: lane owns head dim t*32 + l%32 for 16 query rows ----
#pragma unroll
    for (int t = 0; t < KS; ++t) {
      const int d = t * 32 + ql;
      if (d >= D) continue;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int qr = (r >> 2) * 8 + g * 4 + (r & 3);
        const int qq = qt * 128 + wave * 32 + qr;
        if (qq >= a.Tq) continue;
        const int32_t inv = sInv[wave][qr];
        int32_t y = rshift((int32_t)((uint32_t)o[t][r] * (uint32_t)inv), a.rsqrt_off);
        y = rshift((int32_t)((uint32_t)y * (uint32_t)inv), a.rsqrt_off);
        y = rshift((int32_t)((uint32_t)y * a.av_m), a.av_s);
        a.out[b * a.o_sb + (int64_t)qq * a.o_st + (int64_t)h * D + d] = (int8_t)clampi(y, -127, 127);
      }
    }
    __syncthreads();
  }
}

// ------------------------------------------------------------------------
// Decode attention: one block per (batch, head, query row)
// ------------------------------------------------------------------------
constexpr int DEC_MAX_TK = 4096;

__global__ __launch_bounds__(256) void attn_decode_kernel(AttnArgs a) {
  __shared__ int32_t sS[DEC_MAX_TK];
  __shared__ __attribute__((aligned(16))) uint8_t sP[DEC_MAX_TK];
  __shared__ int32_t sRed[8];
  __shared__ uint32_t sSum[8];
  __shared__ uint32_t sHi;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int qi = blockIdx.y;
  const int64_t bh = blockIdx.x;
  const int h = (int)(bh % a.H);
  const int64_t b = bh / a.H;
  const int D = a.D;
  const int nq = D >> 4;  // 16-byte chunks per row (D % 16 == 0, D <= 128)
  if (tid == 0) sHi = 0;

  uint4 qv[8];
  const int8_t *qr = a.q + b * a.q_sb + (int64_t)qi * a.q_st + (int64_t)h * D;
#pragma unroll
  for (int c = 0; c < 8; ++c) qv[c] = c < nq ? reinterpret_cast<const uint4 *>(qr)[c] : make_uint4(0, 0, 0, 0);
  const int8_t *kb = a.k + b * a.k_sb + (int64_t)h * a.k_sh;

  // phase 1: raw scores and their max over unmasked keys
  int32_t mx = INT32_MIN;
  for (int j = tid; j < a.Tk; j += 256) {
    const uint4 *kr = reinterpret_cast<const uint4 *>(kb + (int64_t)j * a.k_st);
    int32_t acc = 0;
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      if (c < nq) {
        const uint4 kv = kr[c];
        acc = __builtin_amdgcn_sdot4((int)qv[c].x, (int)kv.x, acc, false);
        acc = __builtin_amdgcn_sdot4((int)qv[c].y, (int)kv.y, acc, false);
        acc = __builtin_amdgcn_sdot4((int)qv[c].z, (int)kv.z, acc, false);
        acc = __builtin_amdgcn_sdot4((int)qv[c].w, (int)kv.w, acc, false);
      }
    }
    sS[j] = acc;
    const bool ok = !(a.mask && a.mask[(int64_t)qi * a.Tk + j]);
    if (ok) mx = max(mx, acc);
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) mx = max(mx, __shfl_xor(mx, off));
  if (lane == 0) sRed[wave] = mx;
  __syncthreads();
  mx = max(max(sRed[0], sRed[1]), max(sRed[2], sRed[3]));
  const int32_t rowmax = mx == INT32_MIN ? -32768 : qk_requant16(mx, a.qk_m, a.qk_s);
  const uint32_t rmp1 = (uint32_t)(uint16_t)(rowmax + 1);

  // phase 2: P and its sum
  uint32_t psum = 0, hi = 0;
  for (int j = tid; j < a.Tk; j += 256) {
    uint32_t p = 0;
    if (!(a.mask && a.mask[(int64_t)qi * a.Tk + j])) {
      const int32_t h16 = qk_requant16(sS[j], a.qk_m, a.qk_s);
      // x_sub = qk - rmp1 modulo 2^16
      p = shift_exp_one((int32_t)(int16_t)(uint16_t)((uint32_t)h16 - rmp1), a.frac_bits);
    }
    sP[j] = (uint8_t)p;
    psum += p;
    hi |= p;
  }
  // zero the tail of the last 16-byte chunk
  const int tk16 = (a.Tk + 15) & ~15;
  for (int j = a.Tk + tid; j < tk16; j += 256) sP[j] = 0;
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) psum += (uint32_t)__shfl_xor((int)psum, off);
  if (lane == 0) sSum[wave] = psum;
  if (hi & 0x80u) atomicOr(&sHi, 1u);
  __syncthreads();
  const int32_t total = (int32_t)(sSum[0] + sSum[1] + sSum[2] + sSum[3]);
  const int32_t inv = fisr(total, a.rsqrt_off);
  const bool any_hi = sHi != 0;

  // phase 3: O[d] = sum_j P[j] V^T[d][j]; 256 / D threads per head dim
  int tpd = 1;  // threads per head dim: largest power of two <= 256 / D
  while (tpd * 2 * D <= 256) tpd *= 2;
  const int d = tid / tpd, part = tid % tpd;
  const int8_t *vr = a.vt + b * a.v_sb + (int64_t)h * a.v_sh + (int64_t)(d < D ? d : 0) * a.v_sd;
  uint32_t acc = 0;
  const int nchunk = d < D ? (tk16 >> 4) : 0;
  for (int c = part; c < nchunk; c += tpd) {
    uint4 pv = reinterpret_cast<const uint4 *>(sP)[c];
    uint4 vv = *reinterpret_cast<const uint4 *>(vr + c * 16);
    // keys beyond Tk have P = 0
    if (!any_hi) {
      acc = (uint32_t)__builtin_amdgcn_sdot4((int)pv.x, (int)vv.x, (int)acc, false);
      acc = (uint32_t)__builtin_amdgcn_sdot4((int)pv.y, (int)vv.y, (int)acc, false);
      acc = (uint32_t)__builtin_amdgcn_sdot4((int)pv.z, (int)vv.z, (int)acc, false);
      acc = (uint32_t)__builtin_amdgcn_sdot4((int)pv.w, (int)vv.w, (int)acc, false);
    } else {
      const uint32_t lo[4] = {pv.x & 0x7f7f7f7fu, pv.y & 0x7f7f7f7fu, pv.z & 0x7f7f7f7fu, pv.w & 0x7f7f7f7fu};
      const uint32_t hb[4] = {(pv.x >> 7) & 0x01010101u, (pv.y >> 7) & 0x01010101u,
                              (pv.z >> 7) & 0x01010101u, (pv.w >> 7) & 0x01010101u};
      const uint32_t vw[4] = {vv.x, vv.y, vv.z, vv.w};
      int32_t hs = 0;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        acc = (uint32_t)__builtin_amdgcn_sdot4((int)lo[e], (int)vw[e], (int)acc, false);
        hs = __builtin_amdgcn_sdot4((int)hb[e], (int)vw[e], hs, false);
      }
      acc += (uint32_t)hs << 7;
    }
  }
  for (int off = 1; off < tpd; off <<= 1) acc += (uint32_t)__shfl_xor((int)acc, off);
  if (part == 0 && d < D) {
    int32_t y = rshift((int32_t)(acc * (uint32_t)inv), a.rsqrt_off);
    y = rshift((int32_t)((uint32_t)y * (uint32_t)inv), a.rsqrt_off);
    y = rshift((int32_t)((uint32_t)y * a.av_m), a.av_s);
    a.out[b * a.o_sb + (int64_t)qi * a.o_st + (int64_t)h * D + d] = (int8_t)clampi(y, -127, 127);
  }
}


// ------------------------------------------------------------------------
// Decode attention over per-head KV caches (one query row per (batch, head))
// ------------------------------------------------------------------------
//
// K cache [B, H, T_cap, D] (rows of D bytes contiguous per head), V cache
// transposed [B, H, D, T_cap16]. The key count is k_length, plus *pos when
// pos is given (the self-attention cache length lives on the device, so a
// captured decode step can be replayed). One block of 256 threads per
// (batch, head):
//   1. scores: LPK lanes share a key (16 bytes each), so one wave load reads
//      64 / LPK consecutive keys; raw int32 scores go to LDS and their max
//      gives the row max (the requant is monotone);
//   2. P = shift_exp(requant(s) - row_max - 1) to LDS, with its row sum;
//   3. O[d] = sum_j P[j] V^T[d][j]: each wave owns D / 4 rows of V^T and its
//      lanes walk a row's 16-byte chunks, so each wave load reads 1 KB of one
//      row; the per-lane partial sums are reduced once per row.
constexpr int DC_MAX_TK = 4096;

template <int D, int PRE>
__global__ __launch_bounds__(256) void attn_decode_cache_kernel(AttnArgs a, const int32_t *pos) {
  constexpr int CPK = D / 16;                      // 16-byte chunks per key
  constexpr int LPK = CPK <= 4 ? 4 : 8;            // lanes per key
  constexpr int KPW = 64 / LPK;                    // keys per wave load
  constexpr int RPW = D / 4;                       // V^T rows per wave
  constexpr int UK = 4;                            // key loads in flight per lane
  __shared__ int32_t sS[DC_MAX_TK];
  __shared__ __attribute__((aligned(16))) uint8_t sP[DC_MAX_TK];
  __shared__ int32_t sRed[4];
  __shared__ uint32_t sSum[4];
  __shared__ uint32_t sHi;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t bh = blockIdx.x;
  const int h = (int)(bh % a.H);
  const int64_t b = bh / a.H;
  const int Tk = min(a.Tk + (pos ? *pos : 0), a.max_tk);
  const int tk16 = (Tk + 15) & ~15;
  const int nch = tk16 >> 4;
  if (tid == 0) sHi = 0;

  // V^T rows of this wave: the first PRE chunk sets (chunks lane + 64 i) are
  // requested now, so they stream in while the scores are computed
  const int8_t *vb = a.vt + b * a.v_sb + (int64_t)h * a.v_sh + (int64_t)(wave * RPW) * a.v_sd;
  uint4 vpre[PRE][RPW];
#pragma unroll
  for (int i = 0; i < PRE; ++i) {
    const int c = lane + 64 * i;
#pragma unroll
    for (int r = 0; r < RPW; ++r)
      vpre[i][r] = c < nch ? *reinterpret_cast<const uint4 *>(vb + (int64_t)r * a.v_sd + c * 16)
                           : make_uint4(0, 0, 0, 0);
  }

  // ---- phase 1: raw scores ----
  const int chunk = lane % LPK;
  const bool cvalid = chunk < CPK;
  v4i qv = v4i{0, 0, 0, 0};
  if (cvalid)
    qv = *reinterpret_cast<const v4i *>(a.q + b * a.q_sb + (int64_t)h * D + chunk * 16);
  const int8_t *kb = a.k + b * a.k_sb + (int64_t)h * a.k_sh;
  int32_t mx = INT32_MIN;
  for (int j0 = wave * KPW; j0 < Tk; j0 += 4 * KPW * UK) {
    v4i kv[UK];
#pragma unroll
    for (int u = 0; u < UK; ++u) {
      const int j = j0 + u * 4 * KPW + lane / LPK;
      kv[u] = (j < Tk && cvalid)
                  ? *reinterpret_cast<const v4i *>(kb + (int64_t)j * a.k_st + chunk * 16)
                  : v4i{0, 0, 0, 0};
    }
#pragma unroll
    for (int u = 0; u < UK; ++u) {
      const int j = j0 + u * 4 * KPW + lane / LPK;
      int32_t acc = 0;
      acc = __builtin_amdgcn_sdot4(qv[0], kv[u][0], acc, false);
      acc = __builtin_amdgcn_sdot4(qv[1], kv[u][1], acc, false);
      acc = __builtin_amdgcn_sdot4(qv[2], kv[u][2], acc, false);
      acc = __builtin_amdgcn_sdot4(qv[3], kv[u][3], acc, false);
#pragma unroll
      for (int o = 1; o < LPK; o <<= 1) acc += __shfl_xor(acc, o);
      if (j < Tk) {
        if (chunk == 0) sS[j] = acc;
        mx = max(mx, acc);
      }
    }
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) mx = max(mx, __shfl_xor(mx, off));
  if (lane == 0) sRed[wave] = mx;
  __syncthreads();
  mx = max(max(sRed[0], sRed[1]), max(sRed[2], sRed[3]));
  const int32_t rowmax = mx == INT32_MIN ? -32768 : qk_requant16(mx, a.qk_m, a.qk_s);
  const uint32_t rmp1 = (uint32_t)(uint16_t)(rowmax + 1);

  // ---- phase 2: P and its row sum ----
  uint32_t psum = 0, hi = 0;
  for (int j = tid; j < tk16; j += 256) {
    uint32_t p = 0;
    if (j < Tk) {
      const int32_t h16 = qk_requant16(sS[j], a.qk_m, a.qk_s);
      // x_sub = qk - rmp1 modulo 2^16
      p = shift_exp_one((int32_t)(int16_t)(uint16_t)((uint32_t)h16 - rmp1), a.frac_bits);
    }
    sP[j] = (uint8_t)p;
    psum += p;
    hi |= p;
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) psum += (uint32_t)__shfl_xor((int)psum, off);
  if (lane == 0) sSum[wave] = psum;
  if (hi & 0x80u) atomicOr(&sHi, 1u);
  __syncthreads();
  const int32_t total = (int32_t)(sSum[0] + sSum[1] + sSum[2] + sSum[3]);
  const int32_t inv = fisr(total, a.rsqrt_off);
  const bool any_hi = sHi != 0;

  // ---- phase 3: O = P . V^T ----
  uint32_t accd[RPW];
#pragma unroll
  for (int r = 0; r < RPW; ++r) accd[r] = 0;
  auto consume = [&](const uint4 pv, const uint4 *vv) {
    const uint32_t pw[4] = {pv.x, pv.y, pv.z, pv.w};
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
      const uint32_t vw[4] = {vv[r].x, vv[r].y, vv[r].z, vv[r].w};
      if (!any_hi) {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          accd[r] = (uint32_t)__builtin_amdgcn_sdot4((int)pw[e], (int)vw[e], (int)accd[r], false);
      } else {
        // P = 128 only after an int16 row-max wrap: split off the top bit
        int32_t hs = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          accd[r] = (uint32_t)__builtin_amdgcn_sdot4((int)(pw[e] & 0x7f7f7f7fu), (int)vw[e],
                                                     (int)accd[r], false);
          hs = __builtin_amdgcn_sdot4((int)((pw[e] >> 7) & 0x01010101u), (int)vw[e], hs, false);
        }
        accd[r] += (uint32_t)hs << 7;
      }
    }
  };
#pragma unroll
  for (int i = 0; i < PRE; ++i) {
    const int c = lane + 64 * i;
    if (c < nch) consume(reinterpret_cast<const uint4 *>(sP)[c], vpre[i]);
  }
  for (int c = lane + 64 * PRE; c < nch; c += 64) {
    uint4 vv[RPW];
#pragma unroll
    for (int r = 0; r < RPW; ++r) vv[r] = *reinterpret_cast<const uint4 *>(vb + (int64_t)r * a.v_sd + c * 16);
    consume(reinterpret_cast<const uint4 *>(sP)[c], vv);
  }
#pragma unroll
  for (int r = 0; r < RPW; ++r) {
    uint32_t v = accd[r];
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += (uint32_t)__shfl_xor((int)v, off);
    accd[r] = v;
  }
  if (lane < RPW) {
    uint32_t accv = 0;
#pragma unroll
    for (int r = 0; r < RPW; ++r)
      if (r == lane) accv = accd[r];
    const int d = wave * RPW + lane;
    int32_t y = rshift((int32_t)(accv * (uint32_t)inv), a.rsqrt_off);
    y = rshift((int32_t)((uint32_t)y * (uint32_t)inv), a.rsqrt_off);
    y = rshift((int32_t)((uint32_t)y * a.av_m), a.av_s);
    a.out[decode_out_index(a, b, h * D + d)] = (int8_t)clampi(y, -127, 127);
  }
}

// ---------------------------------------------------------------------------
// Decode attention over the caches for head_dim 64 (every Whisper size),
// streaming K and V through LDS.
//
// One block per (batch, head) reads Tk x 64 bytes of K and 64 x Tk bytes of
// V^T, nothing else of size, so the kernel is HBM-bound and a CU needs many
// bytes in flight (bandwidth x latency). Both operands flow through one ring
// of NR slots in CH-key chunks: K chunks 0 .. nK-1, then V^T chunks, so the
// copies of V are already under way while the row maximum and P are formed.
// A chunk is DPC = CH / (16 NW) global_load_lds_dwordx4 copies for each of
// the block's NW waves (K: 16 keys per copy; V^T: 64 / NW rows), and every
// lane later reads back exactly the 16-byte pieces it copied (K: one key's
// 16 (l % 4)-th piece; V^T: one d-row's piece of 16 keys), so a wave only
// waits for its own copies (vmcnt) and the ring needs no barrier. Keys past
// Tk read the last valid key / piece; their scores are dropped and their P
// is 0.
//
// VQ: V in key quads ([t/4][d][t%4], a quad of keys v_sq bytes apart). A
// chunk of V is then CH/4 whole quads; a copy brings 4 quads, lane l the 16
// bytes of d = 4 (l % 16) .. +3 of one quad, and the lane's four sdot4 take
// the same P word. Each wave sums its own quads, so the d sums of the NW
// waves meet in LDS at the end.
//
// NQ > 1 (V^T): the a.Tq <= NQ query positions of a (batch, head) share the
// stream (the decoder's prompt over the cross-attention cache): each chunk in
// LDS is scored against, then weighted by, every query's P; query i at
// q + b*q_sb + i*q_st, its output at out + b*o_sb + i*o_st. The queries are
// loaded into registers behind the first chunks' copies.
// ---------------------------------------------------------------------------

// 128-key chunks in a 3-slot ring (24 KB): measured fastest among chunks of
// 64 / 128 / 256 keys and rings of 2 to 10 slots (several small blocks per CU
// hide each block's row-maximum pause better than one deep ring).
#ifndef IW_DS_NR
#define IW_DS_NR 3
#endif
#ifndef IW_DS_CH
#define IW_DS_CH 128
#endif
// the self-attention instance (at most 512 keys) has its own ring shape
#ifndef IW_DSS_NR
#define IW_DSS_NR 3
#endif
#ifndef IW_DSS_CH
#define IW_DSS_CH 128
#endif
// waves per (batch, head) of the self-attention instance. Two waves with
// 64-key chunks (13.8 KB of LDS) make the 2560 heads of a batch of 128
// resident at once instead of in two rounds, and are faster on one layer's
// cache replayed (partly Infinity-Cache-resident), but slower inside the
// decode step, where every layer's cache streams from HBM (22.4 against
// 21.4 us per launch).
#ifndef IW_DSS_NW
#define IW_DSS_NW 4
#endif
// waves per (batch, head) of the register-resident self-attention kernel
#ifndef IW_DSELF_NW
#define IW_DSELF_NW 4
#endif
// blocks at the end of the self-attention launch that read the next GEMM's
// weight into L2 (the rest of the launch's K/V stream, which would evict
// those lines, is short by then)
constexpr int kSelfTailBlocks = 128;

// The query of (batch b, head h) for attn_decode_cross_lnq_kernel, as 64
// bytes of LDS: LayerNorm32 of row b (the integer steps of
// layernorm32_row_kernel: thread t owns elements t, t + 256, ..., three
// reduction rounds) into the LDS row hb, then Linear8 of the head's 64
// channels: wave w takes the k32 steps s = w, w + 4, ... of both 32-channel
// fragment rows of wq (lane l: channel 32 r + l % 32, bytes 32 s + 16 (l / 32)
// .. +15, against the same bytes of hb), the partial sums meet in LDS
// (ds_add, modulo 2^32) and threads 0-63 apply the Linear8 epilogue with the
// row sum of hb for the zero-point term. The row, the parameters and the
// first five steps' weight fragments are requested first (ln_query_load),
// ahead of the block's first K/V chunk copies, so that the LayerNorm waits
// for its own loads only; the other five steps' fragments after it.
struct LnqRegs {
  int32_t v[5], gm[5], bt[5];
  int32_t qb, qz, qs;
  uint32_t qm;
  v4i f0[5], f1[5];
};

__device__ __forceinline__ void lnq_frags(const LnQueryArgs &lq, int h, int half, v4i (&f0)[5], v4i (&f1)[5]) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nst = (int)(lq.kp >> 5);  // k32 steps (the padding has zero weights)
  const int8_t *w0 = lq.wq + ((int64_t)(2 * h) * nst) * 1024 + lane * 16;
  const int8_t *w1 = w0 + (int64_t)nst * 1024;
#pragma unroll
  for (int t = 0; t < 5; ++t) {
    const int st = wave + 4 * (5 * half + t);
    const int sc = st < nst ? st : 0;
    f0[t] = *reinterpret_cast<const v4i *>(w0 + (int64_t)sc * 1024);
    f1[t] = *reinterpret_cast<const v4i *>(w1 + (int64_t)sc * 1024);
  }
}

__device__ __forceinline__ void ln_query_load(const LnQueryArgs &lq, int64_t b, int h, LnqRegs &r) {
  const int tid = threadIdx.x;
  const int C = lq.hidden;
  const int16_t *xr = lq.x + b * lq.ldx;
#pragma unroll
  for (int j = 0; j < 5; ++j) {
    const int e = tid + 256 * j;
    const bool ok = e < C;
    r.v[j] = ok ? xr[e] : 0;
    r.gm[j] = ok ? lq.gamma[e] : 0;
    r.bt[j] = (ok && lq.beta) ? lq.beta[e] : 0;
  }
  // the epilogue parameters of channel h * 64 + tid % 64
  const int n = h * 64 + (tid & 63);
  r.qb = lq.bias ? lq.bias[n] : 0;
  r.qz = lq.wz ? (int32_t)lq.wz[n] : 0;
  r.qm = lq.mult[n];
  r.qs = lq.shift[n];
  lnq_frags(lq, h, 0, r.f0, r.f1);
}

// The normalised row (up to 1280 bytes) and the query sums (64 words) use
// sP, which the attention first writes after the scores.
__device__ __forceinline__ const int8_t *ln_query(const LnQueryArgs &lq, LnqRegs &r, int h, uint8_t *sP) {
  constexpr int NWV = 4;
  __shared__ uint32_t sLn[3][NWV];  // the LayerNorm's wave partials
  __shared__ __attribute__((aligned(16))) int8_t q8[64];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int C = lq.hidden;
  int8_t *hb = reinterpret_cast<int8_t *>(sP);
  int32_t *qacc = reinterpret_cast<int32_t *>(sP + 1280);
  if (r.qs < 0 || r.qs >= 32) r.qm = 0, r.qs = 0;  // linear8_scalar.cpp:71-74: such a shift gives 0
  if (tid < 64) qacc[tid] = 0;

  uint32_t sum = 0;
#pragma unroll
  for (int j = 0; j < 5; ++j) sum += (uint32_t)r.v[j];
  sum = wave_sum_dpp(sum);
  if (lane == 0) sLn[0][wave] = sum;
  lds_barrier();
  const int32_t mean = norm_reduce((int32_t)(sLn[0][0] + sLn[0][1] + sLn[0][2] + sLn[0][3]), lq.code);
  int32_t maxsq = 0;
#pragma unroll
  for (int j = 0; j < 5; ++j)
    if (tid + 256 * j < C) {
      const int32_t d = r.v[j] - mean;
      maxsq = max(maxsq, (int32_t)((uint32_t)d * (uint32_t)d));
    }
  maxsq = wave_max_dpp(maxsq);
  if (lane == 0) sLn[1][wave] = (uint32_t)maxsq;
  lds_barrier();
  maxsq = max(max((int32_t)sLn[1][0], (int32_t)sLn[1][1]), max((int32_t)sLn[1][2], (int32_t)sLn[1][3]));
  int32_t rs = bitlen(maxsq) - 16;
  rs = rs < 0 ? 0 : rs;
  rs = (rs + 1) & ~1;
  uint32_t vs = 0;
#pragma unroll
  for (int j = 0; j < 5; ++j)
    if (tid + 256 * j < C) {
      const int32_t d = r.v[j] - mean;
      vs += (uint32_t)rshift((int32_t)((uint32_t)d * (uint32_t)d), (uint32_t)rs);
    }
  vs = wave_sum_dpp(vs);
  if (lane == 0) sLn[2][wave] = vs;
  lds_barrier();
  const int32_t var = norm_reduce((int32_t)(sLn[2][0] + sLn[2][1] + sLn[2][2] + sLn[2][3]), lq.code);
  const int32_t inv = fisr(var, lq.rsqrt_off);
  const uint32_t nshift = (uint32_t)(lq.ln_s + (rs >> 1));
  uint32_t rsum = 0;
#pragma unroll
  for (int j = 0; j < 5; ++j) {
    const int e = tid + 256 * j;
    if (e < C) {
      const int32_t d = r.v[j] - mean;
      const uint32_t t = (uint32_t)d * (uint32_t)inv * lq.ln_m;
      const int32_t y = clampi(rshift((int32_t)t, nshift), -16383, 16383);
      const uint32_t av = (uint32_t)y * (uint32_t)r.gm[j] + (uint32_t)r.bt[j];
      const int32_t yo = clampi(rshift(mulh((int32_t)av, lq.out_m), (uint32_t)lq.out_s), -127, 127);
      hb[e] = (int8_t)yo;
      rsum += (uint32_t)yo;
    }
  }
  // the normalised row's sum, for the zero-point term (the first reduction's
  // words are free: every thread read them before the second barrier)
  rsum = wave_sum_dpp(rsum);
  if (lane == 0) sLn[0][wave] = rsum;
  lds_barrier();

  const int nst = (int)(lq.kp >> 5);
  const int hoff = 16 * (lane >> 5);
  int32_t acc0 = 0, acc1 = 0;
  auto dot = [&](int half, const v4i (&f0)[5], const v4i (&f1)[5]) {
#pragma unroll
    for (int t = 0; t < 5; ++t) {
      const int st = wave + NWV * (5 * half + t);
      if (st < nst) {
        const v4i hv = *reinterpret_cast<const v4i *>(hb + 32 * st + hoff);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          acc0 = __builtin_amdgcn_sdot4(f0[t][e], hv[e], acc0, false);
          acc1 = __builtin_amdgcn_sdot4(f1[t][e], hv[e], acc1, false);
        }
      }
    }
  };
  // then steps 5..9 of each wave (kp <= 1280: at most ten per wave)
  dot(0, r.f0, r.f1);
  lnq_frags(lq, h, 1, r.f0, r.f1);
  dot(1, r.f0, r.f1);
  atomicAdd(&qacc[lane & 31], acc0);
  atomicAdd(&qacc[32 + (lane & 31)], acc1);
  lds_barrier();
  if (tid < 64) {
    const int32_t xsum = (int32_t)(sLn[0][0] + sLn[0][1] + sLn[0][2] + sLn[0][3]);
    // acc - wz * rowsum + bias modulo 2^32 (|rowsum| <= 127 C < 2^23: exact
    // in the 24-bit multiplier), then the Linear8 requantization
    const uint32_t corr = (uint32_t)qacc[tid] - (uint32_t)__mul24(r.qz, xsum) + (uint32_t)r.qb;
    q8[tid] = (int8_t)clampi(rshift(mulh((int32_t)corr, r.qm), (uint32_t)r.qs), -127, 127);
  }
  lds_barrier();
  return q8;
}

template <int MAXK, int NR, int CH, int NW, bool VQ, int NQ, bool LNQ>
__device__ __forceinline__ void attn_decode_stream_body(const AttnArgs &a, const int32_t *pos,
                                                        const LnQueryArgs &lq) {
  constexpr int D = 64;
  constexpr int DPC = CH / (16 * NW);  // copies per wave per chunk
  constexpr int SLOT = 1024 * NW * DPC;  // bytes per ring slot (CH keys x 64 bytes)
  static_assert(DPC >= 1 && 16 * NW * DPC == CH, "a chunk is whole 1 KB copies of every wave");
  constexpr int WB = 1024 * DPC;      // bytes per wave per slot
  constexpr int LPR = CH / 16;        // lanes per V^T row piece set
  constexpr int RPD = 64 / LPR;       // V^T rows per copy
  static_assert(LPR == 4 || LPR == 8 || LPR == 16, "a V^T row's lanes are 4, 8 or 16 of one 16-lane row");
  constexpr int NACC = VQ ? 4 : DPC;  // P.V sums per lane
  static_assert(!VQ || NW * 64 * 4 <= MAXK * 2, "the wave sums of P.V fit in the score array");
  static_assert(NQ == 1 || !VQ, "several queries stream V transposed");
  static_assert(!LNQ || (NQ == 1 && !VQ && NW == 4), "the fused query: one, V transposed");
  // the fused query's LayerNorm keeps its normalised row (up to 1280 bytes) and the 64 query
  // channels' int32 sums (at byte 1280) in sP
  static_assert(!LNQ || NQ * MAXK >= 1280 + 64 * (int)sizeof(int32_t), "the fused query's row and sums fit in sP");
  __shared__ __attribute__((aligned(1024))) int8_t sRing[NR * SLOT];
  __shared__ __attribute__((aligned(16))) int16_t sS[NQ * MAXK];  // requantized scores
  __shared__ __attribute__((aligned(16))) uint8_t sP[NQ * MAXK];
  __shared__ int32_t sRed[NQ][NW];
  __shared__ uint32_t sSum[NQ][NW];
  __shared__ uint32_t sHi;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int64_t bh = blockIdx.x;
  const int h = (int)(bh % a.H);
  const int64_t b = bh / a.H;
  const int Tk = min(a.Tk + (pos ? *pos : 0), a.max_tk);
  const int nK = (Tk + CH - 1) / CH;  // chunks per operand
  const int T = 2 * nK;
  if (tid == 0) sHi = 0;

  // K: copy u of a chunk brings keys wave*16*DPC + 16 u + l/4, piece l % 4
  const int cq = lane & 3;
  const int kkey = wave * 16 * DPC + (lane >> 2);
  const int8_t *kb = a.k + b * a.k_sb + (int64_t)h * a.k_sh + cq * 16;
  // V^T: copy u brings row wave*16 + u*RPD + l/LPR, keys 16 (l % LPR) .. +16
  const int vp = lane % LPR;
  const int vrow = wave * (64 / NW) + lane / LPR;
  const int8_t *vb = a.vt + b * a.v_sb + (int64_t)h * a.v_sh + (int64_t)vrow * a.v_sd;
  const int vlast = Tk > 0 ? ((Tk - 1) & ~15) : 0;  // last V^T piece holding a valid key
  // V in key quads: copy u brings quad vq0 + 4 u of the chunk, d = 4 (l % 16) .. +3
  const int vq0 = wave * DPC * 4 + (lane >> 4);
  const int8_t *vqb = a.vt + b * a.v_sb + (int64_t)h * a.v_sh + (lane & 15) * 16;
  const int qlast = Tk > 0 ? (Tk - 1) >> 2 : 0;  // last quad holding a valid key
  const uint32_t ring =
      __builtin_amdgcn_readfirstlane((uint32_t)reinterpret_cast<uintptr_t>(sRing)) + wave * WB;
  auto issue = [&](int i) {
    const uint32_t dst = ring + (i % NR) * SLOT;
    if (i < nK) {
#pragma unroll
      for (int u = 0; u < DPC; ++u)
        dma16_lds(kb + (int64_t)min(i * CH + kkey + 16 * u, Tk - 1) * a.k_st, dst + u * 1024);
    } else if (VQ) {
#pragma unroll
      for (int u = 0; u < DPC; ++u)
        dma16_lds(vqb + (int64_t)min((i - nK) * (CH / 4) + vq0 + 4 * u, qlast) * a.v_sq, dst + u * 1024);
    } else {
#pragma unroll
      for (int u = 0; u < DPC; ++u)
        dma16_lds(vb + (int64_t)u * RPD * a.v_sd + min((i - nK) * CH + vp * 16, vlast), dst + u * 1024);
    }
  };

  // q: lane l needs bytes 16 (l % 4) of the head's 64. One query is copied
  // first, into the last ring slot (free until chunk NR - 1), so the chunk
  // waits cover it (counted as DPC copies: the waits below are in whole
  // chunks); several are loaded into registers after the first chunks.
  if constexpr (NQ == 1 && !LNQ) {
#pragma unroll
    for (int u = 0; u < DPC; ++u)
      dma16_lds(a.q + b * a.q_sb + (int64_t)h * D + cq * 16, ring + (NR - 1) * SLOT + u * 1024);
  }
  LnqRegs lr;
  if constexpr (LNQ) ln_query_load(lq, b, h, lr);
  // LNQ: the last slot holds no copied query, so chunk NR - 1 is copied now
  // too, during the LayerNorm and projection (the loop then issues chunk
  // i + NR - 1 from i = 1 on; at i = 0 its wait also covers chunk 1)
#pragma unroll
  for (int i = 0; i < (LNQ ? NR : NR - 1); ++i)
    if (i < T) issue(i);
  const int8_t *q8 = nullptr;
  if constexpr (LNQ) q8 = ln_query(lq, lr, h, sP);
  v4i qv[NQ];
  if constexpr (NQ > 1) {
#pragma unroll
    for (int qi = 0; qi < NQ; ++qi)
      qv[qi] = *reinterpret_cast<const v4i *>(a.q + b * a.q_sb + (int64_t)min(qi, a.Tq - 1) * a.q_st +
                                              (int64_t)h * D + cq * 16);
  } else {
    qv[0] = v4i{0, 0, 0, 0};
  }

  int32_t mx[NQ];
  uint32_t accd[NQ][NACC];
  int32_t hs[NQ][NACC];
  int32_t inv[NQ];
#pragma unroll
  for (int qi = 0; qi < NQ; ++qi) {
    mx[qi] = -32768;
    inv[qi] = 0;
#pragma unroll
    for (int u = 0; u < NACC; ++u) accd[qi][u] = 0, hs[qi][u] = 0;
  }
  bool any_hi = false;

  // row maximum, P and its sum once every score is in sS
  auto form_p = [&]() {
#pragma unroll
    for (int qi = 0; qi < NQ; ++qi) {
      mx[qi] = wave_max_dpp(mx[qi]);
      if (lane == 0) sRed[qi][wave] = mx[qi];
    }
    lds_barrier();
    uint32_t hi = 0;
#pragma unroll
    for (int qi = 0; qi < NQ; ++qi) {
      int32_t rowmax = sRed[qi][0];
#pragma unroll
      for (int w = 1; w < NW; ++w) rowmax = max(rowmax, sRed[qi][w]);
      const uint32_t rmp1 = (uint32_t)(uint16_t)(rowmax + 1);
      uint32_t psum = 0;
      for (int j = tid; j < nK * CH; j += 64 * NW) {
        uint32_t p = 0;
        // x_sub = qk - rmp1 modulo 2^16
        if (j < Tk)
          p = shift_exp_one((int32_t)(int16_t)(uint16_t)((uint32_t)sS[qi * MAXK + j] - rmp1), a.frac_bits);
        sP[qi * MAXK + j] = (uint8_t)p;
        psum += p;
        hi |= p;
      }
      psum = wave_sum_dpp(psum);
      if (lane == 0) sSum[qi][wave] = psum;
    }
    if (hi & 0x80u) atomicOr(&sHi, 1u);
    lds_barrier();
#pragma unroll
    for (int qi = 0; qi < NQ; ++qi) {
      uint32_t total = 0;
#pragma unroll
      for (int w = 0; w < NW; ++w) total += sSum[qi][w];
      inv[qi] = fisr((int32_t)total, a.rsqrt_off);
    }
    any_hi = sHi != 0;
  };

  if (nK == 0) {
    wait_vm<0>();
    form_p();
  }
  for (int i = 0; i < T; ++i) {
    wait_vm_upto<NR - 2, DPC>(min(NR - 2, T - 1 - i));
    if (NQ == 1 && i == 0) {
      if constexpr (LNQ)
        qv[0] = *reinterpret_cast<const v4i *>(q8 + cq * 16);
      else
        qv[0] = *reinterpret_cast<const v4i *>(sRing + (NR - 1) * SLOT + wave * WB + lane * 16);
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // q is read before its slot refills
    }
    v4i x[DPC];
#pragma unroll
    for (int u = 0; u < DPC; ++u)
      x[u] = *reinterpret_cast<const v4i *>(sRing + (i % NR) * SLOT + wave * WB + u * 1024 + lane * 16);
    // the slot of chunk i - 1 is free: this wave read it last iteration
    if (i + NR - 1 < T && (!LNQ || i > 0)) issue(i + NR - 1);
    if (i < nK) {
#pragma unroll
      for (int u = 0; u < DPC; ++u) {
        const int j = i * CH + kkey + 16 * u;
#pragma unroll
        for (int qi = 0; qi < NQ; ++qi) {
          int32_t acc = __builtin_amdgcn_sdot4(qv[qi][0], x[u][0], 0, false);
          acc = __builtin_amdgcn_sdot4(qv[qi][1], x[u][1], acc, false);
          acc = __builtin_amdgcn_sdot4(qv[qi][2], x[u][2], acc, false);
          acc = __builtin_amdgcn_sdot4(qv[qi][3], x[u][3], acc, false);
          acc = quad_sum_dpp(acc);  // the key's four 16-byte pieces
          if (j < Tk) {
            const int32_t h16 = qk_requant16(acc, a.qk_m, a.qk_s);
            if (cq == 0) sS[qi * MAXK + j] = (int16_t)h16;
            mx[qi] = max(mx[qi], h16);
          }
        }
      }
      if (i == nK - 1) form_p();
    } else if (VQ) {
#pragma unroll
      for (int u = 0; u < DPC; ++u) {
        const uint32_t pw = *reinterpret_cast<const uint32_t *>(sP + (i - nK) * CH + (vq0 + 4 * u) * 4);
        if (!any_hi) {
#pragma unroll
          for (int j = 0; j < 4; ++j)
            accd[0][j] = (uint32_t)__builtin_amdgcn_sdot4((int)pw, x[u][j], (int)accd[0][j], false);
        } else {
          // P = 128 only after an int16 row-max wrap: split off the top bit
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            accd[0][j] = (uint32_t)__builtin_amdgcn_sdot4((int)(pw & 0x7f7f7f7fu), x[u][j], (int)accd[0][j], false);
            hs[0][j] = __builtin_amdgcn_sdot4((int)((pw >> 7) & 0x01010101u), x[u][j], hs[0][j], false);
          }
        }
      }
    } else {
#pragma unroll
      for (int qi = 0; qi < NQ; ++qi) {
        const uint4 pv = *reinterpret_cast<const uint4 *>(sP + qi * MAXK + (i - nK) * CH + vp * 16);
        const uint32_t pw[4] = {pv.x, pv.y, pv.z, pv.w};
#pragma unroll
        for (int u = 0; u < DPC; ++u) {
          if (!any_hi) {
#pragma unroll
            for (int e = 0; e < 4; ++e)
              accd[qi][u] = (uint32_t)__builtin_amdgcn_sdot4((int)pw[e], x[u][e], (int)accd[qi][u], false);
          } else {
            // P = 128 only after an int16 row-max wrap: split off the top bit
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              accd[qi][u] =
                  (uint32_t)__builtin_amdgcn_sdot4((int)(pw[e] & 0x7f7f7f7fu), x[u][e], (int)accd[qi][u], false);
              hs[qi][u] = __builtin_amdgcn_sdot4((int)((pw[e] >> 7) & 0x01010101u), x[u][e], hs[qi][u], false);
            }
          }
        }
      }
    }
  }
  auto store = [&](uint32_t v, int d, int qi) {
    int32_t y = rshift((int32_t)(v * (uint32_t)inv[qi]), a.rsqrt_off);
    y = rshift((int32_t)((uint32_t)y * (uint32_t)inv[qi]), a.rsqrt_off);
    y = rshift((int32_t)((uint32_t)y * a.av_m), a.av_s);
    const int8_t o = (int8_t)clampi(y, -127, 127);
    if constexpr (NQ == 1)
      a.out[decode_out_index(a, b, h * D + d)] = o;
    else if (qi < a.Tq)
      a.out[b * a.o_sb + (int64_t)qi * a.o_st + h * D + d] = o;
  };
  if (VQ) {
    // lanes l and l ^ 16, l ^ 32 hold other quads of the same d; then the
    // waves' sums meet in sS, free since form_p's last barrier
    uint4 v;
    uint32_t *vw = &v.x;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      uint32_t t = accd[0][j] + ((uint32_t)hs[0][j] << 7);
      t += (uint32_t)__shfl_xor((int)t, 16);
      vw[j] = t + (uint32_t)__shfl_xor((int)t, 32);
    }
    uint32_t *sPart = reinterpret_cast<uint32_t *>(sS);
    if (lane < 16) *reinterpret_cast<uint4 *>(sPart + wave * 64 + 4 * lane) = v;
    lds_barrier();
    if (tid < 64) {
      uint32_t t = 0;
#pragma unroll
      for (int w = 0; w < NW; ++w) t += sPart[w * 64 + tid];
      store(t, tid, 0);
    }
  } else {
#pragma unroll
    for (int qi = 0; qi < NQ; ++qi)
#pragma unroll
      for (int u = 0; u < DPC; ++u) {
        // the row's LPR lanes l .. l + LPR - 1 (l % LPR == 0): quad sums, then
        // row_shl:4 / :8 (lane i reads lane i + n of its 16-lane row) into l
        int32_t v = quad_sum_dpp((int32_t)(accd[qi][u] + ((uint32_t)hs[qi][u] << 7)));
        if (LPR >= 8) v += __builtin_amdgcn_update_dpp(0, v, 0x104, 0xf, 0xf, true);
        if (LPR >= 16) v += __builtin_amdgcn_update_dpp(0, v, 0x108, 0xf, 0xf, true);
        if (vp == 0) store((uint32_t)v, vrow + u * RPD, qi);
      }
  }
}

template <int MAXK, int NR, int CH, int NW = 4, bool VQ = false, int NQ = 1>
__global__ __launch_bounds__(64 * NW) void attn_decode_stream_kernel(AttnArgs a, const int32_t *pos) {
  attn_decode_stream_body<MAXK, NR, CH, NW, VQ, NQ, false>(a, pos, LnQueryArgs());
}

// The decoder cross-attention with its query computed in the block: the
// LayerNorm before the cross-attention (one row per block, 20 blocks per
// row at Whisper-large) and the head's 64 query channels, while the first
// K chunks are in flight; it replaces a LayerNorm and a query GEMM launch.
// (five blocks per CU, as the plain kernel: at most 96 VGPRs)
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(5, 8))) void attn_decode_cross_lnq_kernel(
    AttnArgs a, LnQueryArgs lq) {
  attn_decode_stream_body<2048, IW_DS_NR, IW_DS_CH, 4, false, 1, true>(a, nullptr, lq);
}

// ---------------------------------------------------------------------------
// Decode self-attention over a V cache in key quads, at most 512 keys: every
// load of K and V is issued at the start, into registers.
//
// A self-attention cache holds at most n_text_ctx (448) positions, so one
// (batch, head) pair is at most 56 KB of K and V, which NW waves hold in
// registers (per 16 NW-key chunk and wave: 16 keys of K and 4 quads of V,
// 8 VGPRs). A block issues every load before it waits for any, so it lives
// for about one memory latency plus its transfer, where a ring of chunks
// waits chunk by chunk.
//
// Lanes, chunk c of wave w (keys c*16NW + 16w + 0..15):
//   K lane l: key 4 (l/16) + l%4, bytes 16 p .. +15 with p = (l/4) % 4. The
//     four lanes of a key are one orbit of rotation by 4 inside a 16-lane
//     row, so two DPP adds complete its score in each of them.
//   V lane l: quad 4 (l/16) (keys 4 (l/16) + 0..3), d = 4 (l%16) .. +3.
// Every K lane holds every chunk's score of its key; lane p of the orbit
// keeps chunks 4g + p, so the requantization, the shift-exp and the P sum run
// once per key and chunk, NC/4 times per lane. The P of keys 4 (l/16) + 0..3
// are then one DPP quad, packed into a word by quad broadcasts; a V lane
// takes the word of its chunk from lane 16 (l/16) + 4 (c%4) (one bpermute).
// Two block barriers: the row maximum, and the final sums of P and P.V. NC
// (chunks) is a template argument, so that each case issues exactly its
// loads; the kernel switches on the chunk count of the device-side key count.
// ---------------------------------------------------------------------------

template <int NW>
struct SelfDecodeLds {
  uint4 part[NW * 64];  // per wave and lane: P.V sums of d = 4 (l % 16) .. +3
  int32_t mx[NW];
  uint32_t sum[NW];
};

template <int CTRL>
__device__ __forceinline__ int32_t dpp_mov(int32_t x) {
  return __builtin_amdgcn_update_dpp(0, x, CTRL, 0xf, 0xf, true);
}
constexpr int kDppRowRor4 = 0x124;
constexpr int kDppRowRor8 = 0x128;
template <int J>
__device__ __forceinline__ uint32_t quad_bcast(uint32_t x) {
  return (uint32_t)dpp_mov<J | (J << 2) | (J << 4) | (J << 6)>((int32_t)x);
}

template <int NW>
__device__ __forceinline__ void self_decode_store(const AttnArgs &a, int64_t b, int h, uint32_t v, uint32_t total,
                                                  int d) {
  const int32_t inv = fisr((int32_t)total, a.rsqrt_off);
  int32_t y = rshift((int32_t)(v * (uint32_t)inv), a.rsqrt_off);
  y = rshift((int32_t)((uint32_t)y * (uint32_t)inv), a.rsqrt_off);
  y = rshift((int32_t)((uint32_t)y * a.av_m), a.av_s);
  a.out[decode_out_index(a, b, h * 64 + d)] = (int8_t)clampi(y, -127, 127);
}

template <int NW, int NC>
__device__ __forceinline__ void self_decode_body(const AttnArgs &a, int64_t b, int h, int Tk,
                                                 SelfDecodeLds<NW> &sm, const FragPrefetch &pf, int pf_start) {
  constexpr int CK = 16 * NW;       // keys per chunk
  constexpr int NG = (NC + 3) / 4;  // scores per lane after the regrouping
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int piece = (lane >> 2) & 3;
  const int kl = wave * 16 + ((lane >> 4) << 2) + (lane & 3);  // key of this K lane in a chunk
  const int ql = wave * 4 + (lane >> 4);                       // quad of this V lane in a chunk
  const int8_t *kb = a.k + b * a.k_sb + (int64_t)h * a.k_sh;
  const int8_t *vb = a.vt + b * a.v_sb + (int64_t)h * a.v_sh;
  // 32-bit offsets inside the head (the launcher checks the cache extent)
  const uint32_t k_st = (uint32_t)a.k_st, v_sq = (uint32_t)a.v_sq;
  const uint32_t koff = (uint32_t)kl * k_st + piece * 16, voff = (uint32_t)ql * v_sq + (lane & 15) * 16;

  const v4i qv = *reinterpret_cast<const v4i *>(a.q + b * a.q_sb + (int64_t)h * 64 + piece * 16);
  v4i kx[NC], vx[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    // the last chunk reads the last valid key / quad in place of those past Tk
    const uint32_t off = c < NC - 1 ? (uint32_t)(c * CK) * k_st + koff
                                    : (uint32_t)min(c * CK + kl, Tk - 1) * k_st + piece * 16;
    kx[c] = *reinterpret_cast<const v4i *>(kb + off);
  }
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const uint32_t off = c < NC - 1 ? (uint32_t)(c * 4 * NW) * v_sq + voff
                                    : (uint32_t)min(c * 4 * NW + ql, (Tk - 1) >> 2) * v_sq + (lane & 15) * 16;
    vx[c] = *reinterpret_cast<const v4i *>(vb + off);
  }
  // every load is issued before the first wait (the scheduler would
  // otherwise defer the V loads to reuse registers)
  __builtin_amdgcn_sched_barrier(0);
  // the launch's last blocks read the out-projection's weight into L2
  uint32_t pfv[1];  // one line per thread: 4096 per XCD from 128 blocks
  frag_prefetch_issue_tail(pf, pf_start, kb, pfv);

  int32_t dot[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    int32_t d = __builtin_amdgcn_sdot4(qv[0], kx[c][0], 0, false);
    d = __builtin_amdgcn_sdot4(qv[1], kx[c][1], d, false);
    d = __builtin_amdgcn_sdot4(qv[2], kx[c][2], d, false);
    d = __builtin_amdgcn_sdot4(qv[3], kx[c][3], d, false);
    d += dpp_mov<kDppRowRor8>(d);
    dot[c] = d + dpp_mov<kDppRowRor4>(d);
  }
  // lane p of a key's orbit keeps chunks 4 g + p: scores requantized to
  // int16 (qk_requant16) and their maximum over the valid keys
  int32_t sc[NG];
  int32_t mx = -32768;
#pragma unroll
  for (int g = 0; g < NG; ++g) {
    int32_t d = dot[4 * g];
#pragma unroll
    for (int r = 1; r < 4; ++r)
      if (4 * g + r < NC && piece == r) d = dot[4 * g + r];
    sc[g] = qk_requant16(d, a.qk_m, a.qk_s);
    const int c = 4 * g + piece;
    if (c < NC && c * CK + kl < Tk) mx = max(mx, sc[g]);
  }
  mx = wave_max_dpp(mx);
  if (lane == 0) sm.mx[wave] = mx;
  lds_barrier();
  int32_t rowmax = sm.mx[0];
#pragma unroll
  for (int w = 1; w < NW; ++w) rowmax = max(rowmax, sm.mx[w]);

  // P = shift_exp(score - (rowmax + 1)) in int16 arithmetic, 0 past Tk; the
  // word of keys 4 (l/16) + 0..3 of chunk 4 g + (l/4) % 4 in every lane
  const uint32_t rmp1 = (uint32_t)(uint16_t)(rowmax + 1);
  uint32_t psum = 0, hi = 0;
  uint32_t pword[NG];
#pragma unroll
  for (int g = 0; g < NG; ++g) {
    const int c = 4 * g + piece;
    uint32_t p = 0;
    if (c < NC && c * CK + kl < Tk)
      p = shift_exp_one((int32_t)(int16_t)(uint16_t)((uint32_t)sc[g] - rmp1), a.frac_bits);
    psum += p;
    hi |= p;
    pword[g] = quad_bcast<0>(p) | (quad_bcast<1>(p) << 8) | (quad_bcast<2>(p) << 16) | (quad_bcast<3>(p) << 24);
  }
  // P = 128 only after an int16 row-max wrap: then the top bit is split off
  const bool whi = __any(hi & 0x80u);
  uint32_t acc[4] = {0, 0, 0, 0};
  int32_t hs[4] = {0, 0, 0, 0};
  const int src = (lane & 48) * 4;  // bpermute byte address of lane 16 (l/16)
  if (!whi) {
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const uint32_t pw = (uint32_t)__builtin_amdgcn_ds_bpermute(src + (c & 3) * 16, (int)pword[c >> 2]);
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[j] = (uint32_t)__builtin_amdgcn_sdot4((int)pw, vx[c][j], (int)acc[j], false);
    }
  } else {
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const uint32_t pw = (uint32_t)__builtin_amdgcn_ds_bpermute(src + (c & 3) * 16, (int)pword[c >> 2]);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        acc[j] = (uint32_t)__builtin_amdgcn_sdot4((int)(pw & 0x7f7f7f7fu), vx[c][j], (int)acc[j], false);
        hs[j] = __builtin_amdgcn_sdot4((int)((pw >> 7) & 0x01010101u), vx[c][j], hs[j], false);
      }
    }
  }
  // every lane's sums go to LDS; d = 4 (l % 16) + j is summed over the
  // lanes l % 16 + 16 r of every wave
  sm.part[wave * 64 + lane] = make_uint4(acc[0] + ((uint32_t)hs[0] << 7), acc[1] + ((uint32_t)hs[1] << 7),
                                         acc[2] + ((uint32_t)hs[2] << 7), acc[3] + ((uint32_t)hs[3] << 7));
  psum = wave_sum_dpp(psum);
  if (lane == 0) sm.sum[wave] = psum;
  lds_barrier();
  if (tid < 64) {
    const uint32_t *pw = reinterpret_cast<const uint32_t *>(sm.part) + (tid >> 2) * 4 + (tid & 3);
    uint32_t total = 0, pv = 0;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      total += sm.sum[w];
#pragma unroll
      for (int r = 0; r < 4; ++r) pv += pw[(w * 64 + 16 * r) * 4];
    }
    self_decode_store<NW>(a, b, h, pv, total, tid);
  }
  frag_prefetch_keep(pfv);
}

template <int NW, int NC>
__device__ __forceinline__ void self_decode_dispatch(int nc, const AttnArgs &a, int64_t b, int h, int Tk,
                                                     SelfDecodeLds<NW> &sm, const FragPrefetch &pf, int pf_start) {
  if constexpr (NC == 0) {
    // no keys: every sum is 0
    if (threadIdx.x < 64) self_decode_store<NW>(a, b, h, 0u, 0u, threadIdx.x);
  } else {
    if (nc == NC)
      self_decode_body<NW, NC>(a, b, h, Tk, sm, pf, pf_start);
    else
      self_decode_dispatch<NW, NC - 1>(nc, a, b, h, Tk, sm, pf, pf_start);
  }
}

// at most 16 NW NCMAX keys
template <int NW, int NCMAX>
__global__ __launch_bounds__(64 * NW) void attn_decode_self_kernel(AttnArgs a, const int32_t *pos, FragPrefetch pf,
                                                                    int pf_start) {
  __shared__ __attribute__((aligned(16))) SelfDecodeLds<NW> sm;
  const int64_t bh = blockIdx.x;
  const int h = (int)(bh % a.H);
  const int64_t b = bh / a.H;
  const int Tk = min(a.Tk + (pos ? *pos : 0), a.max_tk);
  const int nc = (Tk + 16 * NW - 1) / (16 * NW);
  self_decode_dispatch<NW, NCMAX>(nc, a, b, h, Tk, sm, pf, pf_start);
}

}  // namespace

int launch_qk_requant_rowmax(const int8_t *q, const int8_t *k, const uint8_t *mask, int16_t *qk,
                             int16_t *rmp1, int64_t bh, int64_t tq, int64_t tk, int64_t dim,
                             uint8_t m, int32_t shift, hipStream_t s) {
  const int64_t rows = bh * tq;
  if (rows == 0) return 0;
  hipLaunchKernelGGL(qk_requant_rowmax_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, s, q,
                     k, mask, qk, rmp1, rows, tq, tk, dim, (uint32_t)m,
                     (uint32_t)(shift > 0 ? shift : 0));
  return check_launch("qk_requant_rowmax_kernel");
}

int launch_shift_exp(const int16_t *qk, const int16_t *rmp1, const uint8_t *mask, uint8_t *p,
                     int32_t *row_sum, int64_t bh, int64_t tq, int64_t tk, int32_t f,
                     hipStream_t s) {
  const int64_t rows = bh * tq;
  if (rows == 0) return 0;
  hipLaunchKernelGGL(shift_exp_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, s, qk, rmp1,
                     mask, p, row_sum, rows, tq, tk, f);
  return check_launch("shift_exp_kernel");
}

int launch_pv_norm_requant(const uint8_t *p, const int8_t *v, const int32_t *row_sum, uint8_t av_m,
                           int8_t av_s, uint32_t off, int8_t *out, int64_t batch, int64_t heads,
                           int64_t tq, int64_t tk, int64_t dim, hipStream_t s) {
  const int64_t rows = batch * heads * tq;
  if (rows == 0) return 0;
  const int32_t as = av_s;
  hipLaunchKernelGGL(pv_norm_requant_kernel, dim3((unsigned)rows), dim3(256), 0, s, p, v, row_sum,
                     (uint32_t)av_m, (uint32_t)(as < 0 ? 0 : (as > 32 ? 32 : as)), off, out, heads,
                     tq, tk, dim);
  return check_launch("pv_norm_requant_kernel");
}

int launch_shift_exp_lut(uint8_t *lut, int32_t f, hipStream_t s) {
  hipLaunchKernelGGL(shift_exp_lut_kernel, dim3(IW_SEXP_LUT / 256), dim3(256), 0, s, lut, f);
  return check_launch("shift_exp_lut_kernel");
}

int launch_attn_prefill(const AttnArgs &a, int max_blocks, hipStream_t s) {
  const int64_t tiles = (int64_t)((a.Tq + 127) / 128) * a.H * a.B;
  if (tiles == 0) return 0;
  const unsigned grid = (unsigned)(tiles < max_blocks ? tiles : max_blocks);
  const int ks = (a.D + 31) / 32;
#define IW_PF(KS_)                                                                                 \
  if (a.mask)                                                                                      \
    hipLaunchKernelGGL((attn_prefill_kernel<KS_, true, false>), dim3(grid), dim3(256), 0, s, a);   \
  else if (a.D == 32 * (KS_))                                                                      \
    hipLaunchKernelGGL((attn_prefill_kernel<KS_, false, true>), dim3(grid), dim3(256), 0, s, a);   \
  else                                                                                             \
    hipLaunchKernelGGL((attn_prefill_kernel<KS_, false, false>), dim3(grid), dim3(256), 0, s, a);
  switch (ks) {
    case 1: IW_PF(1) break;
    case 2: IW_PF(2) break;
    case 3: IW_PF(3) break;
    case 4: IW_PF(4) break;
    default: return fail("fused attention supports head_dim <= 128");
  }
#undef IW_PF
  return check_launch("attn_prefill_kernel");
}

// the blocks blockIdx >= the returned start (a multiple of 8) of a grid of g
// blocks: the last `tail` of them, rounded up to whole XCD rounds
static int tail_start(int64_t g, int tail) {
  const int64_t st = g > tail ? (g - tail) / 8 * 8 : 0;
  return (int)st;
}

int launch_attn_decode_cross_lnq(const AttnArgs &a, const LnQueryArgs &lq, hipStream_t s) {
  if ((int64_t)a.B * a.H == 0) return 0;
  const uintptr_t al = reinterpret_cast<uintptr_t>(a.k) | reinterpret_cast<uintptr_t>(a.vt) | (uintptr_t)a.k_st |
                       (uintptr_t)a.k_sh | (uintptr_t)a.k_sb | (uintptr_t)a.v_sd | (uintptr_t)a.v_sh |
                       (uintptr_t)a.v_sb | reinterpret_cast<uintptr_t>(lq.wq);
  if (a.D != 64 || (al & 15) != 0 || a.v_sq != 4 || a.max_tk != a.Tk || a.Tk > 2048 || lq.hidden != a.H * 64 ||
      lq.hidden > 1280 || lq.kp > 1280 || lq.code < 0)
    return fail("the fused cross-attention takes head_dim 64, V transposed, at most 2048 keys and 1280 channels");
  hipLaunchKernelGGL(attn_decode_cross_lnq_kernel, dim3((unsigned)(a.B * a.H)), dim3(256), 0, s, a, lq);
  return check_launch("attn_decode_cross_lnq_kernel");
}

int launch_attn_decode_cache(const AttnArgs &a, const int32_t *pos, hipStream_t s, const FragPrefetch *tail) {
  if ((int64_t)a.B * a.H == 0) return 0;
  // a set is one 16-key chunk of V^T per lane, 1024 keys per wave; up to two
  // sets are loaded into registers before the scores are computed
  const int sets = ((a.max_tk + 15) / 16 + 63) / 64;
  const dim3 grid((unsigned)(a.B * a.H));
  // head_dim 64 with 16-byte key rows and V^T rows: the streaming kernel
  const bool vq = a.v_sq != 4;  // V in key quads
  const uintptr_t al = reinterpret_cast<uintptr_t>(a.k) | reinterpret_cast<uintptr_t>(a.vt) |
                       reinterpret_cast<uintptr_t>(a.q) | (uintptr_t)a.k_st | (uintptr_t)a.k_sh |
                       (uintptr_t)a.k_sb | (uintptr_t)(vq ? a.v_sq : a.v_sd) | (uintptr_t)a.v_sh |
                       (uintptr_t)a.v_sb | (uintptr_t)a.q_sb;
  if (a.D == 64 && (al & 15) == 0 && a.max_tk <= DC_MAX_TK) {
    // (self-attention caches up to 512 positions get their own, smaller
    // instance, so profiles separate it from cross-attention)
#define IW_DS(VQ_)                                                                                             \
  if (a.max_tk <= 512)                                                                                         \
    hipLaunchKernelGGL((attn_decode_stream_kernel<512, IW_DSS_NR, IW_DSS_CH, IW_DSS_NW, VQ_>), grid,            \
                       dim3(64 * IW_DSS_NW), 0, s, a, pos);                                                    \
  else if (a.max_tk <= 2048)                                                                                   \
    hipLaunchKernelGGL((attn_decode_stream_kernel<2048, IW_DS_NR, IW_DS_CH, 4, VQ_>), grid, dim3(256), 0, s, a, \
                       pos);                                                                                   \
  else                                                                                                         \
    hipLaunchKernelGGL((attn_decode_stream_kernel<DC_MAX_TK, IW_DS_NR, IW_DS_CH, 4, VQ_>), grid, dim3(256), 0, \
                       s, a, pos);
    // (32-bit offsets inside a head's K rows and V quads)
    const bool off32 = (int64_t)a.max_tk * a.k_st < (1ll << 31) && (int64_t)(a.max_tk + 3) / 4 * a.v_sq < (1ll << 31);
    if (vq && a.max_tk <= 16 * IW_DSELF_NW * 8 && off32) {
      // self-attention caches: every load in flight at once; the last
      // kSelfTailBlocks blocks read the next GEMM's weight into L2
      FragPrefetch tpf = tail ? *tail : FragPrefetch();
      const int tstart = tail_start(grid.x, kSelfTailBlocks);
      frag_prefetch_launch(tpf, grid.x - tstart, 64 * IW_DSELF_NW);
      const int ncmax = (a.max_tk + 16 * IW_DSELF_NW - 1) / (16 * IW_DSELF_NW);
      if (ncmax <= 2)
        hipLaunchKernelGGL((attn_decode_self_kernel<IW_DSELF_NW, 2>), grid, dim3(64 * IW_DSELF_NW), 0, s, a, pos,
                           tpf, tstart);
      else if (ncmax <= 4)
        hipLaunchKernelGGL((attn_decode_self_kernel<IW_DSELF_NW, 4>), grid, dim3(64 * IW_DSELF_NW), 0, s, a, pos,
                           tpf, tstart);
      else if (ncmax <= 7)
        hipLaunchKernelGGL((attn_decode_self_kernel<IW_DSELF_NW, 7>), grid, dim3(64 * IW_DSELF_NW), 0, s, a, pos,
                           tpf, tstart);
      else
        hipLaunchKernelGGL((attn_decode_self_kernel<IW_DSELF_NW, 8>), grid, dim3(64 * IW_DSELF_NW), 0, s, a, pos,
                           tpf, tstart);
      return check_launch("attn_decode_self_kernel");
    }
    if (vq) {
      IW_DS(true)
    } else {
      IW_DS(false)
    }
#undef IW_DS
    return check_launch("attn_decode_stream_kernel");
  }
  if (vq) return fail("V in key quads needs head_dim 64 and 16-byte aligned operands");
#define IW_DC(D_, P_) hipLaunchKernelGGL((attn_decode_cache_kernel<D_, P_>), grid, dim3(256), 0, s, a, pos)
  switch (a.D) {
    case 64:
      if (sets <= 1) IW_DC(64, 1); else IW_DC(64, 2);
      break;
    case 96:
      IW_DC(96, 1);
      break;
    case 128:
      IW_DC(128, 1);
      break;
    default:
      return fail("decode attention supports head_dim 64, 96 and 128");
  }
#undef IW_DC
  return check_launch("attn_decode_cache_kernel");
}

int launch_attn_decode(const AttnArgs &a, hipStream_t s) {
  if ((int64_t)a.B * a.H * a.Tq == 0) return 0;
  if (a.Tk > DEC_MAX_TK) return fail("decode attention supports at most 4096 keys");
  // head_dim 64, no mask, 16-byte aligned operands, at most 2048 keys: the
  // streaming kernel, the query positions of a head sharing its K/V stream
  const uintptr_t al = reinterpret_cast<uintptr_t>(a.k) | reinterpret_cast<uintptr_t>(a.vt) |
                       reinterpret_cast<uintptr_t>(a.q) | (uintptr_t)a.k_st | (uintptr_t)a.k_sh |
                       (uintptr_t)a.k_sb | (uintptr_t)a.v_sd | (uintptr_t)a.v_sh | (uintptr_t)a.v_sb |
                       (uintptr_t)a.q_sb | (uintptr_t)a.q_st;
  if (a.D == 64 && !a.mask && (al & 15) == 0 && a.Tk <= 2048 && a.v_sq == 4) {
    AttnArgs c = a;
    c.max_tk = a.Tk;
    c.o_frag_kp = 0;
    const dim3 grid((unsigned)(a.B * a.H));
#define IW_DQ(NQ_) \
  hipLaunchKernelGGL((attn_decode_stream_kernel<2048, IW_DS_NR, IW_DS_CH, 4, false, NQ_>), grid, dim3(256), 0, s, c, \
                     nullptr)
    if (a.Tq <= 2)
      IW_DQ(2);
    else if (a.Tq <= 4)
      IW_DQ(4);
    else
      IW_DQ(8);
#undef IW_DQ
    return check_launch("attn_decode_stream_kernel");
  }
  hipLaunchKernelGGL(attn_decode_kernel, dim3((unsigned)(a.B * a.H), (unsigned)a.Tq), dim3(256), 0,
                     s, a);
  return check_launch("attn_decode_kernel");
}

}  // namespace iw
