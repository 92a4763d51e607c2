// Argument block for the int8 MFMA GEMM (see iw_gemm.hip).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace iw {

enum GemmEpi : int {
  EPI_L8 = 0,      // Linear8 requant (per-channel mult/shift), optional GeLU
  EPI_L32 = 1,     // Linear32: mulh << shift -> int32
  EPI_L32RES = 2,  // Linear32 then residual15 -> int16
  EPI_S8 = 3,      // per-tensor requant with shift clamped at 0 (classifier, conv),
                   // optional GeLU, optional positional add_requant15 -> int16
};

enum GemmOut : int { OUT_ROW = 0, OUT_NCT = 1 };

// The fragment-major weight of the decode GEMM that runs after the current
// kernel (layout: frag_offset below). Its column tile t is the tile_bytes =
// 32 * Kp contiguous bytes at w + t * tile_bytes, and gemm_frag_kernel reads
// it only on the XCD of blockIdx t % 8 (blocks are dealt round-robin over
// the 8 XCDs). A kernel given one reads, on each XCD, the tiles that XCD's
// GEMM blocks will read, so that they come from its L2 rather than HBM.
// A hint: no result depends on it.
struct FragPrefetch {
  const int8_t *w = nullptr;
  int64_t tile_bytes = 0;
  int tiles = 0;
  // the launch that reads them: its grid and block sizes
  // (frag_prefetch_launch fills them in)
  int blocks = 0, threads = 0;
};

struct GemmArgs {
  // A operand
  const int8_t *a = nullptr;
  int64_t lda = 0;
  // implicit-GEMM conv geometry (A = conv input)
  int64_t conv_tin = 0, conv_cin = 0, conv_stride = 1, conv_pad = 0, conv_tout = 1, conv_ksize = 1;
  // B operand [N][K]
  const int8_t *b = nullptr;
  int64_t ldb = 0;
  int64_t M = 0, N = 0, K = 0;
  int epi = EPI_L8;
  // epilogue parameters
  const int32_t *bias = nullptr;
  const int8_t *wz = nullptr;
  const uint32_t *mult = nullptr;
  const int8_t *shift = nullptr;
  int mult_pc = 1;  // multiplier/shift per output channel (else one value)
  uint32_t scalar_mult = 0;  // used when mult == nullptr
  int8_t scalar_shift = 0;   // used when shift == nullptr
  // fused GeLU (lut != nullptr enables it)
  const uint8_t *lut = nullptr;
  const uint8_t *luti_m = nullptr;
  const int8_t *luti_s = nullptr;
  const uint8_t *luto_m = nullptr;
  const int8_t *luto_s = nullptr;
  int luti_pc = 0, luto_pc = 0;
  // fused residual15
  const int16_t *res = nullptr;
  int64_t ldres = 0;
  uint32_t res_mult = 0;
  // fused positional add_requant15 (pe != nullptr enables it; pe is [pe_T][N])
  const int8_t *pe = nullptr;
  const uint16_t *pe_mult = nullptr;
  const int8_t *pe_shift = nullptr;
  int pe_mpc = 0, pe_spc = 0;
  int64_t pe_T = 1;
  // output
  void *out = nullptr;
  int64_t ldc = 0;
  int64_t out_T = 1;  // OUT_NCT: rows are (b, t) with t in [0, out_T)
  // the next decode GEMM's weight, read into L2 (gemm_frag_kernel only)
  FragPrefetch pf;
  // per-tensor int8 epilogue (classifier) only, gemm_frag_kernel: the first
  // maximum of each row within each 32-column tile, amax[m * amax_ld + tile]
  // = (y + 128) << 5 | (31 - column in tile); out may then be null
  uint16_t *amax = nullptr;
  int64_t amax_ld = 0;
};

// Decode-step QKV projection: the epilogue writes Q (columns [0, C)) to
// q[m][n], and appends K / V (columns [C, 2C) / [2C, 3C), head h = c / D,
// d = c % D) of row m = b * T + i at cache position t = *pos + i:
// K to k[b*k_sb + h*k_sh + t*k_st + d], V to
// v[b*v_sb + h*v_sh + d*v_sd + (t/4)*v_sq + t%4] (v_sq = 4: V transposed per
// head; v_sd = 4, v_sq = 4 D: key quads, one step's V of a head in 4 D bytes).
struct SkinnyScatter {
  int8_t *q = nullptr;
  int64_t ldq = 0;
  int8_t *k = nullptr;
  int64_t k_sb = 0, k_sh = 0, k_st = 0;
  int8_t *v = nullptr;
  int64_t v_sb = 0, v_sh = 0, v_sd = 0, v_sq = 4;
  int C = 0, D = 1, T = 1;
  int t_cap = 0;  // cache positions; appends at t >= t_cap are dropped
  const int32_t *pos = nullptr;
};

// Rows up to which the decode kernel (iw_gemm_skinny.hip) is used, and up to
// which it runs over 128-row chunks.
constexpr int64_t kSkinnyMaxRows = 128;
#ifndef IW_SKINNY_CHUNK_ROWS
#define IW_SKINNY_CHUNK_ROWS 512
#endif
constexpr int64_t kSkinnyChunkMaxRows = IW_SKINNY_CHUNK_ROWS;
bool gemm_skinny_eligible(const GemmArgs &g);
int gemm_skinny(const GemmArgs &g, const SkinnyScatter *scatter, hipStream_t s);

// Fragment-major operands of the one-token decode GEMMs (iw_gemm_frag.hip).
// An int8 matrix X[R][K] is stored as [R/32][Kp/32][64][16]: block (i, s)
// is the 1 KB register image of the v_mfma_i32_32x32x32_i8 operand for rows
// 32i .. 32i+31 and k = 32s .. 32s+31, lane l holding row 32i + l % 32,
// bytes k = 32s + 16 (l / 32) .. +15. R is padded to a multiple of 32 and K
// to Kp = a multiple of 320 (frag_kpad); the padding holds zeros, which add
// nothing to a product or a row sum.
constexpr int64_t kFragMaxK = 5120;

__host__ __device__ inline int64_t frag_kpad(int64_t k) { return (k + 319) / 320 * 320; }
__host__ __device__ inline int64_t frag_rpad(int64_t r) { return (r + 31) / 32 * 32; }
__host__ __device__ inline int64_t frag_offset(int64_t r, int64_t k, int64_t kp) {
  return (r >> 5) * 32 * kp + (k >> 5) * 1024 + ((r & 31) + ((k >> 4) & 1) * 32) * 16 + (k & 15);
}

// Fills in the launch geometry of a prefetch (grid and block size).
inline void frag_prefetch_launch(FragPrefetch &p, int64_t blocks, int threads) {
  p.blocks = (int)blocks;
  p.threads = threads;
}

// NL dword loads per thread, one per 64 bytes of the column tiles that the
// next GEMM reads on this block's XCD (XCD blockIdx % 8), spread over this
// launch's blocks on that XCD; lines beyond NL per thread are left to HBM.
// The loads are unconditional, so that the compiler counts them and its
// waits for the kernel's own (earlier) loads leave them in flight: a lane
// with no line to fetch, or a launch with no hint, reads `fallback` (an
// address the kernel reads anyway). Pass v to frag_prefetch_keep at the end.
// The launch geometry comes from p (kernel arguments), not from the
// dispatch packet, whose read would be a vector-memory wait of its own.
// blk: this block's index among the launch's prefetching blocks (blockIdx
// less a multiple of 8, so that blk % 8 is still its XCD); none when !part.
template <int NL>
__device__ inline void frag_prefetch_issue_at(const FragPrefetch &p, int blk, bool part, const void *fallback,
                                              uint32_t (&v)[NL]) {
  const int xcd = blk & 7;
  const bool on = part && p.w != nullptr && p.tiles > xcd;
  const uint32_t per = ((uint32_t)p.blocks - (uint32_t)xcd + 7) >> 3;      // this launch's blocks on the XCD
  const uint32_t ntx = on ? ((uint32_t)p.tiles - (uint32_t)xcd + 7) >> 3 : 0;  // the next GEMM's tiles on it
  const uint32_t tb = (uint32_t)p.tile_bytes;                              // < 2^31 (host-checked)
  const uint32_t lpt = max(tb >> 6, 1u);                                     // 64-byte lines per tile
  const uint32_t step = per * (uint32_t)p.threads;
  const uint32_t u0 = (uint32_t)(blk >> 3) * (uint32_t)p.threads + threadIdx.x;
  // line u of the XCD's tiles = (tile t, line c): walked by `step` per load
  uint32_t t = u0 / lpt, c = u0 - t * lpt;
  const uint32_t dq = step / lpt, dr = step - dq * lpt;
  // 32-bit offsets (the whole weight is < 2^31 bytes) and selects, so that
  // no branch or 64-bit multiply sits between the loads
  const int8_t *base = on ? p.w + (uint32_t)xcd * tb : reinterpret_cast<const int8_t *>(fallback);
#pragma unroll
  for (int i = 0; i < NL; ++i) {
    const bool in = t < ntx;
    const uint32_t off = in ? 8 * t * tb + c * 64 : 0u;
    const int8_t *a = in ? base : reinterpret_cast<const int8_t *>(fallback);
    v[i] = *reinterpret_cast<const uint32_t *>(a + off);
    c += dr;
    t += dq;
    if (c >= lpt) c -= lpt, ++t;
  }
}

template <int NL>
__device__ inline void frag_prefetch_issue(const FragPrefetch &p, const void *fallback, uint32_t (&v)[NL]) {
  frag_prefetch_issue_at(p, (int)blockIdx.x, true, fallback, v);
}

// The same from the blocks blockIdx >= start (a multiple of 8) of the launch
// only, with p.blocks the number of those blocks: the last blocks of a long
// kernel read the next GEMM's weight into L2 shortly before it runs.
template <int NL>
__device__ inline void frag_prefetch_issue_tail(const FragPrefetch &p, int start, const void *fallback,
                                                uint32_t (&v)[NL]) {
  const int blk = (int)blockIdx.x - start;
  frag_prefetch_issue_at(p, blk < 0 ? 0 : blk, blk >= 0, fallback, v);
}

template <int NL>
__device__ inline void frag_prefetch_keep(const uint32_t (&v)[NL]) {
  uint32_t x = 0;
#pragma unroll
  for (int i = 0; i < NL; ++i) x ^= v[i];
  asm volatile("" ::"v"(x));
}

// a and b fragment-major with padded K = frag_kpad(K); out_frag: the int8
// output is itself written fragment-major (padded K = frag_kpad(N)).
int gemm_frag(const GemmArgs &g, const SkinnyScatter *scatter, bool out_frag, hipStream_t s);
// The classifier (EPI_S8, optionally with amax) as one persistent block per
// CU streaming the weight tiles (iw_classifier_stream.hip): M <= 128,
// Kp in {640, 960, 1280}, at least two column tiles per CU.
bool classifier_stream_eligible(const GemmArgs &g);
int classifier_stream(const GemmArgs &g, hipStream_t s);
int launch_frag_pack(const int8_t *src, int64_t rows, int64_t cols, int64_t ld, int8_t *dst, hipStream_t s);

// Rows from which the 256 x 128 tile kernel (iw_gemm_big.hip) is used.
constexpr int64_t kBigGemmMinRows = 8192;

int gemm_dense(const GemmArgs &g, hipStream_t s);
int gemm_big(const GemmArgs &g, bool conv_cl, hipStream_t s);
// Direct-to-LDS kernel (iw_gemm_dtl.hip): dense A, K % 64 == 0, 16-byte aligned.
bool gemm_dtl_eligible(const GemmArgs &g);
int gemm_dtl(const GemmArgs &g, hipStream_t s);
int gemm_conv(const GemmArgs &g, bool channels_last, hipStream_t s);

}  // namespace iw
