// One-token decode GEMMs on fragment-major operands (layout: iw_gemm.hpp,
// frag_offset): Linear8 (+GeLU, optionally writing its output
// fragment-major for the next GEMM), Linear32 + residual15, the
// self-attention QKV projection with the KV-cache append, and the
// classifier's per-tensor requant.
//
// A decode step reads every weight byte once, from HBM, with M <= 128 rows
// of activations: the MFMA work is small and the time is the latency of the
// loads. In the fragment-major layout each v_mfma_i32_32x32x32_i8 operand is
// one contiguous 1 KB piece, so a wave-wide 16-byte-per-lane load fills one
// MFMA operand register quad straight from memory with 8 whole cache lines:
// no LDS staging, no ring, no swizzle. Every wave therefore issues all of
// its loads (its share of K for both operands) with its first instructions
// and the kernel pays the memory latency once.
//
// Block = one 32 x 32 output tile (m-subtile x column tile); its K steps are
// split over NW waves of SPW k32 steps each (NW = Kp / (32 SPW)).
// The waves' partial tiles are added into one tile in LDS (ds_add), and all
// threads run the epilogue. Blocks of one column tile share blockIdx % 8,
// i.e. one XCD, so the tile's weights come from HBM once and from that XCD's
// L2 for the other m-subtiles.
#include "iw_gemm_dev.hpp"

namespace iw {

using namespace gemm;

namespace {

// Classifier epilogue with the row maxima: the int8 logit of (m, n) as
// skinny_store's per-tensor form computes it, stored when g.out is set, and
// the tile's first maximum of row m, reduced over the 32 lanes that hold the
// row's 32 columns (lanes 0-31 or 32-63 of a wave, column = lane % 32).
// Padding columns (n >= N) take key 0; every lane of the 32 takes part.
__device__ __forceinline__ void classifier_argmax_store(const GemmArgs &g, const ColParams &c, int m, int n,
                                                        int tile, bool valid, uint32_t a) {
  uint32_t key = 0;
  if (valid) {
    const int32_t y = clampi(apply_shift(mulh_su((int32_t)a, c.mult), c.shift), -127, 127);
    if (g.out) reinterpret_cast<int8_t *>(g.out)[(int64_t)m * g.ldc + n] = (int8_t)y;
    key = ((uint32_t)(y + 128) << 5) | (uint32_t)(31 - (n & 31));
  }
  // keys < 2^13: the 16-lane row maxima with DPP moves, then each 32-lane
  // half adds its second row's (lanes 16 and 48, read as scalars)
  int32_t k = (int32_t)key;
  k = max(k, __builtin_amdgcn_update_dpp(0, k, 0xB1, 0xf, 0xf, false));   // quad [1,0,3,2]
  k = max(k, __builtin_amdgcn_update_dpp(0, k, 0x4E, 0xf, 0xf, false));   // quad [2,3,0,1]
  k = max(k, __builtin_amdgcn_update_dpp(0, k, 0x141, 0xf, 0xf, false));  // row_half_mirror
  k = max(k, __builtin_amdgcn_update_dpp(0, k, 0x140, 0xf, 0xf, false));  // row_mirror
  const int lane = threadIdx.x & 63;
  const int32_t k16 = __builtin_amdgcn_readlane(k, 16), k48 = __builtin_amdgcn_readlane(k, 48);
  k = max(k, lane < 32 ? k16 : k48);
  if ((lane & 31) == 0 && m < (int)g.M) g.amax[(int64_t)m * g.amax_ld + tile] = (uint16_t)k;
}

// Each wave multiplies the block's 32 x 32 tile over SPW k32 steps; a block
// has MINW .. MAXW waves (MINW bounds the epilogue rows a thread serves).
// ARGMAX: the classifier epilogue that also writes the per-tile row maxima.
template <int EPI, bool GELU, bool SCATTER, bool OUT_FRAG, int SPW, int MAXW, int MINW, bool ARGMAX = false>
__global__ __launch_bounds__(64 * MAXW) void gemm_frag_kernel(GemmArgs g, SkinnyScatter sc, int ms, int tiles,
                                                              int kp) {
  // the waves' partial tiles are added into one tile in LDS (ds_add); row
  // stride 40 words puts the two 32-lane halves of each add (rows 4 apart)
  // on disjoint halves of the 64 banks
  constexpr int PLD = 40;
  __shared__ int32_t sTile[32 * PLD];
  __shared__ int32_t sXs[32];
  __shared__ uint8_t sLut[16];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nt = blockDim.x;
  const int bid = blockIdx.x;
  const int tile = (bid & 7) + 8 * (bid / (8 * ms));
  const int msub = (bid >> 3) % ms;
  if (tile >= tiles) return;
  const int M = (int)g.M, N = (int)g.N;
  const int m0 = msub * 32, n0 = tile * 32;

  // epilogue inputs first: in a decode step they are as cold as the weights
  // (per-layer parameters, the residual rows just written), and requested
  // behind the operands their misses would start only after the operand
  // bytes have drained. Thread t serves column t % 32 and rows
  // t / 32 + (nt / 32) j of the tile.
  const int cl = tid & 31;
  const int n = n0 + cl;
  const int mr0 = tid >> 5, mstep = nt >> 5;
  constexpr int RMAX = (32 * 32 + 64 * MINW - 1) / (64 * MINW);
  uint32_t lutv = 0;
  if (GELU && tid < 16) lutv = g.lut[tid];
  const ColRaw craw = load_col_raw(g, min(n, N - 1));
  int32_t resv[RMAX];
  if (EPI == EPI_L32RES) {
#pragma unroll
    for (int j = 0; j < RMAX; ++j) {
      const int r = mr0 + mstep * j;
      resv[j] = r < 32 ? g.res[(int64_t)min(m0 + r, M - 1) * g.ldres + min(n, N - 1)] : 0;
    }
  }
  int pos = 0;
  if (SCATTER) pos = *sc.pos;
  for (int i = tid; i < 32 * PLD; i += nt) sTile[i] = 0;
  if (tid < 32) sXs[tid] = 0;

  // then every operand load of this wave: SPW fragments of A and of B
  const int64_t kofs = (int64_t)wave * SPW * 1024 + lane * 16;
  const int8_t *pa = g.a + (int64_t)msub * 32 * kp + kofs;
  const int8_t *pb = g.b + (int64_t)tile * 32 * kp + kofs;
  v4i fa[SPW], fb[SPW];
#pragma unroll
  for (int t = 0; t < SPW; ++t) {
    fa[t] = *reinterpret_cast<const v4i *>(pa + t * 1024);
    fb[t] = *reinterpret_cast<const v4i *>(pb + t * 1024);
  }
  // FC1 (the GeLU instances) reads FC2's weight tiles into L2 behind its own
  // operands, when given them: 1 line per thread covers 2.5 MB per XCD with
  // 128 rows of Whisper-large (FC2's weight share is 0.8 MB). The GEMMs
  // before an attention kernel take no hint: the K/V stream evicts the lines
  // before the GEMM after it runs.
  constexpr bool PF = GELU;
  uint32_t pfv[1];
  if constexpr (PF) {
    frag_prefetch_issue(g.pf, pb, pfv);
    // issued here, with the operands, not sunk below the MFMAs: the wait
    // after the partial-tile barrier below covers every load
    __builtin_amdgcn_sched_barrier(0);
  }

  // the zeroed tile is seen by every wave before any adds into it (an LDS-only
  // barrier: the operand loads stay in flight)
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");

  // two accumulator chains so that consecutive MFMAs do not wait on each
  // other; row sums of A for the zero-point term from the same registers
  v16i acc[2];
#pragma unroll
  for (int r = 0; r < 16; ++r) acc[0][r] = acc[1][r] = 0;
  int32_t xs = 0;
#pragma unroll
  for (int t = 0; t < SPW; ++t) {
    acc[t & 1] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[t], fb[t], acc[t & 1], 0, 0, 0);
    xs = sum16v(fa[t], xs);
  }

  // this wave's partial tile added into sTile[row][PLD] (sums modulo 2^32,
  // in any order). 32x32 MFMA layout: lane l holds column l % 32, register r
  // row (r / 4) * 8 + (l / 32) * 4 + r % 4.
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int row = (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
    atomicAdd(&sTile[row * PLD + (lane & 31)], (int32_t)((uint32_t)acc[0][r] + (uint32_t)acc[1][r]));
  }
  atomicAdd(&sXs[lane & 31], xs);  // lanes l and l + 32 hold halves of row l % 32
  if (GELU && tid < 16) sLut[tid] = (uint8_t)lutv;
  __syncthreads();

  if constexpr (ARGMAX) {
    // all lanes stay for the cross-lane row maxima; a row's 32 columns are
    // the 32 threads sharing tid / 32
    const ColParams c = decode_col<EPI>(g, craw);
#pragma unroll
    for (int j = 0; j < RMAX; ++j) {
      const int r = mr0 + mstep * j;
      const int m = m0 + r;
      if (r < 32) {  // uniform over each 32-thread group
        classifier_argmax_store(g, c, m, n, tile, n < N && m < M, (uint32_t)sTile[r * PLD + cl]);
      }
    }
    return;
  }
  if (n >= N) {
    if constexpr (PF) frag_prefetch_keep(pfv);
    return;
  }
  const bool zp = g.wz != nullptr;
  const ColParams c = decode_col<EPI>(g, craw);
#pragma unroll
  for (int j = 0; j < RMAX; ++j) {
    const int r = mr0 + mstep * j;
    const int m = m0 + r;
    if (r < 32 && m < M) {
      skinny_store<EPI, GELU, SCATTER, OUT_FRAG>(g, sc, c, sLut, pos, m, n,
                                                 corrected_k32k(sTile[r * PLD + cl], zp ? sXs[r] : 0, c),
                                                 EPI == EPI_L32RES ? resv[j] : 0);
    }
  }
  if constexpr (PF) frag_prefetch_keep(pfv);
}

template <int EPI, bool GELU, bool SCATTER, bool OUT_FRAG, int SPW, int MAXW, int MINW, bool ARGMAX = false>
int launch_frag_waves(const GemmArgs &g, const SkinnyScatter &sc, int64_t kp, hipStream_t s) {
  const int64_t tiles = (g.N + 31) / 32;
  const int ms = (int)((g.M + 31) / 32);
  const int nw = (int)(kp / (32 * SPW));
  const dim3 grid((unsigned)(((tiles + 7) / 8) * 8 * ms));
  GemmArgs ga = g;
  frag_prefetch_launch(ga.pf, grid.x, 64 * nw);
  hipLaunchKernelGGL((gemm_frag_kernel<EPI, GELU, SCATTER, OUT_FRAG, SPW, MAXW, MINW, ARGMAX>), grid, dim3(64 * nw),
                     0, s, ga, sc, ms, (int)tiles, (int)kp);
  return check_launch("gemm_frag_kernel");
}

// Waves per block: the more waves the machine holds at once, the more of the
// weights are in flight, so K is cut into as many wave shares as the block
// size allows: 5 k32 steps per wave up to Kp = 1280 (<= 8 waves), 10 above
// (5 .. 16 waves).
template <int EPI, bool GELU, bool SCATTER, bool OUT_FRAG, bool ARGMAX = false>
int launch_frag(const GemmArgs &g, const SkinnyScatter &sc, hipStream_t s) {
  const int64_t kp = frag_kpad(g.K);
  if (kp <= 1280) return launch_frag_waves<EPI, GELU, SCATTER, OUT_FRAG, 5, 8, 2, ARGMAX>(g, sc, kp, s);
  if (kp <= 2560) return launch_frag_waves<EPI, GELU, SCATTER, OUT_FRAG, 10, 8, 5, ARGMAX>(g, sc, kp, s);
  return launch_frag_waves<EPI, GELU, SCATTER, OUT_FRAG, 10, 16, 9, ARGMAX>(g, sc, kp, s);
}

// Row-major [rows][cols] (leading dimension ld) to fragment-major with
// zero padding: one thread per 16-byte piece of the destination.
__global__ __launch_bounds__(256) void frag_pack_kernel(const int8_t *__restrict__ src, int64_t rows, int64_t cols,
                                                        int64_t ld, int8_t *__restrict__ dst, int64_t kp,
                                                        int64_t pieces) {
  const int64_t p = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (p >= pieces) return;
  const int64_t off = p * 16;
  const int64_t blk = off >> 10, l = (off >> 4) & 63;
  const int64_t steps = kp >> 5;
  const int64_t r = (blk / steps) * 32 + (l & 31);
  const int64_t k0 = (blk % steps) * 32 + (l >> 5) * 16;
  uint32_t w[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    uint32_t v = 0;
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const int64_t k = k0 + 4 * q + b;
      const uint32_t byte = (r < rows && k < cols) ? (uint8_t)src[r * ld + k] : 0u;
      v |= byte << (8 * b);
    }
    w[q] = v;
  }
  *reinterpret_cast<uint4 *>(dst + off) = make_uint4(w[0], w[1], w[2], w[3]);
}

}  // namespace

int gemm_frag(const GemmArgs &g, const SkinnyScatter *scatter, bool out_frag, hipStream_t s) {
  if (g.M == 0) return 0;
  const bool gelu = g.lut != nullptr;
  SkinnyScatter sc;
  if (scatter) {
    if (g.epi != EPI_L8 || gelu || out_frag) return fail("the KV-cache epilogue is for the Linear8 QKV projection");
    sc = *scatter;
    return launch_frag<EPI_L8, false, true, false>(g, sc, s);
  }
  if (out_frag && g.epi != EPI_L8) return fail("a fragment-major output is int8 (Linear8)");
  switch (g.epi) {
    case EPI_L8:
      if (out_frag) {
        if (gelu) return launch_frag<EPI_L8, true, false, true>(g, sc, s);
        return launch_frag<EPI_L8, false, false, true>(g, sc, s);
      }
      if (gelu) return launch_frag<EPI_L8, true, false, false>(g, sc, s);
      return launch_frag<EPI_L8, false, false, false>(g, sc, s);
    case EPI_L32RES: return launch_frag<EPI_L32RES, false, false, false>(g, sc, s);
    case EPI_S8: {
      if (gelu || out_frag) return fail("the fragment-major classifier has a plain per-tensor epilogue");
      if (classifier_stream_eligible(g)) return classifier_stream(g, s);
      if (g.amax) return launch_frag<EPI_S8, false, false, false, true>(g, sc, s);
      return launch_frag<EPI_S8, false, false, false>(g, sc, s);
    }
    default: return fail("the fragment-major GEMM has Linear8, Linear32 + residual15 and classifier epilogues");
  }
}

int launch_frag_pack(const int8_t *src, int64_t rows, int64_t cols, int64_t ld, int8_t *dst, hipStream_t s) {
  const int64_t pieces = frag_rpad(rows) * frag_kpad(cols) / 16;
  if (pieces == 0) return 0;
  hipLaunchKernelGGL(frag_pack_kernel, dim3((unsigned)((pieces + 255) / 256)), dim3(256), 0, s, src, rows, cols, ld,
                     dst, frag_kpad(cols), pieces);
  return check_launch("frag_pack_kernel");
}

}  // namespace iw
