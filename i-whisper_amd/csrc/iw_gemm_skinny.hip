// Skinny int8 GEMM for the decoder (M = batch rows <= 128): Linear8 (+GeLU),
// Linear32 (+residual15), classifier, and the self-attention QKV projection
// whose epilogue writes Q to a buffer and appends K and V to the KV caches.
//
// A decode GEMM reads every weight byte once; with M <= 128 the MFMA work is
// small and the time goes into moving operands. Each block owns one 32-column
// tile of the output and all of K, so it reads the whole A operand (M x K,
// L2-resident) and its own 32 weight rows: the per-CU load path, not HBM,
// bounds it, and what matters is how many cache lines each wave-wide load
// touches. Two kernels:
//
// * gemm_skinny_lds_kernel (K % 128 == 0, 16-byte aligned rows): operands
//   move global -> LDS with global_load_lds_dwordx4 in 128-byte K stages
//   through a 3-stage ring; every wave-wide copy reads 8 rows x 128 bytes,
//   i.e. 8 whole cache lines. Wave w < MS multiplies m-subtile w (32 rows)
//   by the 32 columns over all of K, reading its v_mfma_i32_32x32x32_i8
//   fragments from LDS, and applies the epilogue from registers.
// * gemm_skinny_kernel (any K % 16 == 0): fragments are loaded straight from
//   global memory into registers (32 rows x 32 bytes per wave-wide load),
//   eight waves split M and K, and the K slices are added in LDS.
#include "iw_gemm_dev.hpp"

namespace iw {

using namespace gemm;

namespace {

constexpr int TN = 32;    // output columns per block

// ---------------------------------------------------------------------------
// LDS-staged kernel
// ---------------------------------------------------------------------------

constexpr int LNT = 256;   // 4 waves
constexpr int SK = 128;    // K bytes per stage (one LDS row)

// One 16-byte global -> LDS copy per lane (global_load_lds_dwordx4): the wave
// writes 1 KB at LDS byte address `lds` (lane l at lds + 16 l). Issued as
// inline assembly so that the compiler adds no waits for it; the loop waits
// on vmcnt itself. No kernel using it keeps a value in M0.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void dma16(const int8_t *src, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(lds)
               : "memory", "m0");
}
#pragma clang diagnostic pop

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// LDS rows are 128 bytes (8 chunks of 16); chunk c of row r sits at position
// c ^ swz8(r). A fragment read (16 consecutive lanes = 16 consecutive rows,
// one logical chunk) then covers every (row parity, position) pair once, so
// the 16 lanes of each ds_read_b128 pass hit distinct banks.
__device__ __forceinline__ int swz8(int r) { return (r >> 1) & 7; }

// SST stages in the ring, SST - 1 of them in flight while one is consumed:
// a CU's load rate is bytes in flight / latency, so a grid with one block per
// CU takes a deep ring (most of the LDS) and a larger grid a shallow one that
// lets blocks share a CU.
template <int EPI, bool GELU, bool SCATTER, int MS, int SST>
__global__ __launch_bounds__(LNT) void gemm_skinny_lds_kernel(GemmArgs g, SkinnyScatter sc) {
  constexpr int A_ST = MS * 32 * SK, B_ST = TN * SK;
  constexpr int DMA_PER_WAVE = MS + 1;  // copies one wave issues per stage
  __shared__ __attribute__((aligned(1024))) int8_t sA[SST * A_ST];
  __shared__ __attribute__((aligned(1024))) int8_t sB[SST * B_ST];
  __shared__ int32_t sXs[MS * 32];
  __shared__ uint8_t sLut[16];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int M = (int)g.M, N = (int)g.N, K = (int)g.K;
  const int n0 = blockIdx.x * TN;
  const bool zp = g.wz != nullptr;
  // the GeLU table goes to LDS after the K loop; only its load is issued now
  uint32_t lutv = 0;
  if (GELU && tid < 16) lutv = g.lut[tid];

  // Copy j of a stage (A: j < 4 MS, B: j < 4) fills LDS rows 8j .. 8j+7;
  // lane l writes row 8j + l/8 at position l % 8 and so fetches chunk
  // (l % 8) ^ swz8(row). Wave w issues A copies w, w + 4, ... and B copy w.
  // Rows past the matrix edge read its last row (their results are never
  // stored).
  const int8_t *ga[MS];
#pragma unroll
  for (int i = 0; i < MS; ++i) {
    const int r = (wave + 4 * i) * 8 + (lane >> 3);
    ga[i] = g.a + (int64_t)min(r, M - 1) * g.lda + ((lane & 7) ^ swz8(r)) * 16;
  }
  const int rb = wave * 8 + (lane >> 3);
  const int8_t *gb = g.b + (int64_t)min(n0 + rb, N - 1) * g.ldb + ((lane & 7) ^ swz8(rb)) * 16;
  const uint32_t ldsA = __builtin_amdgcn_readfirstlane((uint32_t)reinterpret_cast<uintptr_t>(sA));
  const uint32_t ldsB = __builtin_amdgcn_readfirstlane((uint32_t)reinterpret_cast<uintptr_t>(sB));
  auto issue = [&](int kt) {
    const int st = kt % SST;
    const int k0 = kt * SK;
#pragma unroll
    for (int i = 0; i < MS; ++i) dma16(ga[i] + k0, ldsA + st * A_ST + (wave + 4 * i) * 1024);
    dma16(gb + k0, ldsB + st * B_ST + wave * 1024);
  };

  // The epilogue's inputs (column parameters, residual, cache position) are
  // requested first, so their latency is spent under the K loop.
  // (Rows and columns past the edge read the last ones: no branches, so the
  // compiler can count these loads instead of waiting for all of them.)
  const bool active = wave < MS;
  const int n = n0 + (lane & 31);
  ColRaw craw;
  int32_t resv[16];
  int pos = 0;
  if (active) {
    craw = load_col_raw(g, min(n, N - 1));
    if (EPI == EPI_L32RES) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = min(wave * 32 + (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3), M - 1);
        resv[r] = g.res[(int64_t)m * g.ldres + min(n, N - 1)];
      }
    }
    if (SCATTER) pos = *sc.pos;
  }

  // this wave's copies of all but the newest `later` issued stages have landed
  auto wait_stages = [&](int later) {
    if (SST >= 6 && later >= 4)
      wait_vmcnt<4 * DMA_PER_WAVE>();
    else if (SST >= 5 && later >= 3)
      wait_vmcnt<3 * DMA_PER_WAVE>();
    else if (SST >= 4 && later >= 2)
      wait_vmcnt<2 * DMA_PER_WAVE>();
    else if (later >= 1)
      wait_vmcnt<DMA_PER_WAVE>();
    else
      wait_vmcnt<0>();
  };
  // after this wave's LDS reads have completed, every wave's landed copies
  // become visible to all (no release fence: it would drain the copies)
  auto sync = [&]() {
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  };
  // fragment reads: lane l reads row l % 32 of the subtile, logical chunk
  // 2 ks + l / 32 of the stage
  const int sw = swz8(lane & 31);
  // (waves past the m-subtiles recompute subtile 0 and store nothing: the
  // loop then has no branch, which would move the accumulator out of AGPRs
  // every iteration)
  const int aoff = ((active ? wave * 32 : 0) + (lane & 31)) * SK;
  const int boff = (lane & 31) * SK;
  auto read_frags = [&](int kt, v4i *fa, v4i *fb) {
    const int8_t *pa = &sA[(kt % SST) * A_ST + aoff];
    const int8_t *pb = &sB[(kt % SST) * B_ST + boff];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const int p = ((2 * ks + (lane >> 5)) ^ sw) * 16;
      fa[ks] = *reinterpret_cast<const v4i *>(pa + p);
      fb[ks] = *reinterpret_cast<const v4i *>(pb + p);
    }
  };

  // Software pipeline: while the MFMAs consume stage kt from registers, the
  // fragments of stage kt + 1 are read from LDS and stages up to kt + SST - 1
  // are being copied in. Stage kt + SST - 1 overwrites the buffer of stage
  // kt - 1, whose fragments every wave has consumed before the barrier.
  const int nk = K / SK;
#pragma unroll
  for (int i = 0; i < SST - 1; ++i)
    if (i < nk) issue(i);
  wait_stages(min(SST - 2, nk - 1));
  sync();
  // two accumulators, so that consecutive MFMAs do not wait on each other
  v16i acc, acc2;
#pragma unroll
  for (int r = 0; r < 16; ++r) acc[r] = acc2[r] = 0;
  int32_t xs = 0;
  v4i fa[4], fb[4];
  read_frags(0, fa, fb);
  for (int kt = 0; kt < nk; ++kt) {
    v4i na[4], nb[4];
    if (kt + 1 < nk) {
      wait_stages(min(SST - 3, nk - 2 - kt));
      sync();
      if (kt + SST - 1 < nk) issue(kt + SST - 1);
      read_frags(kt + 1, na, nb);
    }
#pragma unroll
    for (int ks = 0; ks < 4; ks += 2) {
      acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[ks], fb[ks], acc, 0, 0, 0);
      acc2 = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[ks + 1], fb[ks + 1], acc2, 0, 0, 0);
    }
    if (zp) {
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) xs = sum16v(fa[ks], xs);
    }
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      fa[ks] = na[ks];
      fb[ks] = nb[ks];
    }
  }
#pragma unroll
  for (int r = 0; r < 16; ++r) acc[r] = (int32_t)((uint32_t)acc[r] + (uint32_t)acc2[r]);
  if (zp && active) {
    xs += __shfl_xor(xs, 32);
    if (lane < 32) sXs[wave * 32 + lane] = xs;
  }
  if (GELU && tid < 16) sLut[tid] = (uint8_t)lutv;
  __syncthreads();
  if (!active) return;

  // Epilogue from registers. 32x32 MFMA layout: lane l holds column l % 32
  // and, for register r, row (r / 4) * 8 + (l / 32) * 4 + (r % 4).
  if (n >= N) return;
  const ColParams c = decode_col<EPI>(g, craw);
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int m = wave * 32 + (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
    if (m < M) {
      const uint32_t a = corrected_k32k(acc[r], zp ? sXs[m] : 0, c);
      skinny_store<EPI, GELU, SCATTER>(g, sc, c, sLut, pos, m, n, a, EPI == EPI_L32RES ? resv[r] : 0);
    }
  }
}

// ---------------------------------------------------------------------------
// M-split kernel: one 32-row m-subtile x 32 NS columns per block
// ---------------------------------------------------------------------------
//
// For decode grids each block takes one 32 x (32 NS) output tile over all of
// K, so it copies 32 x K bytes of A and 32 NS x K of B instead of M x K of A.
// Stage s (128 K bytes: 4 KB of A, 4 NS KB of B) belongs to wave s % 4, which
// copies it into its own LDS ring, reads its fragments back and runs its MFMAs:
// the four waves are independent pipelines with no barrier in the K loop.
// Their partial tiles are added in LDS (the rings' space) at the end. The
// blocks of one column tile share blockIdx % 8, i.e. one XCD, so its B rows
// come from HBM once. NS = 2 halves the A bytes every column of a wide GEMM
// costs (A is re-read once per column tile).
template <int EPI, bool GELU, bool SCATTER, int WST, int NS>
__global__ __launch_bounds__(LNT) void gemm_skinny_msplit_kernel(GemmArgs g, SkinnyScatter sc, int ms,
                                                                 int tiles) {
  constexpr int STB = 4096 * (1 + NS);  // bytes per stage: A rows then B rows, 128 bytes each
  constexpr int CPB = 32 * NS;          // columns per block
  constexpr int PLDM = CPB + 1;
  constexpr int DMA_STAGE = 4 + 4 * NS;  // copies per stage
  constexpr int RPT = CPB / 8;           // epilogue rows per thread
  static_assert(4 * 32 * PLDM * 4 <= WST * 4 * STB, "partials must fit the rings");
  __shared__ __attribute__((aligned(1024))) int8_t sRing[4 * WST * STB];
  __shared__ int32_t sXs[4][32];
  __shared__ uint8_t sLut[16];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int bid = blockIdx.x;
  const int tile = (bid & 7) + 8 * (bid / (8 * ms));
  const int msub = (bid >> 3) % ms;
  if (tile >= tiles) return;
  const int M = (int)g.M, N = (int)g.N, K = (int)g.K;
  const int n0 = tile * CPB, m0 = msub * 32;
  const bool zp = g.wz != nullptr;

  // epilogue inputs, requested before the K loop: thread t serves column
  // t % CPB and rows t / CPB + (256 / CPB) j of the subtile
  const int cl = tid % CPB;
  const int n = n0 + cl;
  const int mr0 = tid / CPB;
  uint32_t lutv = 0;
  if (GELU && tid < 16) lutv = g.lut[tid];
  const ColRaw craw = load_col_raw(g, min(n, N - 1));
  int32_t resv[RPT];
  if (EPI == EPI_L32RES) {
#pragma unroll
    for (int j = 0; j < RPT; ++j)
      resv[j] = g.res[(int64_t)min(m0 + mr0 + (256 / CPB) * j, M - 1) * g.ldres + min(n, N - 1)];
  }
  int pos = 0;
  if (SCATTER) pos = *sc.pos;

  // copy j of a stage fills rows 8 (j % 4) .. +7 of A (j < 4) or rows
  // 8 (j - 4) .. +7 of B; lane l writes row r = 8 (.) + l / 8 at position
  // l % 8, fetching chunk (l % 8) ^ swz8(r)
  const int r8 = lane >> 3;
  const int8_t *ga[4];
  const int8_t *gb[4 * NS];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int r = 8 * j + r8;
    ga[j] = g.a + (int64_t)min(m0 + r, M - 1) * g.lda + ((lane & 7) ^ swz8(r)) * 16;
  }
#pragma unroll
  for (int j = 0; j < 4 * NS; ++j) {
    const int r = 8 * j + r8;
    gb[j] = g.b + (int64_t)min(n0 + r, N - 1) * g.ldb + ((lane & 7) ^ swz8(r)) * 16;
  }
  const uint32_t ring =
      __builtin_amdgcn_readfirstlane((uint32_t)reinterpret_cast<uintptr_t>(sRing)) + wave * WST * STB;
  const int nk = K / SK;
  const int mine = nk > wave ? (nk - wave + 3) / 4 : 0;  // stages wave, wave + 4, ...
  auto issue = [&](int t) {
    const int64_t k0 = (int64_t)(wave + 4 * t) * SK;
    const uint32_t dst = ring + (t % WST) * STB;
#pragma unroll
    for (int j = 0; j < 4; ++j) dma16(ga[j] + k0, dst + j * 1024);
#pragma unroll
    for (int j = 0; j < 4 * NS; ++j) dma16(gb[j] + k0, dst + 4096 + j * 1024);
  };
#pragma unroll
  for (int t = 0; t < WST - 1; ++t)
    if (t < mine) issue(t);

  const int sw = swz8(lane & 31);
  const int8_t *wr = sRing + wave * WST * STB + (lane & 31) * SK;
  // NS == 1: two accumulators so that consecutive MFMAs do not wait on each
  // other; NS == 2: one per column subtile
  v16i acc[2];
#pragma unroll
  for (int r = 0; r < 16; ++r) acc[0][r] = acc[1][r] = 0;
  int32_t xs = 0;
  for (int t = 0; t < mine; ++t) {
    // stage t has landed once the copies of at most min(WST - 2, mine - 1 - t)
    // later stages are outstanding
    const int later = min(WST - 2, mine - 1 - t);
    if (WST >= 4 && later >= 2)
      wait_vmcnt<2 * DMA_STAGE>();
    else if (later >= 1)
      wait_vmcnt<DMA_STAGE>();
    else
      wait_vmcnt<0>();
    const int8_t *pa = wr + (t % WST) * STB;
    v4i fa[4], fb[NS][4];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const int p = ((2 * ks + (lane >> 5)) ^ sw) * 16;
      fa[ks] = *reinterpret_cast<const v4i *>(pa + p);
#pragma unroll
      for (int q = 0; q < NS; ++q) fb[q][ks] = *reinterpret_cast<const v4i *>(pa + 4096 * (1 + q) + p);
    }
    // the slot of stage t - 1 is free: its fragments were consumed
    if (t + WST - 1 < mine) issue(t + WST - 1);
    if (NS == 1) {
#pragma unroll
      for (int ks = 0; ks < 4; ks += 2) {
        acc[0] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[ks], fb[0][ks], acc[0], 0, 0, 0);
        acc[1] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[ks + 1], fb[0][ks + 1], acc[1], 0, 0, 0);
      }
    } else {
#pragma unroll
      for (int ks = 0; ks < 4; ++ks)
#pragma unroll
        for (int q = 0; q < NS; ++q)
          acc[q] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[ks], fb[q][ks], acc[q], 0, 0, 0);
    }
    if (zp) {
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) xs = sum16v(fa[ks], xs);
    }
  }
  if (zp) {
    xs += __shfl_xor(xs, 32);
    if (lane < 32) sXs[wave][lane] = xs;
  }
  // partial tiles into the (now idle) rings: [wave][row][PLDM]. 32x32 MFMA
  // layout: lane l holds column l % 32, register r row (r/4)*8 + (l/32)*4 + r%4.
  __syncthreads();
  int32_t *part = reinterpret_cast<int32_t *>(sRing) + wave * 32 * PLDM;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int row = (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
    if (NS == 1) {
      part[row * PLDM + (lane & 31)] = (int32_t)((uint32_t)acc[0][r] + (uint32_t)acc[1][r]);
    } else {
#pragma unroll
      for (int q = 0; q < NS; ++q) part[row * PLDM + q * 32 + (lane & 31)] = acc[q][r];
    }
  }
  if (GELU && tid < 16) sLut[tid] = (uint8_t)lutv;
  __syncthreads();

  if (n >= N) return;
  const ColParams c = decode_col<EPI>(g, craw);
  const int32_t *ps = reinterpret_cast<const int32_t *>(sRing);
#pragma unroll
  for (int j = 0; j < RPT; ++j) {
    const int r = mr0 + (256 / CPB) * j;
    const int m = m0 + r;
    if (m < M) {
      uint32_t a = 0;
      int32_t xsum = 0;
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        a += (uint32_t)ps[(w * 32 + r) * PLDM + cl];
        if (zp) xsum += sXs[w][r];
      }
      skinny_store<EPI, GELU, SCATTER>(g, sc, c, sLut, pos, m, n, corrected_k32k((int32_t)a, xsum, c),
                                       EPI == EPI_L32RES ? resv[j] : 0);
    }
  }
}

// ---------------------------------------------------------------------------
// Register kernel (any K % 16 == 0)
// ---------------------------------------------------------------------------

constexpr int NT = 512;   // 8 waves
constexpr int BATCH = 8;  // k32 steps whose loads are in flight together
constexpr int PLD = 33;   // LDS row stride of the partial sums (words)

template <int EPI, bool GELU, bool SCATTER>
__global__ __launch_bounds__(NT) void gemm_skinny_kernel(GemmArgs g, SkinnyScatter sc, int ms) {
  __shared__ int32_t sPart[8 * 32 * PLD];
  __shared__ int32_t sXs[8][32];
  __shared__ uint8_t sLut[16];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int M = (int)g.M, N = (int)g.N, K = (int)g.K;
  const int n0 = blockIdx.x * TN;
  const int ks_n = 8 / ms;          // K slices
  const int msub = wave % ms, kslice = wave / ms;
  const bool zp = g.wz != nullptr;
  if (GELU && tid < 16) sLut[tid] = g.lut[tid];

  // fragment rows: lane l reads row l % 32, bytes [(l / 32) * 16, +16) of each k32 step
  const int arow = min(msub * 32 + (lane & 31), M - 1);
  const int brow = min(n0 + (lane & 31), N - 1);
  const int8_t *pa = g.a + (int64_t)arow * g.lda + (lane >> 5) * 16;
  const int8_t *pb = g.b + (int64_t)brow * g.ldb + (lane >> 5) * 16;
  const int steps = (K + 31) / 32;
  const int per = (steps + ks_n - 1) / ks_n;
  const int s0 = kslice * per, s1 = min(steps, s0 + per);

  v16i acc;
#pragma unroll
  for (int r = 0; r < 16; ++r) acc[r] = 0;
  int32_t xs = 0;
  for (int sb = s0; sb < s1; sb += BATCH) {
    v4i fa[BATCH], fb[BATCH];
#pragma unroll
    for (int u = 0; u < BATCH; ++u) {
      const int k = (sb + u) * 32 + (lane >> 5) * 16;
      const bool ok = sb + u < s1 && k < K;
      fa[u] = ok ? *reinterpret_cast<const v4i *>(pa + (int64_t)(sb + u) * 32) : v4i{0, 0, 0, 0};
      fb[u] = ok ? *reinterpret_cast<const v4i *>(pb + (int64_t)(sb + u) * 32) : v4i{0, 0, 0, 0};
    }
#pragma unroll
    for (int u = 0; u < BATCH; ++u) {
      acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[u], fb[u], acc, 0, 0, 0);
      if (zp) xs = sum16v(fa[u], xs);
    }
  }

  // partial sums to LDS: slot (kslice, msub) holds 32 rows x 32 columns.
  // 32x32 MFMA layout: lane l holds column l % 32, register r row
  // (r / 4) * 8 + (l / 32) * 4 + (r % 4).
  int32_t *part = &sPart[(kslice * ms + msub) * 32 * PLD];
#pragma unroll
  for (int r = 0; r < 16; ++r)
    part[((r >> 2) * 8 + (lane >> 5) * 4 + (r & 3)) * PLD + (lane & 31)] = acc[r];
  if (zp) {
    xs += __shfl_xor(xs, 32);
    if (lane < 32) sXs[kslice * ms + msub][lane] = xs;
  }
  __syncthreads();

  // Epilogue: thread t serves column t % 32 and rows t / 32, t / 32 + 16, ...
  const int cl = tid & 31;
  const int n = n0 + cl;
  if (n >= N) return;
  const ColParams c = load_col<EPI>(g, n);
  int pos = 0;
  if (SCATTER) pos = *sc.pos;
  for (int m = tid >> 5; m < M; m += NT / 32) {
    const int mi = m >> 5, mr = m & 31;
    uint32_t a = 0;
    int32_t xsum = 0;
    for (int s = 0; s < ks_n; ++s) {
      a += (uint32_t)sPart[((s * ms + mi) * 32 + mr) * PLD + cl];
      if (zp) xsum += sXs[s * ms + mi][mr];
    }
    const int32_t res = EPI == EPI_L32RES ? g.res[(int64_t)m * g.ldres + n] : 0;
    skinny_store<EPI, GELU, SCATTER>(g, sc, c, sLut, pos, m, n, corrected((int32_t)a, xsum, c), res);
  }
}

constexpr int64_t kDeepRingTiles = 256;  // CUs of an MI355X
// grids up to this many 32 x 32 tiles take the m-split kernel
constexpr int64_t kMsplitMaxBlocks = 1024;

bool lds_eligible(const GemmArgs &g) {
  const uintptr_t al = reinterpret_cast<uintptr_t>(g.a) | reinterpret_cast<uintptr_t>(g.b) |
                       (uintptr_t)g.lda | (uintptr_t)g.ldb;
  // corrected_k32k needs K <= 32768
  return g.K % SK == 0 && g.K <= 32768 && (al & 15) == 0;
}

template <int EPI, bool GELU, bool SCATTER>
int launch_skinny(const GemmArgs &g, const SkinnyScatter &sc, hipStream_t s) {
  const int64_t tiles = (g.N + TN - 1) / TN;
  if (tiles == 0 || g.M == 0) return 0;
  const int ms = (int)((g.M + 31) / 32);
  if (lds_eligible(g) && tiles * ms <= kMsplitMaxBlocks) {
    // one 32 x 32 tile per block; the blocks of a column tile share an XCD.
    // Up to one block per CU: a 4-stage ring per wave (128 KB of LDS); more:
    // 2 stages, two blocks per CU. (64-column tiles, NS = 2, measured slower
    // for N = 3840 and 5120 at M = 128.)
    const dim3 block(LNT);
    const dim3 grid((unsigned)(((tiles + 7) / 8) * 8 * ms));
    if (tiles * ms <= kDeepRingTiles)
      hipLaunchKernelGGL((gemm_skinny_msplit_kernel<EPI, GELU, SCATTER, 4, 1>), grid, block, 0, s, g, sc,
                         ms, (int)tiles);
    else
      hipLaunchKernelGGL((gemm_skinny_msplit_kernel<EPI, GELU, SCATTER, 2, 1>), grid, block, 0, s, g, sc,
                         ms, (int)tiles);
    return check_launch("gemm_skinny_msplit_kernel");
  }
  if (lds_eligible(g)) {
    const dim3 grid((unsigned)tiles), block(LNT);
    // one block per CU: 6 stages (up to 120 KB of LDS); more blocks: 3
    const bool deep = tiles <= kDeepRingTiles;
#define IW_SKL(MS_)                                                                                 \
  do {                                                                                              \
    if (deep)                                                                                       \
      hipLaunchKernelGGL((gemm_skinny_lds_kernel<EPI, GELU, SCATTER, MS_, 6>), grid, block, 0, s, g, sc); \
    else                                                                                            \
      hipLaunchKernelGGL((gemm_skinny_lds_kernel<EPI, GELU, SCATTER, MS_, 3>), grid, block, 0, s, g, sc); \
  } while (0)
    if (ms <= 1)
      IW_SKL(1);
    else if (ms <= 2)
      IW_SKL(2);
    else
      IW_SKL(4);
#undef IW_SKL
    return check_launch("gemm_skinny_lds_kernel");
  }
  const int msp = ms <= 1 ? 1 : (ms <= 2 ? 2 : 4);  // m-subtiles per block: a divisor of 8
  hipLaunchKernelGGL((gemm_skinny_kernel<EPI, GELU, SCATTER>), dim3((unsigned)tiles), dim3(NT), 0, s,
                     g, sc, msp);
  return check_launch("gemm_skinny_kernel");
}

}  // namespace

bool gemm_skinny_eligible(const GemmArgs &g) {
  const uintptr_t al = reinterpret_cast<uintptr_t>(g.a) | reinterpret_cast<uintptr_t>(g.b) |
                       (uintptr_t)g.lda | (uintptr_t)g.ldb;
  return g.M > 0 && g.M <= kSkinnyMaxRows && g.K % 16 == 0 && (al & 15) == 0 && g.pe == nullptr &&
         g.N <= 0x7fffff00LL && g.K <= 0x7fffff00LL;
}

int gemm_skinny(const GemmArgs &g, const SkinnyScatter *scatter, hipStream_t s) {
  const bool gelu = g.lut != nullptr;
  SkinnyScatter sc;
  if (scatter) {
    if (g.epi != EPI_L8 || gelu) return fail("the KV-cache epilogue is for the Linear8 QKV projection");
    sc = *scatter;
    return launch_skinny<EPI_L8, false, true>(g, sc, s);
  }
  switch (g.epi) {
    case EPI_L8:
      if (gelu) return launch_skinny<EPI_L8, true, false>(g, sc, s);
      return launch_skinny<EPI_L8, false, false>(g, sc, s);
    case EPI_L32: return launch_skinny<EPI_L32, false, false>(g, sc, s);
    case EPI_L32RES: return launch_skinny<EPI_L32RES, false, false>(g, sc, s);
    case EPI_S8:
      if (gelu) return launch_skinny<EPI_S8, true, false>(g, sc, s);
      return launch_skinny<EPI_S8, false, false>(g, sc, s);
    default: return fail("unknown GEMM epilogue");
  }
}

}  // namespace iw
