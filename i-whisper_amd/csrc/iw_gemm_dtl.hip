// Large-M dense int8 GEMM with direct-to-LDS operand loads (gfx950
// global_load_lds_dwordx4): the encoder's QKV, out-projection, FC1 (+GeLU)
// and FC2 (+residual15), and any dense Linear with K % 64 == 0.
//
// C[m][n] = sum_k A[m][k] * B[n][k], both operands K-contiguous int8.
// Block tile 256 (M) x 128 (N) x 64 (K); 4 waves in a 2 x 2 grid, each a
// 128 x 64 tile of 4 x 2 v_mfma_i32_32x32x32_i8 blocks. Two blocks share a
// CU so that one block's epilogue (VALU) overlaps the other's MFMAs.
//
// Operands stream global -> LDS without passing through registers, into a
// 3-stage ring: while the MFMAs consume stage k, stages k+1 and k+2 are in
// flight. Each wave waits only for its own loads of stage k (s_waitcnt
// vmcnt), then one s_barrier per K tile publishes the stage to all waves;
// the release fence of __syncthreads() would drain every load and is not
// used in the loop.
//
// LDS rows are 64 bytes (4 chunks of 16) with chunk c of row r stored at
// position c ^ swz(r), swz(r) = 2*bit2(r) + (bit1(r) ^ bit3(r)), so that the
// ds_read_b128 fragment reads of 8 or 16 consecutive rows hit distinct banks.
//
// The zero-point row sums sum_k A[m][k] are taken with v_dot4 from the A
// fragments already in registers (the two waves sharing rows split the
// subtiles). Epilogues are those of iw_gemm_dev.hpp, bit-identical to the
// reference kernels.
#include "iw_gemm_dev.hpp"

namespace iw {

using namespace gemm;

namespace {

constexpr int BM = 256, BN = 128, BK = 64, STAGES = 3;
constexpr int NT = 256;
constexpr int XCDS = 8;
constexpr int A_STAGE = BM * BK, B_STAGE = BN * BK;

// One 16-byte global -> LDS copy per lane (global_load_lds_dwordx4): the wave
// writes 1 KB at LDS byte address `lds` (lane l at lds + 16 l). Issued as
// inline assembly so that the compiler does not add waits for it: the loop
// below waits on vmcnt itself. No kernel using it keeps a value in M0.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void dma16(const int8_t *src, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(lds)
               : "memory", "m0");
}
#pragma clang diagnostic pop

// Fourth word of a raw buffer resource on gfx9-family GPUs (32-bit data
// format; offsets range-checked against the record count).
constexpr int kBufferFlags = 0x00020000;

__device__ __forceinline__ uint32_t lds_addr(const void *p) {
  return (uint32_t)reinterpret_cast<uintptr_t>(p);
}

__device__ __forceinline__ int32_t sum16v(v4i v, int32_t acc) {
  const int ones = 0x01010101;
  acc = __builtin_amdgcn_sdot4(v[0], ones, acc, false);
  acc = __builtin_amdgcn_sdot4(v[1], ones, acc, false);
  acc = __builtin_amdgcn_sdot4(v[2], ones, acc, false);
  return __builtin_amdgcn_sdot4(v[3], ones, acc, false);
}

__device__ __forceinline__ int swz(int r) { return ((r >> 1) & 2) | (((r >> 1) ^ (r >> 3)) & 1); }

template <int EPI, bool GELU>
__global__ __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(2, 2)))
void gemm_dtl_kernel(GemmArgs g, int tiles_n, int tiles_total, int per_xcd) {
  __shared__ __attribute__((aligned(1024))) int8_t sA[STAGES * A_STAGE];
  __shared__ __attribute__((aligned(1024))) int8_t sB[STAGES * B_STAGE];
  __shared__ __attribute__((aligned(16))) int32_t sXsum[BM];
  __shared__ uint8_t sLut[16];

  const int bid = blockIdx.x;
  const int tile = (bid % XCDS) * per_xcd + bid / XCDS;
  if (tile >= tiles_total) return;
  const int m0 = (tile / tiles_n) * BM;
  const int n0 = (tile % tiles_n) * BN;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  const int M = (int)g.M, N = (int)g.N, K = (int)g.K;
  const bool zp = g.wz != nullptr;

  // DMA mapping: instruction j of a stage writes LDS bytes [j*1024, +1024),
  // i.e. rows 16j .. 16j+15; lane l writes row 16j + l/4 at position l % 4
  // and so fetches chunk (l % 4) ^ swz(row). Rows past the matrix edge read
  // the last row instead (their results are never stored).
  const int8_t *ga[4];
  const int8_t *gb[2];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = (wave * 4 + i) * 16 + (lane >> 2);
    const int c = (lane & 3) ^ swz(r);
    ga[i] = g.a + (int64_t)min(m0 + r, M - 1) * g.lda + c * 16;
  }
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int r = (wave * 2 + i) * 16 + (lane >> 2);
    const int c = (lane & 3) ^ swz(r);
    gb[i] = g.b + (int64_t)min(n0 + r, N - 1) * g.ldb + c * 16;
  }
  const uint32_t ldsA = __builtin_amdgcn_readfirstlane(lds_addr(sA) + wave * 4 * 1024);
  const uint32_t ldsB = __builtin_amdgcn_readfirstlane(lds_addr(sB) + wave * 2 * 1024);
  auto issue = [&](int kt) {
    const int st = kt % STAGES;
    const int k0 = kt * BK;
#pragma unroll
    for (int i = 0; i < 4; ++i) dma16(ga[i] + k0, ldsA + st * A_STAGE + i * 1024);
#pragma unroll
    for (int i = 0; i < 2; ++i) dma16(gb[i] + k0, ldsB + st * B_STAGE + i * 1024);
  };

  const int nk = K / BK;
  if (GELU && tid < 16) sLut[tid] = g.lut[tid];
  issue(0);
  if (nk > 1) issue(1);

  v16i acc[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0;
  int32_t xs[2] = {0, 0};

  // Fragment reads: lane l reads row l % 32 of a 32-row subtile, chunk
  // 2*ks + l/32; the swizzle depends only on l % 32.
  const int sw = swz(lane & 31);
  const int fo0 = (((lane >> 5)) ^ sw) * 16;
  const int fo1 = ((2 + (lane >> 5)) ^ sw) * 16;
  const int aoff = (wm * 128 + (lane & 31)) * BK;
  const int boff = (wn * 64 + (lane & 31)) * BK;

  for (int kt = 0; kt < nk; ++kt) {
    if (kt + 1 < nk)
      asm volatile("s_waitcnt vmcnt(6)" ::: "memory");
    else
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    if (kt + 2 < nk) issue(kt + 2);
    const int8_t *pa = &sA[(kt % STAGES) * A_STAGE + aoff];
    const int8_t *pb = &sB[(kt % STAGES) * B_STAGE + boff];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const int fo = ks ? fo1 : fo0;
      v4i fa[4], fb[2];
#pragma unroll
      for (int i = 0; i < 4; ++i) fa[i] = *reinterpret_cast<const v4i *>(pa + i * 32 * BK + fo);
#pragma unroll
      for (int j = 0; j < 2; ++j) fb[j] = *reinterpret_cast<const v4i *>(pb + j * 32 * BK + fo);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[i], fb[j], acc[i][j], 0, 0, 0);
      if (zp) {
        // the two waves of a row half take two subtiles each
        if (wn == 0) {
          xs[0] = sum16v(fa[0], xs[0]);
          xs[1] = sum16v(fa[1], xs[1]);
        } else {
          xs[0] = sum16v(fa[2], xs[0]);
          xs[1] = sum16v(fa[3], xs[1]);
        }
      }
    }
  }

  if (zp) {
#pragma unroll
    for (int ii = 0; ii < 2; ++ii) {
      const int32_t s = xs[ii] + __shfl_xor(xs[ii], 32);
      if (lane < 32) sXsum[wm * 128 + (wn * 2 + ii) * 32 + lane] = s;
    }
  }
  __syncthreads();

  // Epilogue. 32x32 MFMA output layout: lane l holds column l % 32 and, for
  // register r, row (r / 4) * 8 + (l / 32) * 4 + (r % 4).
  // Stores are buffer stores relative to the tile origin with 32-bit offsets;
  // the buffer ends at row M, so rows past the matrix are dropped by the
  // hardware range check, and columns past N get an offset beyond any range.
  // Output bytes per element: int8 (Linear8, per-tensor), int32 (Linear32),
  // int16 (residual15).
  constexpr int OB = (EPI == EPI_L8 || EPI == EPI_S8) ? 1 : (EPI == EPI_L32 ? 4 : 2);
  const int ldo = (int)g.ldc * OB;
  const __amdgpu_buffer_rsrc_t out_rs = __builtin_amdgcn_make_buffer_rsrc(
      reinterpret_cast<char *>(g.out) + ((int64_t)m0 * g.ldc + n0) * OB, (short)0,
      (int)min((int64_t)(M - m0) * ldo, (int64_t)0x7fffffff), kBufferFlags);
  const int ldr = (int)g.ldres * 2;
  __amdgpu_buffer_rsrc_t res_rs = out_rs;
  if (EPI == EPI_L32RES)
    res_rs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<int16_t *>(g.res) + (int64_t)m0 * g.ldres + n0, (short)0,
        (int)min((int64_t)(M - m0) * ldr, (int64_t)0x7fffffff), kBufferFlags);
  const int row_l = wm * 128 + (lane >> 5) * 4;  // first row of this lane
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int nl = wn * 64 + j * 32 + (lane & 31);
    const bool ncol = n0 + nl < N;
    const ColParams c = load_col<EPI>(g, min(n0 + nl, N - 1));
    const uint32_t obase = ncol ? (uint32_t)(row_l * ldo + nl * OB) : 0x80000000u;
    const uint32_t rbase = ncol ? (uint32_t)(row_l * ldr + nl * 2) : 0x80000000u;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int lrow0 = row_l + i * 32 + q * 8;
        int4 x4 = make_int4(0, 0, 0, 0);
        if (zp) x4 = *reinterpret_cast<const int4 *>(&sXsum[lrow0]);
        const int32_t xsv[4] = {x4.x, x4.y, x4.z, x4.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int rr = i * 32 + q * 8 + e;  // row relative to row_l
          const int32_t a = (int32_t)corrected_k32k(acc[i][j][q * 4 + e], xsv[e], c);
          const int ooff = (int)(obase + (uint32_t)(rr * ldo));
          if (EPI == EPI_L8 || EPI == EPI_S8) {
            int32_t y = clampi(apply_shift(mulh_su(a, c.mult), c.shift), -127, 127);
            if (GELU) y = gelu_dec(y, sLut, c);
            __builtin_amdgcn_raw_buffer_store_b8((unsigned char)y, out_rs, ooff, 0, 0);
          } else {
            const int32_t br = (int32_t)((uint32_t)mulh_su(a, c.mult) << c.shift.sh);
            if (EPI == EPI_L32) {
              __builtin_amdgcn_raw_buffer_store_b32((unsigned)br, out_rs, ooff, 0, 0);
            } else {
              const int roff = (int)(rbase + (uint32_t)(rr * ldr));
              const int32_t res = (int16_t)__builtin_amdgcn_raw_buffer_load_b16(res_rs, roff, 0, 0);
              const uint32_t v = (uint32_t)br + (uint32_t)__mul24(res, (int32_t)g.res_mult);
              const int32_t y = clampi(rshift_pos((int32_t)v, 15), -16383, 16383);
              __builtin_amdgcn_raw_buffer_store_b16((unsigned short)y, out_rs, ooff, 0, 0);
            }
          }
        }
      }
    }
  }
}

template <int EPI, bool GELU>
int launch_dtl(const GemmArgs &g, hipStream_t s) {
  const int64_t tm = (g.M + BM - 1) / BM, tn = (g.N + BN - 1) / BN;
  const int64_t tiles = tm * tn;
  if (tiles == 0) return 0;
  const int per_xcd = (int)((tiles + XCDS - 1) / XCDS);
  hipLaunchKernelGGL((gemm_dtl_kernel<EPI, GELU>), dim3((unsigned)(per_xcd * XCDS)), dim3(NT), 0, s,
                     g, (int)tn, (int)tiles, per_xcd);
  return check_launch("gemm_dtl_kernel");
}

}  // namespace

bool gemm_dtl_eligible(const GemmArgs &g) {
  const uintptr_t al = reinterpret_cast<uintptr_t>(g.a) | reinterpret_cast<uintptr_t>(g.b) |
                       (uintptr_t)g.lda | (uintptr_t)g.ldb;
  // 32-bit offsets inside a tile; 24-bit zero-point products (K <= 32768)
  const int64_t ob = g.epi == EPI_L32 ? 4 : (g.epi == EPI_L32RES ? 2 : 1);
  return g.K % BK == 0 && (al & 15) == 0 && g.pe == nullptr && g.M > 0 && g.N > 0 &&
         g.K <= 32768 && g.ldc * ob * BM < 0x7fffffffLL && g.ldres * BM < 0x7fffffffLL &&
         g.M <= 0x7fffff00LL && g.N <= 0x7fffff00LL &&
         ((g.M + BM - 1) / BM) * ((g.N + BN - 1) / BN) <= 0x3fffffffLL;
}

int gemm_dtl(const GemmArgs &g, hipStream_t s) {
  const bool gelu = g.lut != nullptr;
  switch (g.epi) {
    case EPI_L8:
      if (gelu) return launch_dtl<EPI_L8, true>(g, s);
      return launch_dtl<EPI_L8, false>(g, s);
    case EPI_L32: return launch_dtl<EPI_L32, false>(g, s);
    case EPI_L32RES: return launch_dtl<EPI_L32RES, false>(g, s);
    case EPI_S8:
      if (gelu) return launch_dtl<EPI_S8, true>(g, s);
      return launch_dtl<EPI_S8, false>(g, s);
    default: return fail("unknown GEMM epilogue");
  }
}

}  // namespace iw
