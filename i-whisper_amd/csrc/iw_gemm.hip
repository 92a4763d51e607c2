// int8 x int8 -> int32 GEMM on CDNA4 MFMA (v_mfma_i32_32x32x32_i8) with fused
// integer epilogues. One kernel serves every GEMM-shaped op on the path:
//   Linear8            linear8/linear8_scalar.cpp:30-85
//   Linear8 + GeLU     (FC1 fused with gelu/gelu_scalar.cpp:10-181)
//   Linear32           linear32/linear32_scalar.cpp:96-129
//   Linear32 + residual15  (out-proj / FC2 fused with residual15_scalar.cpp:9-28)
//   classifier         classifier/classifier_scalar.cpp:91-142
//   conv1d             conv1d/conv1d_scalar.cpp:186-288 as an implicit GEMM
//
// C[m][n] = sum_k A[m][k] * B[n][k]; both operands are K-contiguous int8.
// Block tile 128x128x64, 256 threads = 4 waves in a 2x2 grid, each wave a
// 64x64 tile of 2x2 MFMA 32x32x32 blocks. Operands are staged through LDS
// with a 16-byte row pad (80-byte stride, conflict-free ds_read_b128),
// double-buffered with a register prefetch of the next K tile.
//
// Integer sums are exact modulo 2^32 in any order, so the zero-point term
// wz[n] * rowsum(A[m]) is formed from per-row sums taken with v_dot4 while
// the A tile passes through registers, and added in the epilogue.
#include <algorithm>

#include "iw_gemm_dev.hpp"

namespace iw {

using namespace gemm;

namespace {

constexpr int BM = 128, BN = 128, BK = 64;
constexpr int LDT = BK + 16;  // LDS row stride in bytes
constexpr int NT = 256;

// Linear32 output: low 32 bits of mulh(acc, m) * 2^shift; 0 outside [0, 31].
__device__ __forceinline__ int32_t linear32_out(int32_t acc, uint32_t m, int32_t s) {
  int32_t h = mulh(acc, m);
  return (s < 0 || s >= 32) ? 0 : (int32_t)((uint32_t)h << s);
}

template <int AMODE, bool BFAST, int EPI, int OUTL>
__global__ __launch_bounds__(NT) void gemm_i8_kernel(GemmArgs g) {
  __shared__ __attribute__((aligned(16))) int8_t sA[2][BM * LDT];
  __shared__ __attribute__((aligned(16))) int8_t sB[2][BN * LDT];
  __shared__ int32_t sXsum[BM];
  __shared__ uint8_t sLut[16];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  // Tile order: consecutive blocks walk N first so that blocks sharing an A
  // row panel run together and reuse it from L2.
  const int ntn = (g.N + BN - 1) / BN;
  const int64_t bid = blockIdx.x;
  const int64_t m0 = (bid / ntn) * BM;
  const int64_t n0 = (bid % ntn) * BN;

  // Each thread moves two 16-byte chunks of A and two of B per K tile.
  const int crow0 = tid >> 2;        // rows crow0 and crow0 + 64
  const int ccol = (tid & 3) * 16;   // byte offset inside the 64-wide K tile
  RowInfo ra[2];
  ra[0] = a_row_info(g, AMODE, m0 + crow0);
  ra[1] = a_row_info(g, AMODE, m0 + crow0 + 64);
  int32_t xs[2] = {0, 0};

  uint4 pa[2], pb[2];
  auto fetch = [&](int64_t k0) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      pa[i] = load_a16(g, AMODE, ra[i], m0 + crow0 + 64 * i, k0 + ccol);
      pb[i] = load_b16(g, BFAST, n0 + crow0 + 64 * i, k0 + ccol);
    }
  };
  auto stash = [&](int buf) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      *reinterpret_cast<uint4 *>(&sA[buf][(crow0 + 64 * i) * LDT + ccol]) = pa[i];
      *reinterpret_cast<uint4 *>(&sB[buf][(crow0 + 64 * i) * LDT + ccol]) = pb[i];
      if (g.wz) xs[i] += sum16(pa[i]);
    }
  };

  v16i acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0;

  const int64_t nk = (g.K + BK - 1) / BK;
  fetch(0);
  stash(0);
  if (tid < 16 && g.lut) sLut[tid] = g.lut[tid];
  __syncthreads();

  // Fragment addressing: lane l reads row (l % 32), 16 bytes at (l / 32) * 16
  // of each 32-wide K step. A and B use the same mapping, so the MFMA sums
  // over the same K index on both sides.
  const int frow = lane & 31;
  const int fk = (lane >> 5) * 16;

  for (int64_t kt = 0; kt < nk; ++kt) {
    const int cur = (int)(kt & 1);
    if (kt + 1 < nk) fetch((kt + 1) * BK);
#pragma unroll
    for (int ks = 0; ks < BK; ks += 32) {
      v4i fa[2], fb[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        fa[i] = *reinterpret_cast<const v4i *>(&sA[cur][(wm * 64 + i * 32 + frow) * LDT + ks + fk]);
        fb[i] = *reinterpret_cast<const v4i *>(&sB[cur][(wn * 64 + i * 32 + frow) * LDT + ks + fk]);
      }
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[i], fb[j], acc[i][j], 0, 0, 0);
    }
    if (kt + 1 < nk) stash(cur ^ 1);
    __syncthreads();
  }

  // Row sums of A: the four threads of a row are adjacent lanes.
  if (g.wz) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      int32_t s = xs[i];
      s += __shfl_xor(s, 1);
      s += __shfl_xor(s, 2);
      if ((tid & 3) == 0) sXsum[crow0 + 64 * i] = s;
    }
  }
  __syncthreads();

  // Epilogue. 32x32 MFMA output layout: lane l holds column l % 32 and, for
  // register r, row (r / 4) * 8 + (l / 32) * 4 + (r % 4).
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int64_t n = n0 + wn * 64 + j * 32 + (lane & 31);
    if (n >= g.N) continue;
    const uint32_t wzn = g.wz ? (uint32_t)(int32_t)g.wz[n] : 0u;
    const uint32_t bn = g.bias ? (uint32_t)g.bias[n] : 0u;
    const uint32_t mn = g.mult ? g.mult[g.mult_pc ? n : 0] : g.scalar_mult;
    const int32_t sn = g.shift ? g.shift[g.mult_pc ? n : 0] : g.scalar_shift;
    uint32_t gi_m = 0, go_m = 0;
    int32_t gi_s = 0, go_s = 0;
    if (g.lut) {
      gi_m = g.luti_m[g.luti_pc ? n : 0];
      gi_s = g.luti_s[g.luti_pc ? n : 0];
      go_m = g.luto_m[g.luto_pc ? n : 0];
      go_s = g.luto_s[g.luto_pc ? n : 0];
    }
    uint32_t pe_m = 0;
    int32_t pe_s = 0;
    if (g.pe) {
      pe_m = g.pe_mult[g.pe_mpc ? n : 0];
      pe_s = g.pe_shift[g.pe_spc ? n : 0];
      pe_s = pe_s < 0 ? 0 : pe_s;
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int lrow = wm * 64 + i * 32 + (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
        const int64_t m = m0 + lrow;
        if (m >= g.M) continue;
        uint32_t a = (uint32_t)acc[i][j][r];
        if (g.wz) a -= wzn * (uint32_t)sXsum[lrow];
        a += bn;
        if (EPI == EPI_L8) {
          int32_t y = rshift(mulh((int32_t)a, mn), (uint32_t)sn);
          y = clampi(y, -127, 127);
          if (g.lut) y = gelu_one(y, sLut, gi_m, gi_s, go_m, go_s);
          reinterpret_cast<int8_t *>(g.out)[m * g.ldc + n] = (int8_t)y;
        } else if (EPI == EPI_L32) {
          reinterpret_cast<int32_t *>(g.out)[m * g.ldc + n] = linear32_out((int32_t)a, mn, sn);
        } else if (EPI == EPI_L32RES) {
          int32_t br = linear32_out((int32_t)a, mn, sn);
          int32_t res = g.res[m * g.ldres + n];
          uint32_t v = (uint32_t)br + (uint32_t)(res * (int32_t)g.res_mult);
          int32_t y = clampi(rshift_pos((int32_t)v, 15), -16383, 16383);
          reinterpret_cast<int16_t *>(g.out)[m * g.ldc + n] = (int16_t)y;
        } else {  // EPI_S8: per-tensor requant with the shift clamped at 0
          int32_t y = rshift(mulh((int32_t)a, mn), (uint32_t)(sn < 0 ? 0 : sn));
          y = clampi(y, -127, 127);
          if (g.lut) y = gelu_one(y, sLut, gi_m, gi_s, go_m, go_s);
          if (g.pe) {
            // add_requant15 of the positional embedding (add_requant15_scalar.cpp:29-81)
            const int64_t t = m % g.pe_T;
            int32_t v = y + (int32_t)g.pe[t * g.N + n];
            int32_t p = (int32_t)((uint32_t)v * pe_m);
            int32_t z = clampi(rshift(p, (uint32_t)pe_s), -16383, 16383);
            reinterpret_cast<int16_t *>(g.out)[m * g.ldc + n] = (int16_t)z;
          } else if (OUTL == OUT_NCT) {
            const int64_t bb = m / g.out_T, t = m % g.out_T;
            reinterpret_cast<int8_t *>(g.out)[(bb * g.N + n) * g.out_T + t] = (int8_t)y;
          } else {
            reinterpret_cast<int8_t *>(g.out)[m * g.ldc + n] = (int8_t)y;
          }
        }
      }
    }
  }
}

template <int AMODE, bool BFAST, int EPI, int OUTL>
int launch(const GemmArgs &g, hipStream_t s) {
  const int64_t tiles = ((g.M + BM - 1) / BM) * ((g.N + BN - 1) / BN);
  if (tiles == 0) return 0;
  if (tiles > 0x7fffffffLL) return fail("GEMM grid too large");
  hipLaunchKernelGGL((gemm_i8_kernel<AMODE, BFAST, EPI, OUTL>), dim3((unsigned)tiles), dim3(NT), 0,
                     s, g);
  return check_launch("gemm_i8_kernel");
}

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

}  // namespace

int gemm_dense(const GemmArgs &g, hipStream_t s) {
  const bool afast = g.K % 16 == 0 && g.lda % 16 == 0 && aligned16(g.a);
  const bool bfast = g.K % 16 == 0 && g.ldb % 16 == 0 && aligned16(g.b);
  if (gemm_skinny_eligible(g)) return gemm_skinny(g, nullptr, s);
  if (g.M > kSkinnyMaxRows && g.M <= kSkinnyChunkMaxRows) {
    // a few hundred rows (the decoder's prompt step): the decode kernel over
    // chunks of 128 rows, whose launches cost less than one launch of the
    // tile kernel at this size
    GemmArgs c = g;
    c.M = kSkinnyMaxRows;
    if (gemm_skinny_eligible(c)) {
      const int64_t esz = g.epi == EPI_L32 ? 4 : (g.epi == EPI_L32RES ? 2 : 1);  // output bytes
      for (int64_t r0 = 0; r0 < g.M; r0 += kSkinnyMaxRows) {
        c.M = std::min<int64_t>(kSkinnyMaxRows, g.M - r0);
        c.a = g.a + r0 * g.lda;
        c.out = static_cast<int8_t *>(g.out) + r0 * g.ldc * esz;
        if (g.res) c.res = g.res + r0 * g.ldres;
        const int rc = gemm_skinny(c, nullptr, s);
        if (rc) return rc;
      }
      return 0;
    }
  }
  if (g.M >= kBigGemmMinRows && gemm_dtl_eligible(g)) return gemm_dtl(g, s);
  if (afast && bfast && g.M >= kBigGemmMinRows) return gemm_big(g, false, s);
  switch (g.epi) {
    case EPI_L8:
      if (afast && bfast) return launch<A_DENSE16, true, EPI_L8, OUT_ROW>(g, s);
      return launch<A_GEN_DENSE, false, EPI_L8, OUT_ROW>(g, s);
    case EPI_L32:
      if (afast && bfast) return launch<A_DENSE16, true, EPI_L32, OUT_ROW>(g, s);
      return launch<A_GEN_DENSE, false, EPI_L32, OUT_ROW>(g, s);
    case EPI_L32RES:
      if (afast && bfast) return launch<A_DENSE16, true, EPI_L32RES, OUT_ROW>(g, s);
      return launch<A_GEN_DENSE, false, EPI_L32RES, OUT_ROW>(g, s);
    case EPI_S8:
      if (afast && bfast) return launch<A_DENSE16, true, EPI_S8, OUT_ROW>(g, s);
      return launch<A_GEN_DENSE, false, EPI_S8, OUT_ROW>(g, s);
    default:
      return fail("unknown GEMM epilogue");
  }
}

int gemm_conv(const GemmArgs &g, bool channels_last, hipStream_t s) {
  if (g.epi != EPI_S8) return fail("conv GEMM supports the per-tensor int8 epilogue only");
  if (channels_last) {
    const bool fast = g.conv_cin % 16 == 0 && aligned16(g.a) && g.K % 16 == 0 &&
                      g.ldb % 16 == 0 && aligned16(g.b);
    if (!fast) return fail("channels-last conv needs Cin % 16 == 0 and 16-byte aligned buffers");
    if (g.M >= kBigGemmMinRows) return gemm_big(g, true, s);
    return launch<A_CONVCL16, true, EPI_S8, OUT_ROW>(g, s);
  }
  return launch<A_GEN_CONVNCT, false, EPI_S8, OUT_NCT>(g, s);
}

}  // namespace iw
