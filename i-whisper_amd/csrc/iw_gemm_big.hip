// Large-M int8 GEMM for the encoder (QKV, out-projection, FC1+GeLU, FC2 +
// residual15, conv1/conv2 as implicit GEMMs) on v_mfma_i32_32x32x32_i8.
//
// C[m][n] = sum_k A[m][k] * B[n][k], both operands K-contiguous int8.
// Block tile 256 (M) x 128 (N) x 64 (K), 256 threads = 4 waves in a 2 x 2
// grid, each wave a 128 x 64 tile = 4 x 2 MFMA blocks of 32 x 32 (128
// accumulator registers). Two blocks share a CU, so one block's epilogue
// (VALU) overlaps the other's MFMA work. Operands go global -> registers ->
// LDS (80-byte padded rows, double-buffered); the next K tile is fetched
// into registers while the current one feeds the MFMAs.
//
// Tile order is XCD-aware: the dispatcher hands block b to XCD b % 8, so
// blocks are renumbered to give each XCD one contiguous range of tiles (N
// fastest), which keeps each A row panel inside one XCD's L2.
//
// The epilogue is bit-identical to the reference kernels (see
// iw_gemm_dev.hpp): zero point and bias, then Linear8 requant (+ GeLU),
// Linear32 (+ residual15) or per-tensor requant (+ GeLU, + positional
// add_requant15).
#include "iw_gemm_dev.hpp"

namespace iw {

using namespace gemm;

namespace {

constexpr int BM = 256, BN = 128, BK = 64;
constexpr int LDT = BK + 16;  // LDS row stride in bytes
constexpr int NT = 256;
constexpr int XCDS = 8;

enum : int { F_GELU = 1, F_PE = 2 };

template <int AMODE, int EPI, int FLAGS>
__global__ __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(2, 2)))
void gemm_big_kernel(GemmArgs g, int tiles_n, int tiles_total, int per_xcd) {
  constexpr bool GELU = (FLAGS & F_GELU) != 0;
  constexpr bool PE = (FLAGS & F_PE) != 0;
  __shared__ __attribute__((aligned(16))) int8_t sA[2][BM * LDT];
  __shared__ __attribute__((aligned(16))) int8_t sB[2][BN * LDT];
  __shared__ __attribute__((aligned(16))) int32_t sXsum[BM];
  __shared__ uint8_t sLut[16];

  const int bid = blockIdx.x;
  const int tile = (bid % XCDS) * per_xcd + bid / XCDS;
  if (tile >= tiles_total) return;
  const int m0 = (tile / tiles_n) * BM;
  const int n0 = (tile % tiles_n) * BN;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int K = (int)g.K;

  // Loader mapping: thread t moves 16-byte chunk (t & 3) of rows (t >> 2) + 64 i.
  const int crow = tid >> 2;
  const int ccol = (tid & 3) * 16;
  const int8_t *arow[4];
  int apos[4];  // conv: first input position of the row; dense: 0
  bool aval[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int m = m0 + crow + 64 * i;
    aval[i] = m < g.M;
    if (AMODE == A_CONVCL16) {
      const int tout = (int)g.conv_tout;
      const int bb = aval[i] ? m / tout : 0, t = aval[i] ? m % tout : 0;
      apos[i] = t * (int)g.conv_stride - (int)g.conv_pad;
      arow[i] = g.a + ((int64_t)bb * g.conv_tin + apos[i]) * g.conv_cin;
    } else {
      apos[i] = 0;
      arow[i] = g.a + (int64_t)m * g.lda;
    }
  }
  const int8_t *brow[2];
  bool bval[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int n = n0 + crow + 64 * i;
    bval[i] = n < g.N;
    brow[i] = g.b + (int64_t)n * g.ldb;
  }
  // conv: kernel tap (k / Cin) of this thread's chunk, advanced with k
  const int cin = (int)g.conv_cin;
  const int tin = (int)g.conv_tin;
  int tap = 0, tapc = ccol;
  if (AMODE == A_CONVCL16) {
    tap = ccol / cin;
    tapc = ccol - tap * cin;
  }
  int32_t xs[4] = {0, 0, 0, 0};

  uint4 pa[4], pb[2];
  auto fetch = [&](int k0) {
    const int k = k0 + ccol;
    const bool kin = k < K;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      bool ok = aval[i] && kin;
      if (AMODE == A_CONVCL16) {
        const int pos = apos[i] + tap;
        ok = ok && pos >= 0 && pos < tin;
      }
      pa[i] = ok ? *reinterpret_cast<const uint4 *>(arow[i] + k) : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < 2; ++i)
      pb[i] = (bval[i] && kin) ? *reinterpret_cast<const uint4 *>(brow[i] + k)
                               : make_uint4(0, 0, 0, 0);
    if (AMODE == A_CONVCL16) {
      tapc += BK;
      while (tapc >= cin) {
        tapc -= cin;
        ++tap;
      }
    }
  };
  auto stash = [&](int buf) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      *reinterpret_cast<uint4 *>(&sA[buf][(crow + 64 * i) * LDT + ccol]) = pa[i];
      if (EPI != EPI_S8) xs[i] += sum16(pa[i]);
    }
#pragma unroll
    for (int i = 0; i < 2; ++i)
      *reinterpret_cast<uint4 *>(&sB[buf][(crow + 64 * i) * LDT + ccol]) = pb[i];
  };

  v16i acc[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0;

  const int nk = (K + BK - 1) / BK;
  fetch(0);
  stash(0);
  if (GELU && tid < 16) sLut[tid] = g.lut[tid];
  __syncthreads();

  // Fragments: lane l reads row l % 32, bytes [(l / 32) * 16, +16) of each
  // 32-wide K step, for A and B alike.
  const int frow = lane & 31;
  const int fk = (lane >> 5) * 16;
  const int8_t *pA0 = &sA[0][(wm * 128 + frow) * LDT + fk];
  const int8_t *pB0 = &sB[0][(wn * 64 + frow) * LDT + fk];

  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < nk) fetch((kt + 1) * BK);
    const int8_t *pA = pA0 + cur * (BM * LDT);
    const int8_t *pB = pB0 + cur * (BN * LDT);
#pragma unroll
    for (int ks = 0; ks < BK; ks += 32) {
      v4i fa[4], fb[2];
#pragma unroll
      for (int i = 0; i < 4; ++i) fa[i] = *reinterpret_cast<const v4i *>(pA + i * 32 * LDT + ks);
#pragma unroll
      for (int j = 0; j < 2; ++j) fb[j] = *reinterpret_cast<const v4i *>(pB + j * 32 * LDT + ks);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[i], fb[j], acc[i][j], 0, 0, 0);
    }
    if (kt + 1 < nk) stash(cur ^ 1);
    __syncthreads();
  }

  // Row sums of A for the zero-point term (per-tensor requant has none).
  if (EPI != EPI_S8) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      int32_t s = xs[i];
      s += __shfl_xor(s, 1);
      s += __shfl_xor(s, 2);
      if ((tid & 3) == 0) sXsum[crow + 64 * i] = s;
    }
    __syncthreads();
  }

  // Epilogue. 32x32 MFMA output layout: lane l holds column l % 32 and, for
  // register r, row (r / 4) * 8 + (l / 32) * 4 + (r % 4).
  constexpr int OB = (EPI == EPI_L8 || (EPI == EPI_S8 && !PE)) ? 1 : (EPI == EPI_L32 ? 4 : 2);
  const int64_t ldo = g.ldc * OB;
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int n = n0 + wn * 64 + j * 32 + (lane & 31);
    if (n >= g.N) continue;
    const ColParams c = load_col<EPI>(g, n);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int lrow0 = wm * 128 + i * 32 + q * 8 + (lane >> 5) * 4;
        const int mrow = m0 + lrow0;
        if (mrow >= g.M) continue;
        int4 x4 = make_int4(0, 0, 0, 0);
        if (EPI != EPI_S8) x4 = *reinterpret_cast<const int4 *>(&sXsum[lrow0]);
        const int32_t xsv[4] = {x4.x, x4.y, x4.z, x4.w};
        char *orow = reinterpret_cast<char *>(g.out) + (int64_t)mrow * ldo + (int64_t)n * OB;
        int t = 0;
        if (PE) t = mrow % (int)g.pe_T;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          if (mrow + e >= g.M) break;
          const int32_t a = (int32_t)corrected(acc[i][j][q * 4 + e], xsv[e], c);
          char *o = orow + e * ldo;
          if (EPI == EPI_L8 || EPI == EPI_S8) {
            int32_t y = clampi(apply_shift(mulh_su(a, c.mult), c.shift), -127, 127);
            if (GELU) y = gelu_dec(y, sLut, c);
            if (PE) {
              // add_requant15 of the positional embedding (add_requant15_scalar.cpp:29-81)
              const int32_t v = y + (int32_t)g.pe[(int64_t)t * g.N + n];
              const int32_t z = apply_shift((int32_t)((uint32_t)v * c.pe_m), c.pe_s);
              *reinterpret_cast<int16_t *>(o) = (int16_t)clampi(z, -16383, 16383);
              if (++t == (int)g.pe_T) t = 0;
            } else {
              *reinterpret_cast<int8_t *>(o) = (int8_t)y;
            }
          } else {
            const int32_t br = (int32_t)((uint32_t)mulh_su(a, c.mult) << c.shift.sh);
            if (EPI == EPI_L32) {
              *reinterpret_cast<int32_t *>(o) = br;
            } else {
              const int32_t res = g.res[(int64_t)(mrow + e) * g.ldres + n];
              const uint32_t v = (uint32_t)br + (uint32_t)(res * (int32_t)g.res_mult);
              const int32_t y = clampi(rshift_pos((int32_t)v, 15), -16383, 16383);
              *reinterpret_cast<int16_t *>(o) = (int16_t)y;
            }
          }
        }
      }
    }
  }
}

template <int AMODE, int EPI, int FLAGS>
int launch_big(const GemmArgs &g, hipStream_t s) {
  const int64_t tm = (g.M + BM - 1) / BM, tn = (g.N + BN - 1) / BN;
  const int64_t tiles = tm * tn;
  if (tiles == 0) return 0;
  if (g.M > 0x7fffff00LL || g.N > 0x7fffff00LL || g.K > 0x7fffff00LL || tiles > 0x3fffffffLL)
    return fail("GEMM too large for the 256x128 tile kernel");
  const int per_xcd = (int)((tiles + XCDS - 1) / XCDS);
  hipLaunchKernelGGL((gemm_big_kernel<AMODE, EPI, FLAGS>), dim3((unsigned)(per_xcd * XCDS)),
                     dim3(NT), 0, s, g, (int)tn, (int)tiles, per_xcd);
  return check_launch("gemm_big_kernel");
}

}  // namespace

// Dispatch for operands that satisfy the 16-byte fast path (checked by the caller).
int gemm_big(const GemmArgs &g, bool conv_cl, hipStream_t s) {
  const bool gelu = g.lut != nullptr, pe = g.pe != nullptr;
  if (conv_cl) {
    if (g.epi != EPI_S8) return fail("conv GEMM supports the per-tensor int8 epilogue only");
    if (gelu && pe) return launch_big<A_CONVCL16, EPI_S8, F_GELU | F_PE>(g, s);
    if (gelu) return launch_big<A_CONVCL16, EPI_S8, F_GELU>(g, s);
    if (pe) return launch_big<A_CONVCL16, EPI_S8, F_PE>(g, s);
    return launch_big<A_CONVCL16, EPI_S8, 0>(g, s);
  }
  if (pe) return fail("the positional add_requant15 epilogue is for the channels-last conv");
  switch (g.epi) {
    case EPI_L8:
      if (gelu) return launch_big<A_DENSE16, EPI_L8, F_GELU>(g, s);
      return launch_big<A_DENSE16, EPI_L8, 0>(g, s);
    case EPI_L32: return launch_big<A_DENSE16, EPI_L32, 0>(g, s);
    case EPI_L32RES: return launch_big<A_DENSE16, EPI_L32RES, 0>(g, s);
    case EPI_S8:
      if (gelu) return launch_big<A_DENSE16, EPI_S8, F_GELU>(g, s);
      return launch_big<A_DENSE16, EPI_S8, 0>(g, s);
    default: return fail("unknown GEMM epilogue");
  }
}

}  // namespace iw
