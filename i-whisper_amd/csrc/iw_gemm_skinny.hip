// Skinny int8 GEMM for the decoder (M = batch rows <= 128): Linear8 (+GeLU),
// Linear32 (+residual15), classifier, and the self-attention QKV projection
// whose epilogue writes Q to a buffer and appends K and V to the KV caches.
//
// Decode GEMMs read every weight byte once and little else, so the kernel is
// organised for HBM streaming, not MFMA reuse: one block of 8 waves per
// 32-column tile of the output; wave w takes m-subtile w % MS (32 rows) and
// the K slice w / MS of KS = 8 / MS slices, loads its 16-byte A and B
// fragments straight from global memory (A stays in L2, B streams from HBM),
// and runs v_mfma_i32_32x32x32_i8 on them. The slices' int32 partial sums are
// added in LDS (exact modulo 2^32 in any order), then all 512 threads run the
// epilogue, one column per 16 threads.
#include "iw_gemm_dev.hpp"

namespace iw {

using namespace gemm;

namespace {

constexpr int NT = 512;   // 8 waves
constexpr int TN = 32;    // output columns per block
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
      if (zp) {
        const int ones = 0x01010101;
        xs = __builtin_amdgcn_sdot4(fa[u][0], ones, xs, false);
        xs = __builtin_amdgcn_sdot4(fa[u][1], ones, xs, false);
        xs = __builtin_amdgcn_sdot4(fa[u][2], ones, xs, false);
        xs = __builtin_amdgcn_sdot4(fa[u][3], ones, xs, false);
      }
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
    a = corrected((int32_t)a, xsum, c);
    if (EPI == EPI_L8 || EPI == EPI_S8) {
      int32_t y = clampi(apply_shift(mulh_su((int32_t)a, c.mult), c.shift), -127, 127);
      if (GELU) y = gelu_dec(y, sLut, c);
      if (SCATTER) {
        // columns [0, C): Q; [C, 2C): K appended at position pos + (m % T)
        // of the [B, H, T_cache, D] cache; [2C, 3C): V appended to the
        // transposed [B, H, D, T_cache] cache
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
          sc.v[(int64_t)b * sc.v_sb + (int64_t)h * sc.v_sh + (int64_t)d * sc.v_sd + t] = (int8_t)y;
        }
      } else {
        reinterpret_cast<int8_t *>(g.out)[(int64_t)m * g.ldc + n] = (int8_t)y;
      }
    } else {
      const int32_t br = (int32_t)((uint32_t)mulh_su((int32_t)a, c.mult) << c.shift.sh);
      if (EPI == EPI_L32) {
        reinterpret_cast<int32_t *>(g.out)[(int64_t)m * g.ldc + n] = br;
      } else {
        const int32_t res = g.res[(int64_t)m * g.ldres + n];
        const uint32_t v = (uint32_t)br + (uint32_t)(res * (int32_t)g.res_mult);
        const int32_t y = clampi(rshift_pos((int32_t)v, 15), -16383, 16383);
        reinterpret_cast<int16_t *>(g.out)[(int64_t)m * g.ldc + n] = (int16_t)y;
      }
    }
  }
}

template <int EPI, bool GELU, bool SCATTER>
int launch_skinny(const GemmArgs &g, const SkinnyScatter &sc, hipStream_t s) {
  const int64_t tiles = (g.N + TN - 1) / TN;
  if (tiles == 0 || g.M == 0) return 0;
  const int ms = (int)((g.M + 31) / 32);
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
