// The classifier of the one-token decode step over a large vocabulary, on
// fragment-major operands (layout: iw_gemm.hpp, frag_offset): one
// persistent block per CU streams its column tiles' weights through an LDS
// ring against activations it holds in registers. It has the epilogue of
// gemm_frag's per-tensor classifier, optionally with the per-tile row maxima
// of the greedy step. A translation unit of its own, so that adding it left
// the other decode kernels' code objects as they were.
#include "iw_gemm_dev.hpp"

namespace iw {

using namespace gemm;

namespace {

// ---------------------------------------------------------------------------
// Classifier over a large vocabulary (Whisper: 51865 columns = 1621 column
// tiles for 256 CUs) with M <= 128 rows. The 32 x 32-tile kernel
// (gemm_frag_kernel, iw_gemm_frag.hip) reads the rows' activations again
// for every column tile (160 KB per tile at M = 128, K = 1280: 0.26 GB of L2
// reads per launch) and pays a block's load latency for each of the ~25
// blocks a CU runs. Here one persistent
// block per CU loads the activations into registers once and streams the
// weights of its column tiles t0, t0 + G, ... through an LDS ring:
//
// * 8 waves; wave w = (i, h) = (w / 2, w % 2) holds m-subtile i (rows
//   32 i .. +31) over K half h: SPW = Kp / 64 operand fragments.
// * The weights of tile t are 32 Kp contiguous bytes (fragment-major). The
//   block's j-th tile goes to ring slot j % NR, copied by all waves, CPW
//   1 KB copies each (copy indices past the tile repeat its last fragment,
//   writing the same bytes twice). Each wave waits for its own copies, and
//   a block barrier publishes the slot; wave (i, h) then multiplies its
//   fragments with K half h of the tile, read from LDS.
// * The two K halves of m-subtile i meet in LDS: wave h = 0 keeps
//   accumulator registers 0-7 (rows 0-15 of the subtile), h = 1 registers
//   8-15 (rows 16-31), each hands the other half to its partner, and after a
//   second barrier runs the epilogue on its 16 rows x 32 columns.
// * A tile's results are stored during the next tile, before that tile's
//   copies are issued, so the wait for a slot (vmcnt counts stores too)
//   never includes stores issued after the copies it waits for.
// ---------------------------------------------------------------------------
constexpr int kClsRing = 3;

template <int SPW, bool ARGMAX>
__global__ __launch_bounds__(512) void classifier_stream_kernel(GemmArgs g, int ms, int tiles, int kp) {
  constexpr int NR = kClsRing;
  constexpr int NF = 2 * SPW;            // k32 fragments per tile
  constexpr int CPW = (NF + 7) / 8;      // copies per wave per tile
  constexpr int SLOT = NF * 1024;        // bytes per ring slot
  __shared__ __attribute__((aligned(1024))) int8_t sRing[NR * SLOT];
  __shared__ uint32_t sX[8 * 8 * 64];    // [wave][register][lane]: the half handed to the partner

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int mi = wave >> 1, kh = wave & 1;
  const bool act = mi < ms;  // waves of m-subtiles past M only copy
  const int G = (int)gridDim.x, t0 = (int)blockIdx.x;
  const int nt = (tiles - t0 + G - 1) / G;  // tiles t0, t0 + G, ... (>= 1: G <= tiles)
  const int M = (int)g.M, N = (int)g.N;
  const ColParams c = decode_col<EPI_S8>(g, load_col_raw(g, 0));

  const uint32_t ring = __builtin_amdgcn_readfirstlane((uint32_t)reinterpret_cast<uintptr_t>(sRing));
  const int f0 = wave * CPW;
  auto issue = [&](int j) {
    const int8_t *src = g.b + (int64_t)(t0 + j * G) * 32 * kp + lane * 16;
    const uint32_t dst = ring + (uint32_t)((j % NR) * SLOT);
#pragma unroll
    for (int u = 0; u < CPW; ++u) {
      const int f = min(f0 + u, NF - 1);
      dma16_lds(src + f * 1024, dst + f * 1024);
    }
  };

  // The first tile's copies, then this wave's activation fragments, which the
  // compiler waits for (together with those copies) before the next tile's
  // copies are issued: no load it tracks is outstanding inside the loop, so
  // it adds no wait there.
  issue(0);
  v4i fa[SPW];
  if (act) {
    const int8_t *pa = g.a + ((int64_t)mi * (kp / 32) + kh * SPW) * 1024 + lane * 16;
#pragma unroll
    for (int s = 0; s < SPW; ++s) fa[s] = *reinterpret_cast<const v4i *>(pa + s * 1024);
#pragma unroll
    for (int s = 0; s < SPW; ++s) asm volatile("" ::"v"(fa[s]));
  }
  if (nt > 1) issue(1);

  // results of the previous tile, stored during the next one
  int32_t ys[8];
  uint32_t ks[8];
  int tprev = 0;
  auto store_prev = [&]() {
#pragma unroll
    for (int jj = 0; jj < 8; ++jj) {
      const int r = kh * 8 + jj;
      const int m = mi * 32 + (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
      const int n = tprev * 32 + (lane & 31);
      if (g.out && n < N && m < M) reinterpret_cast<int8_t *>(g.out)[(int64_t)m * g.ldc + n] = (int8_t)ys[jj];
      if (ARGMAX && (lane & 31) == 0 && m < M) g.amax[(int64_t)m * g.amax_ld + tprev] = (uint16_t)ks[jj];
    }
  };

  for (int j = 0; j < nt; ++j) {
    // this wave's copies of tile j have landed (those of tile j + 1 may be
    // in flight); the barrier makes every wave's copies visible and frees
    // the slot of tile j - 1, which every wave has read
    if (j + 1 < nt)
      wait_vm<CPW>();
    else
      wait_vm<0>();
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    if (act && j > 0) store_prev();
    if (j + NR - 1 < nt) issue(j + NR - 1);

    // every wave meets both barriers of every tile, also those that only copy
    const int t = t0 + j * G;
    uint32_t kept[8];
    if (act) {
      const int8_t *slot = sRing + (j % NR) * SLOT + kh * SPW * 1024 + lane * 16;
      v16i acc[2];
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[0][r] = acc[1][r] = 0;
#pragma unroll
      for (int s = 0; s < SPW; ++s) {
        const v4i fb = *reinterpret_cast<const v4i *>(slot + s * 1024);
        acc[s & 1] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[s], fb, acc[s & 1], 0, 0, 0);
      }
      // 32x32 MFMA layout: lane l holds column l % 32, register r row
      // (r / 4) * 8 + (l / 32) * 4 + r % 4 of the subtile
#pragma unroll
      for (int jj = 0; jj < 8; ++jj) {
        const int give = kh ? jj : 8 + jj, keep = kh ? 8 + jj : jj;
        sX[(wave * 8 + jj) * 64 + lane] = (uint32_t)acc[0][give] + (uint32_t)acc[1][give];
        kept[jj] = (uint32_t)acc[0][keep] + (uint32_t)acc[1][keep];
      }
    }
    lds_barrier();
    if (!act) continue;
#pragma unroll
    for (int jj = 0; jj < 8; ++jj) kept[jj] += sX[((wave ^ 1) * 8 + jj) * 64 + lane];

    // int8 logits (the per-tensor epilogue of skinny_store) and, with ARGMAX,
    // each row's first maximum in the tile: key (y + 128) << 5 | (31 - column),
    // the maximum over the 32 lanes of the row (16-lane DPP row maxima, then
    // lanes 16 / 48 read as scalars); padding columns take key 0
    const int n = t * 32 + (lane & 31);
#pragma unroll
    for (int jj = 0; jj < 8; ++jj) {
      const int r = kh * 8 + jj;
      const int m = mi * 32 + (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
      const int32_t y = clampi(apply_shift(mulh_su((int32_t)kept[jj], c.mult), c.shift), -127, 127);
      ys[jj] = y;
      if constexpr (ARGMAX) {
        int32_t k = (n < N && m < M) ? (int32_t)(((uint32_t)(y + 128) << 5) | (uint32_t)(31 - (n & 31))) : 0;
        k = max(k, __builtin_amdgcn_update_dpp(0, k, 0xB1, 0xf, 0xf, false));   // quad [1,0,3,2]
        k = max(k, __builtin_amdgcn_update_dpp(0, k, 0x4E, 0xf, 0xf, false));   // quad [2,3,0,1]
        k = max(k, __builtin_amdgcn_update_dpp(0, k, 0x141, 0xf, 0xf, false));  // row_half_mirror
        k = max(k, __builtin_amdgcn_update_dpp(0, k, 0x140, 0xf, 0xf, false));  // row_mirror
        const int32_t k16 = __builtin_amdgcn_readlane(k, 16), k48 = __builtin_amdgcn_readlane(k, 48);
        ks[jj] = (uint32_t)max(k, lane < 32 ? k16 : k48);
      }
    }
    tprev = t;
  }
  if (act) store_prev();
}

int classifier_stream_blocks() {
  static const int cus = [] {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) !=
                                                hipSuccess || n <= 0) {
      (void)hipGetLastError();
      return 256;
    }
    return n;
  }();
  return cus;
}

// The streaming classifier takes M <= 128 rows, Kp in {640, 960, 1280} and at
// least two column tiles per CU (fewer: the tile kernel's blocks already
// cover the machine, and a block would not reuse its activations).
}  // namespace

bool classifier_stream_eligible(const GemmArgs &g) {
  const int64_t kp = frag_kpad(g.K);
  const int64_t tiles = (g.N + 31) / 32;
  return g.M <= 128 && g.wz == nullptr && g.bias == nullptr && g.mult_pc == 0 &&
         (kp == 640 || kp == 960 || kp == 1280) && tiles >= 2 * (int64_t)classifier_stream_blocks();
}

namespace {

template <bool ARGMAX>
int launch_classifier_stream(const GemmArgs &g, int64_t kp, hipStream_t s) {
  const int tiles = (int)((g.N + 31) / 32);
  const int ms = (int)((g.M + 31) / 32);
  const dim3 grid((unsigned)min(tiles, classifier_stream_blocks()));
  switch (kp) {
    case 640:
      hipLaunchKernelGGL((classifier_stream_kernel<10, ARGMAX>), grid, dim3(512), 0, s, g, ms, tiles, (int)kp);
      break;
    case 960:
      hipLaunchKernelGGL((classifier_stream_kernel<15, ARGMAX>), grid, dim3(512), 0, s, g, ms, tiles, (int)kp);
      break;
    default:
      hipLaunchKernelGGL((classifier_stream_kernel<20, ARGMAX>), grid, dim3(512), 0, s, g, ms, tiles, (int)kp);
      break;
  }
  return check_launch("classifier_stream_kernel");
}


}  // namespace

int classifier_stream(const GemmArgs &g, hipStream_t s) {
  const int64_t kp = frag_kpad(g.K);
  return g.amax ? launch_classifier_stream<true>(g, kp, s) : launch_classifier_stream<false>(g, kp, s);
}

}  // namespace iw
