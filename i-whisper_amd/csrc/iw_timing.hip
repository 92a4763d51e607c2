// Word-timestamp kernels: dynamic time warping over an alignment cost matrix
// and a sliding median filter (the reference's GPU path, triton_ops.py:13-109,
// used by timing.py:19-55 and :108-141). Both are float32 and exact: each
// DTW cell is one addition after a three-way minimum, the median is a
// selection.
#include "iw_common.hpp"
#include "iw_kernels.hpp"

namespace iw {

namespace {

constexpr int kDtwThreads = 1024;  // one thread per row of x (rows < 1024)

// Cost recurrence over the (M+1) x (N+1) matrix with cost[0][0] = 0 and
// +inf on the other borders: cost[i][j] = x[i-1][j-1] + min(c0, c1, c2) with
// c0 = cost[i-1][j-1], c1 = cost[i-1][j], c2 = cost[i][j-1]; trace[i][j] is
// the first of 0, 1, 2 whose cost equals that minimum (the order in which the
// reference kernel's three masked stores overwrite each other,
// triton_ops.py:35-38). One block walks the anti-diagonals k = i + j; thread
// i owns row i and the last two diagonals stay in LDS, indexed by row.
__global__ __launch_bounds__(kDtwThreads) void dtw_kernel(const float *__restrict__ x, int M, int N, int64_t ld,
                                                          int8_t *__restrict__ trace, int64_t tld) {
  __shared__ float sD[3][kDtwThreads + 1];  // diagonal k at sD[k % 3][i], i = 0 .. M
  const int i = threadIdx.x;                 // row 0 .. M (M < 1024)
  const float inf = __builtin_inff();
  // trace borders as the backtrace reads them (timing.py:59-60)
  for (int j = i; j <= N; j += blockDim.x) trace[j] = 2;
  for (int r = i; r <= M; r += blockDim.x) trace[(int64_t)r * tld] = 1;
  // diagonals 0 and 1: cost[0][0] = 0, everything else on them is a border
  if (i <= M) {
    sD[0][i] = i == 0 ? 0.f : inf;
    sD[1][i] = inf;
  }
  __syncthreads();
  // x along the anti-diagonals, requested one group of G diagonals ahead so
  // the loads never stall the recurrence
  constexpr int G = 8;
  auto load_x = [&](int k) -> float {
    const int j = k - i;
    return (i >= 1 && i <= M && j >= 1 && j <= N) ? x[(int64_t)(i - 1) * ld + (j - 1)] : 0.f;
  };
  float cur[G], nxt[G];
#pragma unroll
  for (int g = 0; g < G; ++g) cur[g] = load_x(2 + g);
  for (int k0 = 2; k0 <= M + N; k0 += G) {
#pragma unroll
    for (int g = 0; g < G; ++g) nxt[g] = load_x(k0 + G + g);
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const int k = k0 + g;
      if (k > M + N) break;  // uniform
      const float *d1 = sD[(k - 1) % 3];
      const float *d2 = sD[(k - 2) % 3];
      float v = inf;
      const int j = k - i;
      if (i >= 1 && i <= M && j >= 1 && j <= N) {
        const float c0 = d2[i - 1], c1 = d1[i - 1], c2 = d1[i];
        int8_t t;
        float c;
        if (c0 <= c1 && c0 <= c2) {
          c = c0, t = 0;
        } else if (c1 <= c0 && c1 <= c2) {
          c = c1, t = 1;
        } else {
          c = c2, t = 2;
        }
        v = __fadd_rn(cur[g], c);
        trace[(int64_t)i * tld + j] = t;
      }
      // row 0 of every diagonal k >= 1 is a border (+inf), as are rows whose
      // column is outside 1 .. N
      if (i <= M) sD[k % 3][i] = v;
      __syncthreads();
    }
#pragma unroll
    for (int g = 0; g < G; ++g) cur[g] = nxt[g];
  }
}

// Median of the `width` values of a reflect-padded window (timing.py:19-55:
// F.pad(mode="reflect") then unfold/sort, middle element), one output per
// thread. Widths are odd and at most kMaxMedianWidth; the window is sorted
// in registers by insertion (NaN inputs are not ordered as torch.sort orders
// them).
constexpr int kMaxMedianWidth = 31;

template <int W>
__device__ __forceinline__ float median_of(const float *__restrict__ xr, int n, int t) {
  float v[W];
  const int p = W / 2;
#pragma unroll
  for (int q = 0; q < W; ++q) {
    int s = t - p + q;
    s = s < 0 ? -s : (s >= n ? 2 * (n - 1) - s : s);  // reflect, edge not repeated
    v[q] = xr[s];
  }
#pragma unroll
  for (int a = 1; a < W; ++a) {
#pragma unroll
    for (int b = a; b > 0; --b) {
      const float lo = fminf(v[b - 1], v[b]), hi = fmaxf(v[b - 1], v[b]);
      v[b - 1] = lo;
      v[b] = hi;
    }
  }
  return v[p];
}

template <int W>
__global__ __launch_bounds__(256) void median_kernel(const float *__restrict__ x, int64_t rows, int n, int64_t ld,
                                                     float *__restrict__ y, int64_t ldy) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= rows * n) return;
  const int64_t r = idx / n;
  const int t = (int)(idx - r * n);
  y[r * ldy + t] = median_of<W>(x + r * ld, n, t);
}

// runtime width -> template instance (odd widths up to kMaxMedianWidth)
template <int W>
int launch_median_w(int width, const float *x, int64_t rows, int n, int64_t ld, float *y, int64_t ldy,
                    hipStream_t s) {
  if constexpr (W > kMaxMedianWidth) {
    return fail("median filter width must be odd and at most 31");
  } else {
    if (width != W) return launch_median_w<W + 2>(width, x, rows, n, ld, y, ldy, s);
    const int64_t total = rows * n;
    hipLaunchKernelGGL((median_kernel<W>), dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, x, rows, n, ld,
                       y, ldy);
    return check_launch("median_kernel");
  }
}

}  // namespace

int launch_dtw(const float *x, int64_t M, int64_t N, int64_t ld, int8_t *trace, int64_t tld, hipStream_t s) {
  hipLaunchKernelGGL(dtw_kernel, dim3(1), dim3(kDtwThreads), 0, s, x, (int)M, (int)N, ld, trace, tld);
  return check_launch("dtw_kernel");
}

int launch_median_filter(const float *x, int64_t rows, int64_t cols, int64_t ld, int32_t width, float *y,
                         int64_t ldy, hipStream_t s) {
  if (rows == 0) return 0;
  return launch_median_w<1>(width, x, rows, (int)cols, ld, y, ldy, s);
}

}  // namespace iw
