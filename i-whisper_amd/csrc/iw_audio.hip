// Log-mel front end (i_whisper/audio.py:216-267) in float32: centred STFT
// frames of a periodic Hann window with reflect padding, |X|^2, the mel
// filterbank, log10 of max(., 1e-10); then per audio the floor
// max(log, max_all - 8) and log / 4 + 1.
#include "../../include/iwhisper_amd.h"
#include "iw_common.hpp"
#include "iw_kernels.hpp"

#include <mutex>

// Block maxima of iw_log_mel_noalloc: a fixed device array instead of a
// caller workspace, for callers that cannot allocate. Each GPU holds its own
// copy (at its own address, looked up once per device below) until the process
// ends; every call on one GPU shares it, so calls that overlap on one GPU race.
static __device__ __align__(256) float scratch[IW_LOG_MEL_SCRATCH_FLOATS];

namespace iw {

namespace {
constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mu;
float *g_scratch_ptr[kMaxScratchDevices] = {};
}  // namespace

int log_mel_scratch(hipStream_t stream, float **ptr) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxScratchDevices)
    return fail("iw_log_mel_noalloc: no usable current device");
  if (stream != nullptr) {
    hipDevice_t sdev = -1;
    if (hipStreamGetDevice(stream, &sdev) != hipSuccess || sdev != dev)
      return fail("iw_log_mel_noalloc: the stream does not belong to the current device");
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    // device address of this device's copy (the host-side name `scratch` is
    // not a device address and is never passed to a kernel)
    void *p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr)
      return fail(std::string("iw_log_mel_noalloc: hipGetSymbolAddress failed: ") + hipGetErrorString(e));
    g_scratch_ptr[dev] = static_cast<float *>(p);
  }
  *ptr = g_scratch_ptr[dev];
  return IW_OK;
}

namespace {

constexpr int kFft = 512;         // N_FFT
constexpr int kBins = kFft / 2 + 1;
constexpr int kFramesPerBlock = 64;
constexpr int kMaxMels = 128;
constexpr int kMaxFilterTaps = 2048;  // nonzero filterbank weights

__device__ __forceinline__ int bitrev9(int n) { return (int)(__brev((unsigned)n) >> 23); }

// One block = 4 waves = 64 consecutive frames of one audio (16 per wave, one
// at a time). A frame's 512-point transform is an in-place radix-2
// decimation-in-time FFT in the wave's own LDS buffer (bit-reversed load,
// 9 butterfly stages, twiddles exp(-2 pi i j / 512) from a table computed in
// float64 on the host). Each mel bin then sums its filter's nonzero taps
// (sparse rows: first bin, tap count, offset into the weights), and the
// block writes [n_mels][64] rows of log10 values plus its maximum.
__global__ __launch_bounds__(256) void logmel_kernel(const float *__restrict__ audio, int64_t n_samples,
                                                     int64_t audio_ld, const float2 *__restrict__ twiddle,
                                                     const float *__restrict__ window, const int *__restrict__ fstart,
                                                     const int *__restrict__ flen, const int *__restrict__ foff,
                                                     const float *__restrict__ fw, int n_taps, int n_mels,
                                                     int n_frames, float *__restrict__ out, int64_t out_ld_b,
                                                     float *__restrict__ blockmax) {
  __shared__ float sRe[4][kFft], sIm[4][kFft];
  __shared__ float2 sTw[kFft / 2];
  __shared__ float sWin[kFft];
  __shared__ int sStart[kMaxMels], sLen[kMaxMels], sOff[kMaxMels];
  __shared__ float sW[kMaxFilterTaps];
  __shared__ float sOut[kMaxMels][kFramesPerBlock + 1];
  __shared__ float sMax[4];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t b = blockIdx.y;
  const int t0 = blockIdx.x * kFramesPerBlock;
  const float *x = audio + b * audio_ld;
  for (int i = tid; i < kFft / 2; i += 256) sTw[i] = twiddle[i];
  for (int i = tid; i < kFft; i += 256) sWin[i] = window[i];
  for (int i = tid; i < n_mels; i += 256) sStart[i] = fstart[i], sLen[i] = flen[i], sOff[i] = foff[i];
  for (int i = tid; i < n_taps; i += 256) sW[i] = fw[i];
  __syncthreads();

  float vmax = -__builtin_inff();
  float *re = sRe[wave], *im = sIm[wave];
  for (int q = 0; q < kFramesPerBlock / 4; ++q) {
    const int fl = wave * (kFramesPerBlock / 4) + q;  // frame within the block
    const int t = t0 + fl;
    if (t >= n_frames) break;  // uniform per wave
    // windowed frame t: padded samples [t*160, t*160 + 512) of the signal
    // reflect-padded by 256 on each side (torch.stft center=True)
    for (int n = lane; n < kFft; n += 64) {
      int64_t u = (int64_t)t * 160 - kFft / 2 + n;
      u = u < 0 ? -u : (u >= n_samples ? 2 * (n_samples - 1) - u : u);
      const int r = bitrev9(n);
      re[r] = __fmul_rn(x[u], sWin[n]);
      im[r] = 0.f;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    for (int s = 1; s <= 9; ++s) {
      const int half = 1 << (s - 1);
      const int tstep = kFft >> s;  // twiddle index stride
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int j = lane + 64 * u;  // butterfly 0 .. 255
        const int pos = j & (half - 1);
        const int i0 = ((j >> (s - 1)) << s) + pos, i1 = i0 + half;
        const float2 w = sTw[pos * tstep];
        const float ar = re[i1], ai = im[i1];
        const float tr = __fsub_rn(__fmul_rn(w.x, ar), __fmul_rn(w.y, ai));
        const float ti = __fadd_rn(__fmul_rn(w.x, ai), __fmul_rn(w.y, ar));
        const float br = re[i0], bi = im[i0];
        re[i1] = __fsub_rn(br, tr);
        im[i1] = __fsub_rn(bi, ti);
        re[i0] = __fadd_rn(br, tr);
        im[i0] = __fadd_rn(bi, ti);
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
    // power spectrum of bins 0 .. 256, into re[]
    for (int k = lane; k < kBins; k += 64) re[k] = __fadd_rn(__fmul_rn(re[k], re[k]), __fmul_rn(im[k], im[k]));
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    for (int m = lane; m < n_mels; m += 64) {
      float acc = 0.f;
      const int st = sStart[m], len = sLen[m], off = sOff[m];
      for (int e = 0; e < len; ++e) acc = __fmaf_rn(sW[off + e], re[st + e], acc);
      const float lv = log10f(fmaxf(acc, 1e-10f));
      sOut[m][fl] = lv;
      vmax = fmaxf(vmax, lv);
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }
  // block maximum and the [n_mels][64] rows
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) vmax = fmaxf(vmax, __shfl_xor(vmax, o));
  if (lane == 0) sMax[wave] = vmax;
  __syncthreads();
  if (tid == 0) blockmax[b * gridDim.x + blockIdx.x] = fmaxf(fmaxf(sMax[0], sMax[1]), fmaxf(sMax[2], sMax[3]));
  const int nf = min(kFramesPerBlock, n_frames - t0);
  for (int i = tid; i < n_mels * kFramesPerBlock; i += 256) {
    const int m = i / kFramesPerBlock, f = i % kFramesPerBlock;
    if (f < nf) out[b * out_ld_b + (int64_t)m * n_frames + t0 + f] = sOut[m][f];
  }
}

// log_spec = max(log_spec, max(log_spec) - 8) / 4 + 1 over one audio
__global__ __launch_bounds__(256) void logmel_finish_kernel(float *__restrict__ out, int64_t out_ld_b, int64_t count,
                                                            const float *__restrict__ blockmax, int nblk) {
  __shared__ float sM[4];
  const int64_t b = blockIdx.y;
  const int tid = threadIdx.x;
  float m = -__builtin_inff();
  for (int i = tid; i < nblk; i += 256) m = fmaxf(m, blockmax[b * nblk + i]);
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
  if ((tid & 63) == 0) sM[tid >> 6] = m;
  __syncthreads();
  const float floor8 = __fsub_rn(fmaxf(fmaxf(sM[0], sM[1]), fmaxf(sM[2], sM[3])), 8.0f);
  float *o = out + b * out_ld_b;
  for (int64_t i = (int64_t)blockIdx.x * 256 + tid; i < count; i += (int64_t)gridDim.x * 256)
    o[i] = __fadd_rn(__fmul_rn(fmaxf(o[i], floor8), 0.25f), 1.0f);
}

}  // namespace

int launch_log_mel(const float *audio, int64_t batch, int64_t n_samples, int64_t audio_ld, const float *twiddle,
                   const float *window, const int *fstart, const int *flen, const int *foff, const float *fw,
                   int n_taps, int n_mels, float *out, int64_t out_ld_b, float *blockmax, hipStream_t s) {
  const int n_frames = (int)(n_samples / 160);
  const int nblk = (n_frames + kFramesPerBlock - 1) / kFramesPerBlock;
  hipLaunchKernelGGL(logmel_kernel, dim3((unsigned)nblk, (unsigned)batch), dim3(256), 0, s, audio, n_samples,
                     audio_ld, reinterpret_cast<const float2 *>(twiddle), window, fstart, flen, foff, fw, n_taps,
                     n_mels, n_frames, out, out_ld_b, blockmax);
  int rc = check_launch("logmel_kernel");
  if (rc) return rc;
  const int64_t count = (int64_t)n_mels * n_frames;
  hipLaunchKernelGGL(logmel_finish_kernel, dim3(64, (unsigned)batch), dim3(256), 0, s, out, out_ld_b, count,
                     blockmax, nblk);
  return check_launch("logmel_finish_kernel");
}

int log_mel_limits(int *max_mels, int *max_taps) {
  *max_mels = kMaxMels;
  *max_taps = kMaxFilterTaps;
  return 0;
}

}  // namespace iw
