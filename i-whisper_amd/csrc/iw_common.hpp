// Shared device helpers for the I-Whisper integer kernels on gfx950.
//
// The fixed-point primitives restate i_whisper/kernels/csrc/common/fixedpoint.h:35-102
// bit for bit: mulh is the high word of the signed-by-unsigned 64-bit product,
// rshift rounds half away from zero with a modulo-2^32 add, shift 0 is the
// identity and shift >= 32 gives 0.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <string>

namespace iw {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

__device__ __forceinline__ int32_t mulh(int32_t x, uint32_t m) {
  return (int32_t)(((int64_t)x * (int64_t)(uint64_t)m) >> 32);
}

__device__ __forceinline__ int32_t rshift(int32_t x, uint32_t s) {
  if (s == 0) return x;
  if (s >= 32) return 0;
  uint32_t bias = (1u << (s - 1)) - ((uint32_t)x >> 31);
  return (int32_t)((uint32_t)x + bias) >> s;
}

// rshift for 1 <= s <= 31 known on entry (no special cases).
__device__ __forceinline__ int32_t rshift_pos(int32_t x, uint32_t s) {
  uint32_t bias = (1u << (s - 1)) + (uint32_t)(x >> 31);
  return (int32_t)((uint32_t)x + bias) >> s;
}

__device__ __forceinline__ int32_t clampi(int32_t v, int32_t lo, int32_t hi) {
  return min(max(v, lo), hi);
}

__device__ __forceinline__ uint32_t clamp_shift_0_32(int32_t s) {
  return (uint32_t)min(max(s, 0), 32);
}

// Integer GeLU on one int8 value (gelu/gelu_scalar.cpp:29-180).
__device__ __forceinline__ int8_t gelu_one(int32_t x, const uint8_t *lut, uint32_t luti_m,
                                           int32_t luti_s, uint32_t luto_m, int32_t luto_s) {
  int32_t idx = rshift(x * (int32_t)luti_m, clamp_shift_0_32(luti_s)) + 8;
  idx = clampi(idx, 0, 15);
  int32_t v = x * (int32_t)lut[idx];
  v = (int32_t)((uint32_t)v * luto_m);
  v = rshift(v, clamp_shift_0_32(luto_s));
  return (int8_t)clampi(v, -127, 127);
}

// Division by the LayerNorm width as adds and floor shifts
// (layernorm/layernorm_scalar.cpp:14-56), modulo 2^32; code 0..4 for the
// widths 384, 512, 768, 1024, 1280.
__device__ __forceinline__ int32_t norm_reduce(int32_t v, int code) {
  switch (code) {
    case 0: return (int32_t)((uint32_t)v + (uint32_t)(v >> 2) + (uint32_t)(v >> 3)) >> 9;
    case 1: return v >> 9;
    case 2: return (int32_t)((uint32_t)v + (uint32_t)(v >> 2) + (uint32_t)(v >> 3)) >> 10;
    case 3: return v >> 10;
    default: return (int32_t)((uint32_t)v + (uint32_t)(v >> 1)) >> 11;
  }
}

// Integer fast inverse square root, two Newton steps
// (layernorm/layernorm_scalar.cpp:309-438).
__device__ __forceinline__ int32_t bitlen(int32_t v) { return v == 0 ? 0 : 32 - __clz(v); }

__device__ inline int32_t fisr(int32_t x, uint32_t off) {
  int32_t i;
  if (x == 0) {
    i = 0;
  } else {
    int32_t e = bitlen(x) - 1;
    uint32_t ux = (uint32_t)x;
    uint32_t sig = e <= 23 ? (ux << (23 - e)) : (ux >> (e - 23));
    i = (int32_t)(((uint32_t)(e + 127) << 23) | (sig & 0x007FFFFFu));
  }
  i = (int32_t)(0x5f3759dfu - (uint32_t)(i >> 1));
  uint32_t raw = (uint32_t)i + (off << 23);
  int32_t e = (int32_t)((raw >> 23) & 0xFFu) - 127;
  uint64_t sig = (uint64_t)((1u << 23) | (raw & 0x007FFFFFu));
  int32_t y;
  if (e < 0) {
    y = 0;
  } else {
    uint64_t v = e >= 23 ? (sig << (e - 23)) : (sig >> (23 - e));
    y = (int32_t)(uint32_t)v;
  }
  uint32_t three = 3u << off;
  for (int it = 0; it < 2; ++it) {
    int32_t xy = (int32_t)((uint32_t)x * (uint32_t)y);
    int32_t xs = rshift(xy, off);
    uint32_t t = (uint32_t)xs * (uint32_t)y;
    int32_t prod = (int32_t)((uint32_t)y * (three - t));
    y = rshift(prod, off + 1);
  }
  return y;
}

// One lane of the shift-exponential (attention/attention_scalar.cpp:449-554),
// int16 arithmetic modulo 2^16. Used to fill the per-launch lookup table.
__device__ inline uint32_t shift_exp_one(int32_t x_sub16, int32_t f) {
  int16_t xs = (int16_t)x_sub16;
  if (xs > 0) return 0;
  int16_t half = (int16_t)(xs >> 1);
  int16_t six = (int16_t)(xs >> 4);
  int16_t fix = (int16_t)(uint16_t)((uint16_t)(uint16_t)(xs + half) - (uint16_t)six);
  int16_t xi = (int16_t)(fix >> f);
  int16_t ip = (int16_t)(uint16_t)(uint32_t)((int32_t)xi * (1 << f));
  int16_t frac = (int16_t)(uint16_t)(uint32_t)((int32_t)fix - (int32_t)ip);
  int16_t num = (int16_t)(uint16_t)(uint32_t)((1 << f) + (int32_t)(frac >> 1));
  int32_t e;
  if (xi > 0) {
    e = 0;
  } else {
    int32_t sh = -(int32_t)xi;
    e = sh >= 16 ? 0 : (int32_t)(int16_t)(num >> sh);
  }
  int32_t o = f > 7 ? (e >> (f - 7)) : e;
  return (uint32_t)(uint8_t)o;
}

// Sum over the four lanes of a DPP quad (xor-1 and xor-2 quad permutes), in
// every lane of it.
__device__ __forceinline__ int32_t quad_sum_dpp(int32_t v) {
  v += __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xf, 0xf, true);  // quad [1,0,3,2]
  return v + __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xf, 0xf, true);  // quad [2,3,0,1]
}

// Wave-wide sum / max with DPP moves (no LDS round trips): xor-1 and xor-2
// quad permutes, then the half-row and row mirrors give every lane its
// 16-lane row's total; the four rows are added from lanes 0, 16, 32, 48.
__device__ __forceinline__ uint32_t row16_sum(uint32_t v) {
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xB1, 0xf, 0xf, true);   // quad [1,0,3,2]
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x4E, 0xf, 0xf, true);   // quad [2,3,0,1]
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x141, 0xf, 0xf, true);  // row_half_mirror
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x140, 0xf, 0xf, true);  // row_mirror
  return v;
}
__device__ __forceinline__ uint32_t wave_sum_dpp(uint32_t v) {
  v = row16_sum(v);
  return (uint32_t)__builtin_amdgcn_readlane((int)v, 0) + (uint32_t)__builtin_amdgcn_readlane((int)v, 16) +
         (uint32_t)__builtin_amdgcn_readlane((int)v, 32) + (uint32_t)__builtin_amdgcn_readlane((int)v, 48);
}
__device__ __forceinline__ int32_t wave_max_dpp(int32_t v) {
  v = max(v, __builtin_amdgcn_update_dpp(INT32_MIN, v, 0xB1, 0xf, 0xf, false));
  v = max(v, __builtin_amdgcn_update_dpp(INT32_MIN, v, 0x4E, 0xf, 0xf, false));
  v = max(v, __builtin_amdgcn_update_dpp(INT32_MIN, v, 0x141, 0xf, 0xf, false));
  v = max(v, __builtin_amdgcn_update_dpp(INT32_MIN, v, 0x140, 0xf, 0xf, false));
  return max(max(__builtin_amdgcn_readlane(v, 0), __builtin_amdgcn_readlane(v, 16)),
             max(__builtin_amdgcn_readlane(v, 32), __builtin_amdgcn_readlane(v, 48)));
}

#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
// global_load_lds_dwordx4: lane l copies 16 bytes from src to LDS byte
// address lds + 16 l (lds wave-uniform). Inline assembly, so that the
// compiler adds no waits for it: its users wait on vmcnt themselves. No
// kernel using it keeps a value in M0.
__device__ __forceinline__ void dma16_lds(const int8_t *src, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(lds)
               : "memory", "m0");
}
#pragma clang diagnostic pop

template <int N>
__device__ __forceinline__ void wait_vm() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// s_waitcnt vmcnt(n * F) for a run-time n in [0, N]
template <int N, int F>
__device__ __forceinline__ void wait_vm_upto(int n) {
  if (n >= N) {
    wait_vm<N * F>();
  } else if constexpr (N > 0) {
    wait_vm_upto<N - 1, F>(n);
  }
}

// the LDS part of a barrier: this wave's LDS writes are done, then all waves
// meet (without __syncthreads' release fence, which would drain the
// outstanding global loads and LDS copies)
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

}  // namespace iw

// ---------------------------------------------------------------------------
// Host-side error plumbing for the C ABI: every entry point returns 0 on
// success or a negative code, and leaves a message for iw_last_error().
// ---------------------------------------------------------------------------
namespace iw {
void set_error(const std::string &msg);
int fail(const std::string &msg);  // sets the message, returns IW_EINVAL
int check_launch(const char *what);
}  // namespace iw

#define IW_REQUIRE(cond, msg) \
  do {                        \
    if (!(cond)) return ::iw::fail(msg); \
  } while (0)
