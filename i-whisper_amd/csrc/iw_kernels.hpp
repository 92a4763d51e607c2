// Launch wrappers shared between the kernel files and the C ABI (iw_api.hip).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#define IW_SEXP_LUT 32768  // shift-exp table entries (one byte each)

namespace iw {

struct FragPrefetch;  // iw_gemm.hpp

// Fused attention arguments. Element (b, t, h, d) of a [B, T, H*D] operand
// lives at base + b * sb + t * st + h * D + d. V is given transposed per
// head: vt + b * v_sb + h * v_sh + d * v_sd + t (prefill: v_sh = D * vt_ld,
// v_sd = vt_ld, v_sb = H * D * vt_ld); the decode kernels over caches also
// take it in key quads (v_sq != 4, v_sd = 4): vt + b * v_sb + h * v_sh +
// (t / 4) * v_sq + 4 d + t % 4.
struct AttnArgs {
  const int8_t *q = nullptr;
  int64_t q_sb = 0, q_st = 0;
  const int8_t *k = nullptr;
  int64_t k_sb = 0, k_sh = 0, k_st = 0;  // decode: explicit per-head stride
  const int8_t *vt = nullptr;
  int64_t v_sb = 0, v_sh = 0, v_sd = 0, vt_ld = 0;
  int64_t v_sq = 4;  // key-quad stride; 4 = transposed rows
  int8_t *out = nullptr;
  int64_t o_sb = 0, o_st = 0;
  const uint8_t *mask = nullptr;  // [Tq][Tk] bool bytes, or null
  int32_t B = 0, H = 0, Tq = 0, Tk = 0, D = 0;
  uint32_t qk_m = 0;   // uint8 multiplier
  uint32_t qk_s = 0;   // shift clamped at 0
  int32_t frac_bits = 7;
  uint32_t av_m = 0;   // uint8 multiplier
  uint32_t av_s = 0;   // shift clamped to [0, 32]
  uint32_t rsqrt_off = 16;
  const uint8_t *lut = nullptr;  // IW_SEXP_LUT entries for frac_bits
  int32_t max_tk = 0;            // decode over caches: bound of Tk + *pos
  int64_t o_frag_kp = 0;         // decode over caches: > 0 writes out fragment-major [B][H*D]
};

// The LayerNorm and query projection that the fused decode cross-attention
// (launch_attn_decode_cross_lnq) runs for its (batch, head) before the
// attention: LayerNorm32 of residual row b (x + b * ldx, C = hidden int16)
// with the LayerNorm's parameters, then the head's 64 query channels
// h * 64 .. +63 of Linear8 over the fragment-major weight wq ([C][kp], kp =
// frag_kpad(C)) with per-channel bias / weight zero point / multiplier /
// shift (bias and wz may be null).
struct LnQueryArgs {
  const int16_t *x = nullptr;
  int64_t ldx = 0;
  const int8_t *gamma = nullptr;
  const int32_t *beta = nullptr;
  uint32_t ln_m = 0;
  int32_t ln_s = 0;
  uint32_t out_m = 0;
  int32_t out_s = 0;
  uint32_t rsqrt_off = 0;
  int32_t code = 0;    // layernorm_width_code(hidden)
  int32_t hidden = 0;
  const int8_t *wq = nullptr;
  int64_t kp = 0;
  const int32_t *bias = nullptr;
  const int8_t *wz = nullptr;
  const uint32_t *mult = nullptr;
  const int8_t *shift = nullptr;
};

int layernorm_width_code(int64_t h);
// out_frag: out is the fragment-major image of [rows][hidden] (rows <= 128)
int launch_layernorm32(const int16_t *x, const int8_t *gamma, const int32_t *beta, uint8_t ln_m,
                       int8_t ln_s, uint32_t out_m, int8_t out_s, uint32_t rsqrt_off, int8_t *out,
                       int64_t rows, int64_t hidden, hipStream_t s, bool out_frag = false,
                       const FragPrefetch *pf = nullptr);
int launch_rsqrt(const int32_t *x, int32_t *out, int64_t n, uint32_t off, hipStream_t s);
int launch_gelu(const int8_t *x, const uint8_t *lut, const uint8_t *luti_m, const int8_t *luti_s,
                const uint8_t *luto_m, const int8_t *luto_s, int8_t *out, int64_t numel,
                int64_t channels, int luti_pc, int luto_pc, hipStream_t s);
int launch_residual15(const int32_t *br, const int16_t *res, uint16_t m, int16_t *out, int64_t n,
                      hipStream_t s);
int launch_add_requant15(const int8_t *x, const int64_t *tokens, const int8_t *addend,
                         const uint16_t *mult, const int8_t *shift, int16_t *out, int64_t batch,
                         int64_t positions, int64_t channels, int mpc, int spc, hipStream_t s,
                         const int32_t *pos = nullptr, int64_t addend_rows = 0);
// argmax of each logits row into next (and history[row][*step] when
// *step < hist_cols), then *step += 1, *pos += pos_inc
int launch_greedy_step(const int8_t *logits, int64_t rows, int64_t cols, int64_t ld, int64_t *next,
                       int64_t *history, int64_t hist_ld, int64_t hist_cols, int32_t *step,
                       int32_t *pos, int32_t pos_inc, hipStream_t s);
int launch_quantize_mel(const float *mel, float alpha, int8_t *out, int64_t b, int64_t m,
                        int64_t t, hipStream_t s);
int launch_log_mel(const float *audio, int64_t batch, int64_t n_samples, int64_t audio_ld, const float *twiddle,
                   const float *window, const int *fstart, const int *flen, const int *foff, const float *fw,
                   int n_taps, int n_mels, float *out, int64_t out_ld_b, float *blockmax, hipStream_t s);
int log_mel_limits(int *max_mels, int *max_taps);
// this device's IW_LOG_MEL_SCRATCH_FLOATS-float block-maxima array (the
// stream must belong to the current device)
int log_mel_scratch(hipStream_t stream, float **ptr);
int launch_dtw(const float *x, int64_t M, int64_t N, int64_t ld, int8_t *trace, int64_t tld, hipStream_t s);
int launch_median_filter(const float *x, int64_t rows, int64_t cols, int64_t ld, int32_t width, float *y,
                         int64_t ldy, hipStream_t s);
int launch_greedy_step_filtered(const int8_t *logits, int64_t rows, int64_t cols, int64_t ld, int64_t *next,
                                int64_t *history, int64_t hist_ld, int64_t hist_cols, int32_t *step,
                                int32_t *pos, int32_t pos_inc, const uint32_t *mask, const uint32_t *mask_first,
                                const int64_t *prev0, int32_t eot, int32_t ts_begin, int32_t max_init,
                                float scale, float *sum_logprobs, int32_t *eot_count, hipStream_t s);
// GreedyDecoder.update from the classifier's per-tile row maxima (or the
// logits), with optional log-probability sum, EOT freeze and EOT count
int launch_greedy_update(const uint16_t *amax, int64_t tiles, const int8_t *logits, int64_t ld, int64_t rows,
                         int64_t cols, int64_t *next, int64_t *history, int64_t hist_ld, int64_t hist_cols,
                         int32_t *step, int32_t *pos, int32_t pos_inc, int32_t eot, const int64_t *prev0,
                         float *sum_logprobs, float scale, int32_t *eot_count, uint32_t *arrive, hipStream_t s);
int launch_token_prob(const int8_t *logits, int64_t rows, int64_t cols, int64_t ld, int64_t token, float scale,
                      float *out, hipStream_t s);
int launch_argmax_rows(const int8_t *x, int64_t rows, int64_t cols, int64_t ld, int64_t *out,
                       hipStream_t s);
// dst[b*dst_sb + h*dst_sh + d*dst_sd + (t/4)*dst_sq + t%4] for t = t_off + i
int launch_transpose_heads(const int8_t *src, int64_t src_sb, int64_t src_st, int8_t *dst,
                           int64_t dst_sb, int64_t dst_sh, int64_t dst_sd, int64_t dst_sq, int64_t t_off,
                           int64_t B, int64_t T, int64_t H, int64_t D, hipStream_t s);
int launch_gather_heads(const int8_t *src, int64_t src_sb, int64_t src_st, int8_t *dst,
                        int64_t dst_sb, int64_t dst_sh, int64_t dst_st, int64_t t_off, int64_t B,
                        int64_t T, int64_t H, int64_t D, hipStream_t s);
int launch_copy_rows(const int8_t *src, int64_t src_sb, int64_t src_st, int8_t *dst,
                     int64_t dst_sb, int64_t dst_st, int64_t t_off, int64_t B, int64_t T,
                     int64_t C, hipStream_t s);

int launch_qk_requant_rowmax(const int8_t *q, const int8_t *k, const uint8_t *mask, int16_t *qk,
                             int16_t *rmp1, int64_t bh, int64_t tq, int64_t tk, int64_t dim,
                             uint8_t m, int32_t shift, hipStream_t s);
int launch_shift_exp(const int16_t *qk, const int16_t *rmp1, const uint8_t *mask, uint8_t *p,
                     int32_t *row_sum, int64_t bh, int64_t tq, int64_t tk, int32_t f,
                     hipStream_t s);
int launch_pv_norm_requant(const uint8_t *p, const int8_t *v, const int32_t *row_sum, uint8_t av_m,
                           int8_t av_s, uint32_t off, int8_t *out, int64_t batch, int64_t heads,
                           int64_t tq, int64_t tk, int64_t dim, hipStream_t s);
int launch_shift_exp_lut(uint8_t *lut, int32_t f, hipStream_t s);
int launch_attn_prefill(const AttnArgs &a, int max_blocks, hipStream_t s);
int launch_attn_decode(const AttnArgs &a, hipStream_t s);
// Decode attention over [B,H,T_cap,D] / [B,H,D,T_cap16] caches; key count
// a.Tk + *pos (pos may be null). At most 4096 keys.
constexpr int kDecodeCacheMaxKeys = 4096;
// tail: the next GEMM's weight, read into L2 by the self-attention kernel's
// last blocks (V in key quads, at most 512 keys), or null
int launch_attn_decode_cache(const AttnArgs &a, const int32_t *pos, hipStream_t s,
                             const FragPrefetch *tail = nullptr);
// Decode cross-attention (one query per (batch, head), keys 0 .. a.Tk - 1,
// V transposed, head_dim 64) whose query the kernel computes itself from
// lq; a.q unused. a.o_frag_kp as for launch_attn_decode_cache.
int launch_attn_decode_cross_lnq(const AttnArgs &a, const LnQueryArgs &lq, hipStream_t s);

}  // namespace iw
