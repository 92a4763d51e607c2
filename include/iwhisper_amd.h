/*
 * iwhisper_amd.h - C ABI of the MI355X (gfx950) kernels for I-Whisper's
 * integer-only encoder/decoder path.
 *
 * Conventions
 *   - Every tensor argument is a DEVICE pointer to contiguous memory in the
 *     layout the reference uses for the same argument; the caller allocates
 *     inputs and outputs (nothing is returned by allocation).
 *   - Sizes are int64_t; scalar quantisation parameters are passed by value.
 *   - `stream` is a hipStream_t (NULL selects the null stream). Calls are
 *     asynchronous on that stream.
 *   - Return value: IW_OK (0) or a negative code; iw_last_error() then holds a
 *     message (per calling thread). No exception crosses the ABI.
 *   - Integer semantics are bit-exact with the reference's scalar kernels,
 *     including modulo-2^32 wrap of accumulators.
 *
 * Paths in the comments are relative to the reference repository root
 * (vcsd-lab/I-Whisper); each drop-in entry point names the function of the
 * reference's raw-pointer C++ API (csrc/<op>/<op>.h) and of its torch binding
 * (csrc/<op>/<op>_torch.cpp, bound in csrc/pybind.cpp) that it replaces.
 */
#ifndef IWHISPER_AMD_H
#define IWHISPER_AMD_H

#include <stdbool.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define IW_OK 0
#define IW_EINVAL (-1)  /* invalid argument (shape, size, parameter range) */
#define IW_ELAUNCH (-2) /* HIP runtime error at launch */

/* 2: iw_transpose_heads (dst_sq), iw_linear8_qkv_cache[_frag] and iw_attention_decode_cache (v_sq),
 * iw_attention_decode_cache_frag (v_sq, next-weight prefetch) and iw_greedy_advance_filtered
 * (sum_logprobs, eot_count) changed their argument lists; a caller built against version 1 must
 * not bind this library. */
#define IW_ABI_VERSION 2
#define IW_SHIFT_EXP_TABLE_BYTES 32768

typedef void *iw_stream_t; /* hipStream_t */

int iw_abi_version(void);
const char *iw_last_error(void);

/* ---------------------------------------------------------------------------
 * Drop-in replacements for the reference's per-op kernels.
 * ------------------------------------------------------------------------- */

/* Linear8: out[m,n] = clamp(requant(x.w + bias - wz*rowsum(x), mult[n], shift[n]), +-127).
 * Replaces iwhisper::linear8_simd (i_whisper/kernels/csrc/linear8/linear8.h:26-38)
 * behind _C.linear8_simd (linear8/linear8_torch.cpp:14-152, pybind.cpp:61-69).
 * x [M,K] int8, weight [N,K] int8, bias [N] int32, weight_zero [N] int8,
 * multiplier [N] uint32, shift [N] int8, out [M,N] int8. */
int iw_linear8(const int8_t *x, const int8_t *weight, const int32_t *bias,
               const int8_t *weight_zero, const uint32_t *multiplier, const int8_t *shift,
               int8_t *out, int64_t M, int64_t K, int64_t N, bool has_bias, bool asymmetric,
               iw_stream_t stream);

/* Linear32: out[m,n] = (int32)(mulh(acc, mult[n]) << shift[n]) (0 for shifts outside [0,31]).
 * Replaces iwhisper::linear32_simd (linear32/linear32.h:47-59) behind _C.linear32_simd
 * (linear32/linear32_torch.cpp:10-150, pybind.cpp:92-100). out [M,N] int32. */
int iw_linear32(const int8_t *x, const int8_t *weight, const int32_t *bias,
                const int8_t *weight_zero, const uint32_t *multiplier, const int8_t *shift,
                int32_t *out, int64_t M, int64_t K, int64_t N, bool has_bias, bool asymmetric,
                iw_stream_t stream);

/* LayerNorm32 over rows of width hidden in {384, 512, 768, 1024, 1280}.
 * Replaces iwhisper::layernorm32_simd (layernorm/layernorm.h:36-48) behind
 * _C.layernorm32_simd (layernorm/layernorm_torch.cpp:200-305, pybind.cpp:141-150, which fixes
 * rsqrt_offset = 13). x [rows,hidden] int16 -> out int8. */
int iw_layernorm32(const int16_t *x, const int8_t *weight, const int32_t *bias,
                   uint8_t ln_multiplier, int8_t ln_shift, uint32_t out_multiplier,
                   int8_t out_shift, uint32_t rsqrt_offset, int8_t *out, int64_t rows,
                   int64_t hidden, bool has_bias, iw_stream_t stream);

/* Integer fast inverse square root, elementwise.
 * Replaces iwhisper::layernorm32_rsqrt_scalar (layernorm/layernorm.h:30-34),
 * _C.layernorm32_rsqrt_scalar (pybind.cpp:195-199). */
int iw_layernorm32_rsqrt(const int32_t *x, int32_t *out, int64_t n, uint32_t offset,
                         iw_stream_t stream);

/* Integer GeLU (16-entry LUT). Parameter counts are 1 or channels.
 * Replaces iwhisper::gelu_simd (gelu/gelu.h:21-32) behind _C.gelu_simd
 * (gelu/gelu_torch.cpp:9-153, pybind.cpp:226-234). */
int iw_gelu(const int8_t *x, const uint8_t *lut, const uint8_t *luti_multiplier,
            const int8_t *luti_shift, const uint8_t *luto_multiplier, const int8_t *luto_shift,
            int8_t *out, int64_t numel, int64_t channels, int64_t luti_count,
            int64_t luto_count, iw_stream_t stream);

/* out = clamp(Rshift(branch + residual*multiplier, 15), +-16383) int16.
 * Replaces iwhisper::residual15_simd (residual15/residual15.h:15-20) behind
 * _C.residual15_simd (residual15/residual15_torch.cpp:7-70, pybind.cpp:122-127). */
int iw_residual15(const int32_t *branch, const int16_t *residual, uint16_t multiplier,
                  int16_t *out, int64_t numel, iw_stream_t stream);

/* out[b,t,c] = clamp(Rshift((x[b,t,c] + addend[t,c]) * m, max(s,0)), +-16383) int16.
 * Replaces iwhisper::add_requant15_simd (add_requant15/add_requant15.h:17-28) behind
 * _C.add_requant15_simd (add_requant15/add_requant15_torch.cpp:8-77, pybind.cpp:377-383). */
int iw_add_requant15(const int8_t *x, const int8_t *addend, const uint16_t *multiplier,
                     const int8_t *shift, int16_t *out, int64_t batch, int64_t positions,
                     int64_t channels, int64_t multiplier_count, int64_t shift_count,
                     iw_stream_t stream);

/* int8 Conv1d (dilation 1, groups 1) + bias + per-tensor requant, [B,Cin,Tin] -> [B,Cout,Tout].
 * weight is [Cout, Cin*kernel_size] with the kernel index fastest.
 * Replaces iwhisper::conv1d_simd (conv1d/conv1d.h:71-85) behind _C.conv1d_simd
 * (conv1d/conv1d_torch.cpp:243-340, pybind.cpp:357-366). */
int iw_conv1d(const int8_t *x, const int8_t *weight, const int32_t *bias, uint32_t multiplier,
              int8_t shift, int8_t *out, int64_t batch, int64_t in_channels,
              int64_t input_length, int64_t out_channels, int64_t kernel_size, int64_t stride,
              int64_t padding, bool has_bias, iw_stream_t stream);

/* Logits before dequant: out = clamp(Rshift(mulh(x.E, m), max(s,0)), +-127) int8.
 * Replaces iwhisper::classifier_simd (classifier/classifier.h:52-60) behind
 * _C.classifier_simd (classifier/classifier_torch.cpp:145-212, pybind.cpp:407-414). */
int iw_classifier(const int8_t *x, const int8_t *weight, uint32_t multiplier, int8_t shift,
                  int8_t *out, int64_t M, int64_t K, int64_t N, iw_stream_t stream);

/* q [B,H,Tq,D], k [B,H,Tk,D] int8; mask [Tq,Tk] or NULL -> qk [B,H,Tq,Tk] int16,
 * row_max_plus1 [B,H,Tq] int16. Replaces iwhisper::qk_requant_rowmax_simd
 * (attention/attention.h:33-46) behind _C.qk_requant_rowmax_simd
 * (attention/attention_torch.cpp:117-229, pybind.cpp:261-269). */
int iw_qk_requant_rowmax(const int8_t *q, const int8_t *k, const bool *mask, int16_t *qk,
                         int16_t *row_max_plus1, int64_t batch, int64_t heads, int64_t q_length,
                         int64_t k_length, int64_t head_dim, uint8_t multiplier, int32_t shift,
                         bool has_mask, iw_stream_t stream);

/* qk [B,H,Tq,Tk] int16 -> p uint8 (same shape), row_sum [B,H,Tq] int32.
 * frac_bits must be in [1, 13]. Replaces iwhisper::shift_exp_simd
 * (attention/attention.h:71-82) behind _C.shift_exp_simd
 * (attention/attention_torch.cpp:266-369, pybind.cpp:280-287). */
int iw_shift_exp(const int16_t *qk, const int16_t *row_max_plus1, const bool *mask, uint8_t *p,
                 int32_t *row_sum, int64_t batch, int64_t heads, int64_t q_length,
                 int64_t k_length, int32_t frac_bits, bool has_mask, iw_stream_t stream);

/* p [B,H,Tq,Tk] uint8, v [B,H,D,Tk] int8, row_sum [B,H,Tq] int32 (must be >= 0;
 * the caller validates it, as the reference kernel throws) -> out [B,Tq,H*D] int8.
 * rsqrt_offset must be in [0, 29]. Replaces iwhisper::pv_norm_requant_simd
 * (attention/attention.h:151-164) behind _C.pv_norm_requant_simd
 * (attention/attention_torch.cpp:523-669, pybind.cpp:314-322). */
int iw_pv_norm_requant(const uint8_t *p, const int8_t *v, const int32_t *row_sum,
                       uint8_t av_multiplier, int8_t av_shift, uint32_t rsqrt_offset,
                       int8_t *out, int64_t batch, int64_t heads, int64_t q_length,
                       int64_t k_length, int64_t head_dim, iw_stream_t stream);

/* ---------------------------------------------------------------------------
 * Fused entry points used by the MI355X layer API. Each is bit-identical to
 * the chain of reference ops named in its comment; none has a single
 * counterpart in the reference.
 * ------------------------------------------------------------------------- */

/* Linear8 followed by GELU_int on its int8 output (model_int.py:1103-1107,
 * the MLP's first two modules). GeLU parameter counts are 1 or N. */
int iw_linear8_gelu(const int8_t *x, const int8_t *weight, const int32_t *bias,
                    const int8_t *weight_zero, const uint32_t *multiplier, const int8_t *shift,
                    const uint8_t *lut, const uint8_t *luti_multiplier, const int8_t *luti_shift,
                    const uint8_t *luto_multiplier, const int8_t *luto_shift, int64_t luti_count,
                    int64_t luto_count, int8_t *out, int64_t M, int64_t K, int64_t N,
                    bool has_bias, bool asymmetric, iw_stream_t stream);

/* Linear32 followed by residual15 with the block input (model_int.py:1126-1169):
 * out = residual15(linear32(x), residual, residual_multiplier), [M,N] int16.
 * out may alias residual (each element is read before it is written). */
int iw_linear32_residual15(const int8_t *x, const int8_t *weight, const int32_t *bias,
                           const int8_t *weight_zero, const uint32_t *multiplier,
                           const int8_t *shift, const int16_t *residual,
                           uint16_t residual_multiplier, int16_t *out, int64_t M, int64_t K,
                           int64_t N, bool has_bias, bool asymmetric, iw_stream_t stream);

/* Encoder input quantisation round(mel*alpha) clamped to +-127 (model_int.py:1265-1267,
 * round half to even), mel [B,n_mels,T] float32 -> out [B,T,n_mels] int8 (channels-last). */
int iw_quantize_mel(const float *mel, float alpha, int8_t *out, int64_t batch, int64_t n_mels,
                    int64_t frames, iw_stream_t stream);

/* Channels-last Conv1d_int then GELU_int, optionally then the encoder's
 * positional add_requant15 (model_int.py:1269-1296):
 *   x [B,Tin,Cin] int8 (Cin % 16 == 0), weight_kc [Cout, kernel_size*Cin] (the
 *   reference weight reordered to kernel-index-major), out [B,Tout,Cout].
 * With pe == NULL the output is int8 (conv1 + gelu1); otherwise int16 =
 * add_requant15(gelu(conv(x)), pe [Tout,Cout], pe_multiplier, pe_shift). */
int iw_conv1d_cl(const int8_t *x, const int8_t *weight_kc, const int32_t *bias,
                 uint32_t multiplier, int8_t shift, const uint8_t *lut,
                 const uint8_t *luti_multiplier, const int8_t *luti_shift,
                 const uint8_t *luto_multiplier, const int8_t *luto_shift, int64_t luti_count,
                 int64_t luto_count, const int8_t *pe, const uint16_t *pe_multiplier,
                 const int8_t *pe_shift, int64_t pe_multiplier_count, int64_t pe_shift_count,
                 void *out, int64_t batch, int64_t in_channels, int64_t input_length,
                 int64_t out_channels, int64_t kernel_size, int64_t stride, int64_t padding,
                 bool has_bias, iw_stream_t stream);

/* Decoder input: token-embedding gather then add_requant15 with the positional
 * rows [offset, offset+T) (model_int.py:1411-1439). tokens [B,T] int64,
 * table [vocab,C], pe [n_ctx,C], multiplier/shift scalars -> out [B,T,C] int16. */
int iw_embed_add_requant15(const int64_t *tokens, const int8_t *table, const int8_t *pe,
                           int64_t offset, const uint16_t *multiplier, const int8_t *shift,
                           int16_t *out, int64_t batch, int64_t positions, int64_t channels,
                           iw_stream_t stream);

/* Fills the IW_SHIFT_EXP_TABLE_BYTES-entry table used by the fused attention:
 * table[i] = shift_exp(x_sub = -i) for frac_bits in [1, 13]
 * (attention/attention_scalar.cpp:449-554). */
int iw_shift_exp_table(uint8_t *table, int32_t frac_bits, iw_stream_t stream);

/* Fused MultiHeadAttention_int.qkv_attention (model_int.py:774-1040), i.e.
 * qk_requant_rowmax -> shift_exp -> pv_norm_requant, without materialising the
 * int16 scores or uint8 probabilities. q/k: element (b,t,h,d) at
 * base + b*sb + t*st + h*head_dim + d; v is transposed per head:
 * vt + b*v_sb + h*v_sh + d*v_sd + t (v_sd % 16 == 0 and at least round_up(k_length, 16)
 * columns readable). out element (b,t,h,d) at out + b*o_sb + t*o_st + h*head_dim + d.
 * head_dim % 16 == 0, head_dim <= 128. mask [Tq,Tk] bool or NULL.
 * The prefill form uses int8 MFMA and needs the table from iw_shift_exp_table;
 * the decode form (q_length <= 8, k_length <= 4096) takes table == NULL and also
 * needs k_sh (per-head stride of k). */
int iw_attention(const int8_t *q, int64_t q_sb, int64_t q_st, const int8_t *k, int64_t k_sb,
                 int64_t k_sh, int64_t k_st, const int8_t *vt, int64_t v_sb, int64_t v_sh,
                 int64_t v_sd, int8_t *out, int64_t o_sb, int64_t o_st, const bool *mask,
                 int64_t batch, int64_t heads, int64_t q_length, int64_t k_length,
                 int64_t head_dim, uint8_t qk_multiplier, int8_t qk_shift, int32_t frac_bits,
                 uint8_t av_multiplier, int8_t av_shift, uint32_t rsqrt_offset,
                 const uint8_t *table, bool decode, iw_stream_t stream);

/* Layout helpers for the KV caches (the reference's view/permute/.contiguous()
 * copies and hook-side torch.cat, model_int.py:842-949 and 1604-1610):
 * transpose_heads writes, with p = t_offset + t,
 * dst[b*dst_sb + h*dst_sh + d*dst_sd + (p/4)*dst_sq + p%4] = src[b*src_sb + t*src_st + h*D + d]
 * (dst_sq = 4: V^T per head, dst[b][h][d][p]; dst_sd = 4, dst_sq >= 4*head_dim:
 * V in key quads, see the decode step below); copy_rows writes
 * dst[b*dst_sb + (t_offset+t)*dst_st + c] = src[b*src_sb + t*src_st + c] for c < channels. */
int iw_transpose_heads(const int8_t *src, int64_t src_sb, int64_t src_st, int8_t *dst,
                       int64_t dst_sb, int64_t dst_sh, int64_t dst_sd, int64_t dst_sq,
                       int64_t t_offset, int64_t batch, int64_t positions, int64_t heads,
                       int64_t head_dim, iw_stream_t stream);
int iw_copy_rows(const int8_t *src, int64_t src_sb, int64_t src_st, int8_t *dst, int64_t dst_sb,
                 int64_t dst_st, int64_t t_offset, int64_t batch, int64_t positions,
                 int64_t channels, iw_stream_t stream);

/* First index of the maximum of each row of int8 logits (greedy decoding,
 * decoding.py:280-296 on the int8 logits, which dequantisation by a positive
 * scale does not reorder). x [rows, ld], out [rows] int64. */
int iw_argmax_rows(const int8_t *x, int64_t rows, int64_t cols, int64_t ld, int64_t *out,
                   iw_stream_t stream);

/* ---------------------------------------------------------------------------
 * Decode step over preallocated KV caches with the cache position on the
 * device (*pos), so that one captured step replays for every token.
 * Replaces the reference's per-step chain: TextDecoder_int.forward with
 * offset = cached length (model_int.py:1398-1442), the hook-side torch.cat
 * of the self-attention K/V (model_int.py:1587-1618), the cross-attention
 * K/V reuse (model_int.py:722-730) and GreedyDecoder.update
 * (decoding.py:280-296). Cache layouts: K [b][h][t][d] at
 * k + b*k_sb + h*k_sh + t*k_st + d; V at v + b*v_sb + h*v_sh + d*v_sd + (t/4)*v_sq + t%4,
 * in one of two forms:
 *   transposed per head [b][h][d][t]: v_sq = 4, row d of a head at d*v_sd;
 *   key quads [b][h][t/4][d][t%4]: v_sd = 4, v_sq >= 4*head_dim (v_sq = 4*head_dim
 *   packs them): one token's V of a head is 4*head_dim bytes of one quad, so
 *   the per-step append touches 4 cache lines per head instead of head_dim.
 * The decode attention reads key quads for head_dim 64 (v_sq % 16 == 0).
 * ------------------------------------------------------------------------- */

/* Self-attention Q/K/V projection (MultiHeadAttention_int.forward,
 * model_int.py:720-726) as one Linear8 over the concatenated [3C, K] weight:
 * columns [0, C) go to q_out[m*q_ld + c]; columns [C, 2C) (K) and [2C, 3C)
 * (V) of row m = b*T + i are appended at cache position t = *pos + i
 * (T = tokens_per_row_group), dropped when t >= cache_positions. */
int iw_linear8_qkv_cache(const int8_t *x, const int8_t *weight, const int32_t *bias,
                         const int8_t *weight_zero, const uint32_t *multiplier, const int8_t *shift,
                         int64_t M, int64_t K, bool has_bias, bool asymmetric, int8_t *q_out,
                         int64_t q_ld, int8_t *k_cache, int64_t k_sb, int64_t k_sh, int64_t k_st,
                         int8_t *v_cache, int64_t v_sb, int64_t v_sh, int64_t v_sd, int64_t v_sq,
                         int64_t channels, int64_t head_dim, int64_t tokens_per_row_group,
                         int64_t cache_positions, const int32_t *pos, iw_stream_t stream);

/* One-query attention over the caches (qkv_attention for q_length 1,
 * model_int.py:774-1040): q [b][h*D] at q + b*q_sb, out at out + b*o_sb.
 * The key count is min(k_length + *pos, max_keys) (pos may be NULL when
 * max_keys == k_length); max_keys <= 4096; transposed V rows (v_sq = 4) hold
 * round_up(max_keys, 16) bytes, key quads cover round_up(max_keys, 4) keys. */
int iw_attention_decode_cache(const int8_t *q, int64_t q_sb, const int8_t *k, int64_t k_sb,
                              int64_t k_sh, int64_t k_st, const int8_t *vt, int64_t v_sb,
                              int64_t v_sh, int64_t v_sd, int64_t v_sq, int8_t *out, int64_t o_sb,
                              int64_t batch, int64_t heads, int64_t head_dim, int64_t k_length,
                              const int32_t *pos, int64_t max_keys, uint8_t qk_multiplier,
                              int8_t qk_shift, int32_t frac_bits, uint8_t av_multiplier,
                              int8_t av_shift, uint32_t rsqrt_offset, iw_stream_t stream);

/* Decoder input of one token per row at position *pos (model_int.py:1408-1425):
 * out[b, c] = add_requant15(table[tokens[b], c], pe[min(*pos, pe_rows - 1), c]). */
int iw_embed_tokens(const int64_t *tokens, const int8_t *table, const int8_t *pe,
                    int64_t pe_rows, const int32_t *pos, const uint16_t *multiplier,
                    const int8_t *shift, int16_t *out, int64_t batch, int64_t channels,
                    iw_stream_t stream);

/* Greedy step bookkeeping (GreedyDecoder.update, decoding.py:280-296, on the
 * int8 logits): next_tokens[r] = first argmax of row r; when *step <
 * history_cols, history[r*history_ld + *step] = next_tokens[r]; then
 * *step += 1 and *pos += pos_increment. */
int iw_greedy_advance(const int8_t *logits, int64_t rows, int64_t cols, int64_t ld,
                      int64_t *next_tokens, int64_t *history, int64_t history_ld,
                      int64_t history_cols, int32_t *step, int32_t *pos, int32_t pos_increment,
                      iw_stream_t stream);

/* The greedy step with the decoding task's logit filters applied on the
 * device (decoding.py:410-509: SuppressBlank, SuppressTokens,
 * ApplyTimestampRules; GreedyDecoder.update :275-296 for the EOT freeze),
 * replacing the host-side filter loop of decoding.py:698-701. history[r][0 ..
 * *step) holds the tokens sampled so far (column 0 is the first token after
 * the prompt, i.e. sample_begin). Arguments after pos_increment:
 *   suppress        bitmask, bit i of word i/32 set = token i suppressed at
 *                   every step (SuppressTokens ids, and <|notimestamps|> when
 *                   the timestamp rules are on); (cols + 31)/32 words; or NULL
 *   suppress_first  the same for the first sampled step (adds SuppressBlank's
 *                   " " and EOT); NULL = suppress
 *   prev0           [rows] the token before the first sampled one (the
 *                   prompt's last); NULL = none
 *   eot             EOT id: rows whose previous token is EOT emit EOT; < 0
 *                   disables this and the timestamp rules
 *   timestamp_begin first timestamp id; < 0 disables the timestamp rules
 *   max_initial_timestamp  max_initial_timestamp_index, < 0 = none
 *   logit_scale     the logits' dequantisation scale (> 0), for the rule that
 *                   compares logsumexp over timestamps with the best text
 *                   logit in fp32
 *   sum_logprobs    [rows] float32 or NULL: += log_softmax of the filtered,
 *                   dequantised logits (x * logit_scale, suppressed = -inf)
 *                   at the chosen token, unless the previous token is EOT
 *                   (GreedyDecoder.update, decoding.py:287-289); NaN for an
 *                   all-suppressed row
 *   eot_count       [history_cols] int32 or NULL: eot_count[*step] += the
 *                   number of rows whose new token is EOT
 * All-suppressed rows give token 0 (torch.argmax over -inf). Then as
 * iw_greedy_advance: history[r][*step] = next, *step += 1, *pos += pos_increment. */
int iw_greedy_advance_filtered(const int8_t *logits, int64_t rows, int64_t cols, int64_t ld,
                               int64_t *next_tokens, int64_t *history, int64_t history_ld,
                               int64_t history_cols, int32_t *step, int32_t *pos,
                               int32_t pos_increment, const uint32_t *suppress,
                               const uint32_t *suppress_first, const int64_t *prev0, int32_t eot,
                               int32_t timestamp_begin, int32_t max_initial_timestamp,
                               float logit_scale, float *sum_logprobs, int32_t *eot_count,
                               iw_stream_t stream);

/* -------------------------------------------------------------------------
 * Fragment-major operands of the one-token decode step. No counterpart in
 * the reference: an operand layout for the batched greedy step above, in
 * which each int8 MFMA operand is one contiguous 1 KB piece so that a decode
 * GEMM issues all of its loads at once. An int8 matrix X[R][K] is stored as
 * [Rp/32][Kp/32][64][16] with Rp = R rounded up to 32 and Kp = K rounded up
 * to a multiple of 320, K <= 5120: byte k of row r sits at
 *   (r/32)*32*Kp + (k/32)*1024 + (r%32 + 32*((k/16)%2))*16 + k%16,
 * and the padding holds zeros. Results equal the row-major entry points'.
 * ------------------------------------------------------------------------- */

/* Bytes of the fragment-major image of an int8 [rows][cols] matrix
 * (0 for cols > 5120 or a negative size). */
int64_t iw_frag_bytes(int64_t rows, int64_t cols);

/* The decode step's cross-attention with the LayerNorm and query projection
 * before it fused in (model_int.py:1139-1145, cross_attn_ln then cross_attn,
 * whose forward, :713-735, projects the query and attends over the cached
 * K/V): each
 * (batch b, head h) block normalises residual row b (x + b * x_ld, C =
 * heads * 64 int16, LayerNorm32 with iw_layernorm32's parameters), projects
 * it onto the head's 64 query channels (q_weight fragment-major [C][Kp],
 * Linear8 parameters as iw_linear8) and attends as
 * iw_attention_decode_cache_frag over k_length cached keys (V transposed:
 * v_sq == 4). out is the fragment-major image of [batch][C], as
 * iw_attention_decode_cache_frag writes it. Results equal iw_layernorm32 ->
 * iw_linear8 -> iw_attention_decode_cache_frag; batch <= 128, head_dim 64,
 * C in {384, 512, 768, 1024, 1280}, k_length <= 2048. No single counterpart
 * in the reference, which runs the three calls. */
int iw_attention_decode_cross_lnq(const int16_t *x, int64_t x_ld, const int8_t *ln_weight, const int32_t *ln_bias,
                                  uint8_t ln_multiplier, int8_t ln_shift, uint32_t ln_out_multiplier,
                                  int8_t ln_out_shift, uint32_t ln_rsqrt_offset, bool ln_has_bias,
                                  const int8_t *q_weight, const int32_t *q_bias, const int8_t *q_weight_zero,
                                  const uint32_t *q_multiplier, const int8_t *q_shift, bool q_has_bias,
                                  bool q_asymmetric, const int8_t *k, int64_t k_sb, int64_t k_sh, int64_t k_st,
                                  const int8_t *vt, int64_t v_sb, int64_t v_sh, int64_t v_sd, int8_t *out,
                                  int64_t batch, int64_t heads, int64_t head_dim, int64_t k_length,
                                  uint8_t qk_multiplier, int8_t qk_shift, int32_t frac_bits,
                                  uint8_t av_multiplier, int8_t av_shift, uint32_t rsqrt_offset,
                                  iw_stream_t stream);

/* Row-major src [rows][cols] (row stride ld) to its fragment-major image,
 * padding included (dst holds iw_frag_bytes(rows, cols) bytes). */
int iw_frag_pack(const int8_t *src, int64_t rows, int64_t cols, int64_t ld, int8_t *dst,
                 iw_stream_t stream);

/* iw_linear8 / iw_linear8_gelu with x and weight fragment-major (M <= 128);
 * out is row-major [M][N] or, when out_frag, the fragment-major image of
 * [M][N]. iw_linear8_gelu_frag's next_weight (optional, NULL for none): the
 * fragment-major weight [next_n][next_k] of the decode GEMM that runs next;
 * the launch also reads its column tiles into the L2 of the XCD that GEMM
 * reads each tile on. A prefetch hint: the results do not depend on it. */
int iw_linear8_frag(const int8_t *x, const int8_t *weight, const int32_t *bias,
                    const int8_t *weight_zero, const uint32_t *multiplier, const int8_t *shift,
                    int8_t *out, int64_t M, int64_t K, int64_t N, bool has_bias, bool asymmetric,
                    bool out_frag, iw_stream_t stream);
int iw_linear8_gelu_frag(const int8_t *x, const int8_t *weight, const int32_t *bias,
                         const int8_t *weight_zero, const uint32_t *multiplier, const int8_t *shift,
                         const uint8_t *lut, const uint8_t *luti_multiplier, const int8_t *luti_shift,
                         const uint8_t *luto_multiplier, const int8_t *luto_shift, int64_t luti_count,
                         int64_t luto_count, int8_t *out, int64_t M, int64_t K, int64_t N,
                         bool has_bias, bool asymmetric, bool out_frag, const int8_t *next_weight,
                         int64_t next_n, int64_t next_k, iw_stream_t stream);

/* iw_linear32_residual15 with x and weight fragment-major (M <= 128). */
int iw_linear32_residual15_frag(const int8_t *x, const int8_t *weight, const int32_t *bias,
                                const int8_t *weight_zero, const uint32_t *multiplier,
                                const int8_t *shift, const int16_t *residual,
                                uint16_t residual_multiplier, int16_t *out, int64_t M, int64_t K,
                                int64_t N, bool has_bias, bool asymmetric, iw_stream_t stream);

/* iw_linear8_qkv_cache with x and weight fragment-major. */
int iw_linear8_qkv_cache_frag(const int8_t *x, const int8_t *weight, const int32_t *bias,
                              const int8_t *weight_zero, const uint32_t *multiplier,
                              const int8_t *shift, int64_t M, int64_t K, bool has_bias,
                              bool asymmetric, int8_t *q_out, int64_t q_ld, int8_t *k_cache,
                              int64_t k_sb, int64_t k_sh, int64_t k_st, int8_t *v_cache,
                              int64_t v_sb, int64_t v_sh, int64_t v_sd, int64_t v_sq,
                              int64_t channels, int64_t head_dim, int64_t tokens_per_row_group,
                              int64_t cache_positions, const int32_t *pos, iw_stream_t stream);

/* iw_layernorm32 writing the fragment-major image of out [rows][hidden]
 * (rows <= 128); next_weight / next_n / next_k: the prefetch hint of
 * iw_linear8_gelu_frag (the GEMM that reads out). */
int iw_layernorm32_frag(const int16_t *x, const int8_t *weight, const int32_t *bias,
                        uint8_t ln_multiplier, int8_t ln_shift, uint32_t out_multiplier,
                        int8_t out_shift, uint32_t rsqrt_offset, int8_t *out, int64_t rows,
                        int64_t hidden, bool has_bias, const int8_t *next_weight, int64_t next_n,
                        int64_t next_k, iw_stream_t stream);

/* iw_attention_decode_cache writing the fragment-major image of out
 * [batch][heads*head_dim] (batch <= 128, heads*head_dim <= 5120).
 * next_weight / next_n / next_k (NULL, 0, 0 for none): the fragment-major
 * weight of the GEMM that runs next, which the launch's last blocks read
 * into the L2 of the XCD that reads each of its 32-column tiles (a hint, as
 * for iw_layernorm32_frag; taken by the self-attention kernel: V in key
 * quads, at most 512 keys). */
int iw_attention_decode_cache_frag(const int8_t *q, int64_t q_sb, const int8_t *k, int64_t k_sb,
                                   int64_t k_sh, int64_t k_st, const int8_t *vt, int64_t v_sb,
                                   int64_t v_sh, int64_t v_sd, int64_t v_sq, int8_t *out,
                                   int64_t batch, int64_t heads, int64_t head_dim, int64_t k_length,
                                   const int32_t *pos, int64_t max_keys, uint8_t qk_multiplier,
                                   int8_t qk_shift, int32_t frac_bits, uint8_t av_multiplier,
                                   int8_t av_shift, uint32_t rsqrt_offset, const int8_t *next_weight,
                                   int64_t next_n, int64_t next_k, iw_stream_t stream);

/* iw_classifier with x and weight fragment-major (M <= 128, K <= 5120); out
 * row-major [M][N]. */
int iw_classifier_frag(const int8_t *x, const int8_t *weight, uint32_t multiplier, int8_t shift,
                       int8_t *out, int64_t M, int64_t K, int64_t N, iw_stream_t stream);

/* iw_classifier_frag with the greedy argmax fused into its epilogue (the
 * classifier of model_int.py:1446-1484 followed by the argmax of
 * GreedyDecoder.update, decoding.py:280-296): also writes, for each row m and
 * each 32-column tile t, the first maximum of the int8 logits in the tile,
 * row_max[m * ceil(N / 32) + t] = (y + 128) << 5 | (31 - column in tile).
 * out may be NULL (no logits written). N < 2^23. */
int iw_classifier_argmax_frag(const int8_t *x, const int8_t *weight, uint32_t multiplier,
                              int8_t shift, int8_t *out, uint16_t *row_max, int64_t M, int64_t K,
                              int64_t N, iw_stream_t stream);

/* One step of GreedyDecoder.update (decoding.py:280-296) at temperature 0
 * for rows of int8 logits (dequantised by logit_scale > 0):
 *   next token   the first index of the row maximum, from row_max (the
 *                tile maxima of iw_classifier_argmax_frag, tiles = ceil(cols /
 *                32)) or, when row_max is NULL, from logits [rows][ld];
 *   EOT freeze   with eot >= 0, a row whose previous token (history[r][*step -
 *                1], or prev0[r] at *step 0) is EOT emits EOT;
 *   sum_logprobs [rows] or NULL: += log_softmax(logits * logit_scale) at the
 *                token, unless the previous token is EOT (needs logits);
 *   eot_count    [history_cols] or NULL: eot_count[*step] += rows whose new
 *                token is EOT (all rows finished = the count equals rows);
 * then history[r][*step] = next_tokens[r] = token, *step += 1, *pos +=
 * pos_increment. arrive: one uint32 that is 0 between calls (the kernel's
 * blocks count their arrival there; the last one resets it). */
int iw_greedy_update(const uint16_t *row_max, int64_t tiles, const int8_t *logits, int64_t ld,
                     int64_t rows, int64_t cols, int64_t *next_tokens, int64_t *history,
                     int64_t history_ld, int64_t history_cols, int32_t *step, int32_t *pos,
                     int32_t pos_increment, int32_t eot, const int64_t *prev0, float *sum_logprobs,
                     float logit_scale, int32_t *eot_count, uint32_t *arrive, iw_stream_t stream);

/* out[r] = softmax(logits[r] * logit_scale)[token] in float32: the no-speech
 * probability at the start-of-transcript position (DecodingTask._main_loop,
 * decoding.py:690-695). */
int iw_token_prob(const int8_t *logits, int64_t rows, int64_t cols, int64_t ld, int64_t token,
                  float logit_scale, float *out, iw_stream_t stream);

/* Log-mel spectrogram (log_mel_spectrogram, audio.py:216-267, with N_FFT =
 * 512, HOP_LENGTH = 160): for each of `batch` rows of float32 audio
 * (n_samples > 256, row stride audio_ld) and frame t < n_samples / 160, the
 * 512-point FFT of the window-weighted frame centred at 160 t (reflect padding
 * by 256), |X[k]|^2 for k = 0 .. 256, the mel projection
 * mel[m] = sum_e w[off[m] + e] * |X[start[m] + e]|^2 (e < len[m]; the nonzero
 * taps of the filterbank row m), then log10(max(mel, 1e-10)); finally per
 * row y = max(y, max(row) - 8) / 4 + 1. out[b][m][t] (batch stride
 * out_batch_stride >= n_mels * (n_samples / 160)). twiddle: 256 complex
 * exp(-2 pi i j / 512) as (re, im) pairs; window: 512 Hann weights;
 * n_mels <= 128, n_taps <= 2048; workspace: batch * ceil(frames / 64) floats. */
int iw_log_mel(const float *audio, int64_t batch, int64_t n_samples, int64_t audio_ld, const float *twiddle,
               const float *window, const int32_t *filter_start, const int32_t *filter_len,
               const int32_t *filter_offset, const float *filter_weights, int32_t n_taps, int32_t n_mels,
               float *out, int64_t out_batch_stride, float *workspace, iw_stream_t stream);

/* Block-maximum entries of iw_log_mel's workspace for batch rows of n_samples
 * samples: batch * ceil((n_samples / 160) / 64) (-1 for negative sizes). */
int64_t iw_log_mel_scratch_floats(int64_t batch, int64_t n_samples);

/* Maximum iw_log_mel_scratch_floats() that iw_log_mel_noalloc takes (256 KB of
 * float block maxima per GPU: 1394 rows of 30 s audio). */
#define IW_LOG_MEL_SCRATCH_FLOATS 65536

/* iw_log_mel without the workspace argument, allocating nothing: no
 * counterpart in the reference. For callers that cannot allocate device memory
 * (code under HIP graph capture, serving loops, harnesses that forbid
 * hipMalloc). The block maxima live in a fixed device array of
 * IW_LOG_MEL_SCRATCH_FLOATS floats that each GPU holds from its first call until
 * the process ends; larger inputs are rejected (IW_EINVAL). Every call on one
 * GPU shares that array, so calls that overlap on one GPU (several streams or
 * threads) race; calls in order on one stream do not. The stream must belong to
 * the current device. Results equal iw_log_mel's. */
int iw_log_mel_noalloc(const float *audio, int64_t batch, int64_t n_samples, int64_t audio_ld,
                       const float *twiddle, const float *window, const int32_t *filter_start,
                       const int32_t *filter_len, const int32_t *filter_offset,
                       const float *filter_weights, int32_t n_taps, int32_t n_mels, float *out,
                       int64_t out_batch_stride, iw_stream_t stream);

/* Dynamic time warping for word timestamps (triton_ops.py:13-40, dtw_cuda
 * timing.py:108-141; it replaces the Triton kernel launch): over float32 costs
 * x [rows][cols] (row stride ld; rows < 1024, the reference's M < BLOCK_SIZE),
 * cost[i][j] = x[i-1][j-1] + min(cost[i-1][j-1], cost[i-1][j], cost[i][j-1])
 * with cost[0][0] = 0 and +inf borders; writes trace [rows+1][cols+1] (row
 * stride trace_ld >= cols + 1): trace[i][j] = 0, 1 or 2 for the first of the
 * three predecessors holding the minimum (the reference kernel's store order),
 * trace[0][*] = 2, trace[*][0] = 1, as timing.py's backtrace expects. */
int iw_dtw(const float *x, int64_t rows, int64_t cols, int64_t ld, int8_t *trace, int64_t trace_ld,
           iw_stream_t stream);

/* Sliding median along the last dimension (median_filter, timing.py:19-55,
 * replacing median_filter_cuda, triton_ops.py:43-109): y[r][t] = median of
 * x[r][reflect(t - width/2 .. t + width/2)] (reflect padding without repeating
 * the edge, F.pad(mode="reflect")). width odd, at most 31; cols > width / 2
 * (the reference returns x unchanged otherwise). */
int iw_median_filter(const float *x, int64_t rows, int64_t cols, int64_t ld, int32_t width, float *y,
                     int64_t y_ld, iw_stream_t stream);

/* Per-head gather into a [b][h][t][d] cache (the cross-attention K of
 * model_int.py:722-730, computed once per utterance):
 * dst[b*dst_sb + h*dst_sh + (t_offset+t)*dst_st + d] = src[b*src_sb + t*src_st + h*D + d]. */
int iw_gather_heads(const int8_t *src, int64_t src_sb, int64_t src_st, int8_t *dst, int64_t dst_sb,
                    int64_t dst_sh, int64_t dst_st, int64_t t_offset, int64_t batch,
                    int64_t positions, int64_t heads, int64_t head_dim, iw_stream_t stream);

#ifdef __cplusplus
}
#endif
#endif /* IWHISPER_AMD_H */
