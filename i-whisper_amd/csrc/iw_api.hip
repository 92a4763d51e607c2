// C ABI entry points (include/iwhisper_amd.h): argument checks, then launch.
#include "../../include/iwhisper_amd.h"
#include "iw_common.hpp"
#include "iw_gemm.hpp"
#include "iw_kernels.hpp"

#include <string>

namespace iw {

namespace {
thread_local std::string g_last_error;
}

void set_error(const std::string &msg) { g_last_error = msg; }

int fail(const std::string &msg) {
  g_last_error = msg;
  return IW_EINVAL;
}

int check_launch(const char *what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    g_last_error = std::string(what) + ": " + hipGetErrorString(e);
    return IW_ELAUNCH;
  }
  return IW_OK;
}

namespace {

hipStream_t as_stream(iw_stream_t s) { return reinterpret_cast<hipStream_t>(s); }

GemmArgs linear_args(const int8_t *x, const int8_t *w, const int32_t *bias, const int8_t *wz,
                     const uint32_t *mult, const int8_t *shift, void *out, int64_t M, int64_t K,
                     int64_t N, bool has_bias, bool asym, int epi) {
  GemmArgs g;
  g.a = x;
  g.lda = K;
  g.b = w;
  g.ldb = K;
  g.M = M;
  g.N = N;
  g.K = K;
  g.epi = epi;
  g.bias = has_bias ? bias : nullptr;
  g.wz = asym ? wz : nullptr;
  g.mult = mult;
  g.shift = shift;
  g.mult_pc = 1;
  g.out = out;
  g.ldc = N;
  return g;
}

int check_linear(const void *x, const void *w, const int32_t *bias, const int8_t *wz,
                 const void *mult, const void *shift, const void *out, int64_t M, int64_t K,
                 int64_t N, bool has_bias, bool asym) {
  IW_REQUIRE(M >= 0 && N > 0, "invalid GEMM shape");
  IW_REQUIRE(K > 0, "x.size(-1) must be greater than 0");
  IW_REQUIRE(M == 0 || (x && w && mult && shift && out), "null tensor pointer");
  IW_REQUIRE(!has_bias || bias, "has_bias set but bias is null");
  IW_REQUIRE(!asym || wz, "asymmetric set but weight_zero is null");
  return IW_OK;
}

int check_gelu_counts(int64_t channels, int64_t luti_count, int64_t luto_count) {
  IW_REQUIRE(luti_count == 1 || luti_count == channels,
             "luti parameters must be scalar or match input.size(-1)");
  IW_REQUIRE(luto_count == 1 || luto_count == channels,
             "luto parameters must be scalar or match input.size(-1)");
  return IW_OK;
}

int qkv_cache_args(const int8_t *x, const int8_t *weight, const int32_t *bias, const int8_t *weight_zero,
                   const uint32_t *multiplier, const int8_t *shift, int64_t M, int64_t K, bool has_bias,
                   bool asymmetric, int8_t *q_out, int64_t q_ld, int8_t *k_cache, int64_t k_sb, int64_t k_sh,
                   int64_t k_st, int8_t *v_cache, int64_t v_sb, int64_t v_sh, int64_t v_sd, int64_t v_sq,
                   int64_t channels, int64_t head_dim, int64_t tokens_per_row_group, int64_t cache_positions,
                   const int32_t *pos, GemmArgs *g, SkinnyScatter *sc) {
  const int64_t N = 3 * channels;
  int rc = check_linear(x, weight, bias, weight_zero, multiplier, shift, q_out, M, K, N, has_bias,
                        asymmetric);
  if (rc) return rc;
  if (M == 0) return IW_OK;
  IW_REQUIRE(M <= kSkinnyMaxRows, "the KV-cache QKV projection takes at most 128 rows");
  IW_REQUIRE(channels > 0 && head_dim > 0 && channels % head_dim == 0, "invalid head geometry");
  IW_REQUIRE(channels <= 0x3fffffff && tokens_per_row_group > 0 && M % tokens_per_row_group == 0,
             "rows must be whole groups of tokens_per_row_group");
  IW_REQUIRE(k_cache && v_cache && pos, "null cache pointer");
  IW_REQUIRE(cache_positions > 0 && cache_positions <= 0x7fffffff, "cache_positions must be positive");
  // V transposed per head (the rows hold every position) or in key quads
  // (a quad holds every d of the head)
  IW_REQUIRE((v_sq == 4 && cache_positions <= v_sd) || (v_sd == 4 && v_sq >= 4 * head_dim),
             "V cache: v_sq == 4 with transposed rows of at least cache_positions bytes, "
             "or v_sd == 4 with v_sq >= 4 * head_dim (key quads)");
  *g = linear_args(x, weight, bias, weight_zero, multiplier, shift, q_out, M, K, N, has_bias, asymmetric,
                   EPI_L8);
  sc->q = q_out;
  sc->ldq = q_ld;
  sc->k = k_cache;
  sc->k_sb = k_sb;
  sc->k_sh = k_sh;
  sc->k_st = k_st;
  sc->v = v_cache;
  sc->v_sb = v_sb;
  sc->v_sh = v_sh;
  sc->v_sd = v_sd;
  sc->v_sq = v_sq;
  sc->C = (int)channels;
  sc->D = (int)head_dim;
  sc->T = (int)tokens_per_row_group;
  sc->t_cap = (int)cache_positions;
  sc->pos = pos;
  return IW_OK;
}

int layernorm32_entry(const int16_t *x, const int8_t *weight, const int32_t *bias, uint8_t ln_multiplier,
                      int8_t ln_shift, uint32_t out_multiplier, int8_t out_shift, uint32_t rsqrt_offset,
                      int8_t *out, int64_t rows, int64_t hidden, bool has_bias, bool out_frag,
                      iw_stream_t stream, const FragPrefetch *pf = nullptr) {
  IW_REQUIRE(layernorm_width_code(hidden) >= 0,
             "unsupported LayerNorm hidden size: " + std::to_string(hidden));
  IW_REQUIRE(rows >= 0, "invalid row count");
  if (rows == 0) return IW_OK;
  IW_REQUIRE(x && weight && out, "null tensor pointer");
  IW_REQUIRE(!has_bias || bias, "has_bias set but bias is null");
  IW_REQUIRE((reinterpret_cast<uintptr_t>(x) & 7) == 0 && (reinterpret_cast<uintptr_t>(out) & 3) == 0,
             "LayerNorm input must be 8-byte and output 4-byte aligned");
  return launch_layernorm32(x, weight, has_bias ? bias : nullptr, ln_multiplier, ln_shift,
                            out_multiplier, out_shift, rsqrt_offset, out, rows, hidden,
                            as_stream(stream), out_frag, pf);
}

int attention_decode_cache_entry(const int8_t *q, int64_t q_sb, const int8_t *k, int64_t k_sb, int64_t k_sh,
                                 int64_t k_st, const int8_t *vt, int64_t v_sb, int64_t v_sh, int64_t v_sd,
                                 int64_t v_sq, int8_t *out, int64_t o_sb, int64_t batch, int64_t heads,
                                 int64_t head_dim,
                                 int64_t k_length, const int32_t *pos, int64_t max_keys, uint8_t qk_multiplier,
                                 int8_t qk_shift, int32_t frac_bits, uint8_t av_multiplier, int8_t av_shift,
                                 uint32_t rsqrt_offset, bool out_frag, iw_stream_t stream,
                                 const FragPrefetch *tail = nullptr) {
  IW_REQUIRE(frac_bits > 0 && frac_bits < 14, "frac_bits must be in [1, 14)");
  IW_REQUIRE(rsqrt_offset <= 29, "rsqrt_offset must be in [0,29]");
  IW_REQUIRE(head_dim == 64 || head_dim == 96 || head_dim == 128,
             "decode attention supports head_dim 64, 96 and 128");
  IW_REQUIRE(batch >= 0 && heads > 0 && k_length >= 0 && batch * heads <= 0x7fffffff,
             "invalid attention shape");
  // the key count on the device is k_length + *pos <= max_keys
  IW_REQUIRE(max_keys >= k_length && max_keys <= kDecodeCacheMaxKeys && (pos || max_keys == k_length),
             "at most 4096 keys, and max_keys bounds k_length + *pos");
  const bool quads = v_sq != 4;
  if (quads)
    IW_REQUIRE(v_sd == 4 && v_sq % 16 == 0 && v_sq >= 4 * head_dim && head_dim == 64,
               "V in key quads needs v_sd == 4, v_sq >= 4 * head_dim, v_sq % 16 == 0 and head_dim 64");
  else
    IW_REQUIRE(v_sd % 16 == 0 && v_sd >= ((max_keys + 15) / 16) * 16,
               "transposed V rows must be 16-byte multiples covering max_keys");
  if (batch == 0) return IW_OK;
  IW_REQUIRE(q && k && vt && out, "null tensor pointer");
  const uintptr_t align = reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k) |
                          reinterpret_cast<uintptr_t>(vt) | (uintptr_t)q_sb | (uintptr_t)k_sb |
                          (uintptr_t)k_sh | (uintptr_t)k_st | (uintptr_t)v_sb | (uintptr_t)v_sh |
                          (uintptr_t)(quads ? v_sq : 0);
  IW_REQUIRE((align & 15) == 0, "decode attention operands must be 16-byte aligned");
  AttnArgs a;
  a.q = q;
  a.q_sb = q_sb;
  a.k = k;
  a.k_sb = k_sb;
  a.k_sh = k_sh;
  a.k_st = k_st;
  a.vt = vt;
  a.v_sb = v_sb;
  a.v_sh = v_sh;
  a.v_sd = v_sd;
  a.v_sq = v_sq;
  a.vt_ld = v_sd;
  a.out = out;
  a.o_sb = o_sb;
  a.B = (int32_t)batch;
  a.H = (int32_t)heads;
  a.Tq = 1;
  a.Tk = (int32_t)k_length;
  a.D = (int32_t)head_dim;
  a.qk_m = qk_multiplier;
  a.qk_s = (uint32_t)(qk_shift > 0 ? qk_shift : 0);
  a.frac_bits = frac_bits;
  a.av_m = av_multiplier;
  a.av_s = (uint32_t)(av_shift < 0 ? 0 : (av_shift > 32 ? 32 : av_shift));
  a.rsqrt_off = rsqrt_offset;
  a.max_tk = (int32_t)max_keys;
  if (out_frag) {
    IW_REQUIRE(batch <= kSkinnyMaxRows && heads * head_dim <= kFragMaxK,
               "a fragment-major attention output takes at most 128 rows of 5120 channels");
    a.o_frag_kp = frag_kpad(heads * head_dim);
  }
  return launch_attn_decode_cache(a, pos, as_stream(stream), tail);
}

// Fragment-major operands: sizes the kernels take and 16-byte alignment.
int check_frag(const void *x, const void *w, int64_t M, int64_t K, int64_t N) {
  IW_REQUIRE(M <= kSkinnyMaxRows, "the fragment-major GEMMs take at most 128 rows");
  IW_REQUIRE(K <= kFragMaxK, "the fragment-major GEMMs take K <= 5120");
  IW_REQUIRE(N <= 0x7fffff00LL, "N too large");
  IW_REQUIRE(((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(w)) & 15) == 0,
             "fragment-major operands must be 16-byte aligned");
  return IW_OK;
}

// The fragment-major weight [next_n][next_k] of the decode GEMM that runs
// next, as a prefetch hint; none when next_weight is null.
int frag_prefetch_args(const int8_t *next_weight, int64_t next_n, int64_t next_k, FragPrefetch *pf) {
  *pf = FragPrefetch();
  if (!next_weight) return IW_OK;
  IW_REQUIRE(next_n > 0 && next_k > 0 && next_k <= kFragMaxK && frag_rpad(next_n) * frag_kpad(next_k) < (1LL << 31),
             "invalid prefetch weight shape");
  IW_REQUIRE((reinterpret_cast<uintptr_t>(next_weight) & 15) == 0, "prefetch weight must be 16-byte aligned");
  pf->w = next_weight;
  pf->tile_bytes = 32 * frag_kpad(next_k);
  pf->tiles = (int)((next_n + 31) / 32);
  return IW_OK;
}


// argument checks shared by iw_log_mel and iw_log_mel_noalloc (workspace
// excluded)
int check_log_mel(const float *audio, int64_t batch, int64_t n_samples, int64_t audio_ld,
                  const float *twiddle, const float *window, const int32_t *filter_start,
                  const int32_t *filter_len, const int32_t *filter_offset, const float *filter_weights,
                  int32_t n_taps, int32_t n_mels, const float *out, int64_t out_batch_stride) {
  int max_mels = 0, max_taps = 0;
  log_mel_limits(&max_mels, &max_taps);
  IW_REQUIRE(batch >= 0 && n_samples > 256 && n_samples / 160 < (1 << 30) && audio_ld >= n_samples,
             "invalid audio shape (more than 256 samples per row)");
  IW_REQUIRE(n_mels > 0 && n_mels <= max_mels, "n_mels must be in 1 .. 128");
  IW_REQUIRE(n_taps >= 0 && n_taps <= max_taps, "too many filterbank taps");
  IW_REQUIRE(out_batch_stride >= (int64_t)n_mels * (n_samples / 160), "output batch stride too small");
  if (batch == 0) return IW_OK;
  IW_REQUIRE(audio && twiddle && window && filter_start && filter_len && filter_offset && out &&
                 (n_taps == 0 || filter_weights),
             "null tensor pointer");
  return IW_OK;
}
}  // namespace
}  // namespace iw

using namespace iw;

extern "C" {

int iw_abi_version(void) { return IW_ABI_VERSION; }

const char *iw_last_error(void) { return g_last_error.c_str(); }

int iw_linear8(const int8_t *x, const int8_t *weight, const int32_t *bias,
               const int8_t *weight_zero, const uint32_t *multiplier, const int8_t *shift,
               int8_t *out, int64_t M, int64_t K, int64_t N, bool has_bias, bool asymmetric,
               iw_stream_t stream) {
  int rc = check_linear(x, weight, bias, weight_zero, multiplier, shift, out, M, K, N, has_bias,
                        asymmetric);
  if (rc) return rc;
  GemmArgs g = linear_args(x, weight, bias, weight_zero, multiplier, shift, out, M, K, N,
                           has_bias, asymmetric, EPI_L8);
  return gemm_dense(g, as_stream(stream));
}

int iw_linear8_gelu(const int8_t *x, const int8_t *weight, const int32_t *bias,
                    const int8_t *weight_zero, const uint32_t *multiplier, const int8_t *shift,
                    const uint8_t *lut, const uint8_t *luti_multiplier, const int8_t *luti_shift,
                    const uint8_t *luto_multiplier, const int8_t *luto_shift, int64_t luti_count,
                    int64_t luto_count, int8_t *out, int64_t M, int64_t K, int64_t N,
                    bool has_bias, bool asymmetric, iw_stream_t stream) {
  int rc = check_linear(x, weight, bias, weight_zero, multiplier, shift, out, M, K, N, has_bias,
                        asymmetric);
  if (rc) return rc;
  rc = check_gelu_counts(N, luti_count, luto_count);
  if (rc) return rc;
  IW_REQUIRE(lut && luti_multiplier && luti_shift && luto_multiplier && luto_shift,
             "null GeLU parameter pointer");
  GemmArgs g = linear_args(x, weight, bias, weight_zero, multiplier, shift, out, M, K, N,
                           has_bias, asymmetric, EPI_L8);
  g.lut = lut;
  g.luti_m = luti_multiplier;
  g.luti_s = luti_shift;
  g.luto_m = luto_multiplier;
  g.luto_s = luto_shift;
  g.luti_pc = luti_count != 1;
  g.luto_pc = luto_count != 1;
  return gemm_dense(g, as_stream(stream));
}

int iw_linear32(const int8_t *x, const int8_t *weight, const int32_t *bias,
                const int8_t *weight_zero, const uint32_t *multiplier, const int8_t *shift,
                int32_t *out, int64_t M, int64_t K, int64_t N, bool has_bias, bool asymmetric,
                iw_stream_t stream) {
  int rc = check_linear(x, weight, bias, weight_zero, multiplier, shift, out, M, K, N, has_bias,
                        asymmetric);
  if (rc) return rc;
  GemmArgs g = linear_args(x, weight, bias, weight_zero, multiplier, shift, out, M, K, N,
                           has_bias, asymmetric, EPI_L32);
  return gemm_dense(g, as_stream(stream));
}

int iw_linear32_residual15(const int8_t *x, const int8_t *weight, const int32_t *bias,
                           const int8_t *weight_zero, const uint32_t *multiplier,
                           const int8_t *shift, const int16_t *residual,
                           uint16_t residual_multiplier, int16_t *out, int64_t M, int64_t K,
                           int64_t N, bool has_bias, bool asymmetric, iw_stream_t stream) {
  int rc = check_linear(x, weight, bias, weight_zero, multiplier, shift, out, M, K, N, has_bias,
                        asymmetric);
  if (rc) return rc;
  IW_REQUIRE(M == 0 || residual, "null residual pointer");
  GemmArgs g = linear_args(x, weight, bias, weight_zero, multiplier, shift, out, M, K, N,
                           has_bias, asymmetric, EPI_L32RES);
  g.res = residual;
  g.ldres = N;
  g.res_mult = residual_multiplier;
  return gemm_dense(g, as_stream(stream));
}

int iw_classifier(const int8_t *x, const int8_t *weight, uint32_t multiplier, int8_t shift,
                  int8_t *out, int64_t M, int64_t K, int64_t N, iw_stream_t stream) {
  IW_REQUIRE(K > 0, "hidden size must be positive");
  IW_REQUIRE(N > 0, "vocabulary size must be positive");
  IW_REQUIRE(M >= 0, "invalid row count");
  if (M == 0) return IW_OK;
  IW_REQUIRE(x && weight && out, "null tensor pointer");
  GemmArgs g;
  g.a = x;
  g.lda = K;
  g.b = weight;
  g.ldb = K;
  g.M = M;
  g.N = N;
  g.K = K;
  g.epi = EPI_S8;
  g.mult_pc = 0;
  g.out = out;
  g.ldc = N;
  g.scalar_mult = multiplier;
  g.scalar_shift = shift;
  return gemm_dense(g, as_stream(stream));
}

int iw_layernorm32(const int16_t *x, const int8_t *weight, const int32_t *bias,
                   uint8_t ln_multiplier, int8_t ln_shift, uint32_t out_multiplier,
                   int8_t out_shift, uint32_t rsqrt_offset, int8_t *out, int64_t rows,
                   int64_t hidden, bool has_bias, iw_stream_t stream) {
  return layernorm32_entry(x, weight, bias, ln_multiplier, ln_shift, out_multiplier, out_shift, rsqrt_offset, out,
                           rows, hidden, has_bias, false, stream);
}

int iw_layernorm32_rsqrt(const int32_t *x, int32_t *out, int64_t n, uint32_t offset,
                         iw_stream_t stream) {
  IW_REQUIRE(n >= 0, "invalid element count");
  IW_REQUIRE(n == 0 || (x && out), "null tensor pointer");
  IW_REQUIRE(offset <= 29, "rsqrt_offset must be in [0,29]");
  return launch_rsqrt(x, out, n, offset, as_stream(stream));
}

int iw_gelu(const int8_t *x, const uint8_t *lut, const uint8_t *luti_multiplier,
            const int8_t *luti_shift, const uint8_t *luto_multiplier, const int8_t *luto_shift,
            int8_t *out, int64_t numel, int64_t channels, int64_t luti_count,
            int64_t luto_count, iw_stream_t stream) {
  IW_REQUIRE(numel >= 0 && channels > 0 && numel % channels == 0, "invalid GeLU shape");
  int rc = check_gelu_counts(channels, luti_count, luto_count);
  if (rc) return rc;
  if (numel == 0) return IW_OK;
  IW_REQUIRE(x && lut && luti_multiplier && luti_shift && luto_multiplier && luto_shift && out,
             "null tensor pointer");
  return launch_gelu(x, lut, luti_multiplier, luti_shift, luto_multiplier, luto_shift, out, numel,
                     channels, luti_count != 1, luto_count != 1, as_stream(stream));
}

int iw_residual15(const int32_t *branch, const int16_t *residual, uint16_t multiplier,
                  int16_t *out, int64_t numel, iw_stream_t stream) {
  IW_REQUIRE(numel >= 0, "invalid element count");
  IW_REQUIRE(numel == 0 || (branch && residual && out), "null tensor pointer");
  return launch_residual15(branch, residual, multiplier, out, numel, as_stream(stream));
}

int iw_add_requant15(const int8_t *x, const int8_t *addend, const uint16_t *multiplier,
                     const int8_t *shift, int16_t *out, int64_t batch, int64_t positions,
                     int64_t channels, int64_t multiplier_count, int64_t shift_count,
                     iw_stream_t stream) {
  IW_REQUIRE(batch >= 0 && positions >= 0 && channels > 0, "invalid add_requant15 shape");
  IW_REQUIRE(multiplier_count == 1 || multiplier_count == channels,
             "multiplier must contain 1 or C elements");
  IW_REQUIRE(shift_count == 1 || shift_count == channels, "shift must contain 1 or C elements");
  if (batch * positions == 0) return IW_OK;
  IW_REQUIRE(x && addend && multiplier && shift && out, "null tensor pointer");
  return launch_add_requant15(x, nullptr, addend, multiplier, shift, out, batch, positions,
                              channels, multiplier_count != 1, shift_count != 1,
                              as_stream(stream));
}

int iw_embed_add_requant15(const int64_t *tokens, const int8_t *table, const int8_t *pe,
                           int64_t offset, const uint16_t *multiplier, const int8_t *shift,
                           int16_t *out, int64_t batch, int64_t positions, int64_t channels,
                           iw_stream_t stream) {
  IW_REQUIRE(batch >= 0 && positions >= 0 && channels > 0 && offset >= 0,
             "invalid embedding shape");
  if (batch * positions == 0) return IW_OK;
  IW_REQUIRE(tokens && table && pe && multiplier && shift && out, "null tensor pointer");
  return launch_add_requant15(table, tokens, pe + offset * channels, multiplier, shift, out, batch,
                              positions, channels, 0, 0, as_stream(stream));
}

int iw_conv1d(const int8_t *x, const int8_t *weight, const int32_t *bias, uint32_t multiplier,
              int8_t shift, int8_t *out, int64_t batch, int64_t in_channels,
              int64_t input_length, int64_t out_channels, int64_t kernel_size, int64_t stride,
              int64_t padding, bool has_bias, iw_stream_t stream) {
  IW_REQUIRE(batch >= 0 && in_channels > 0 && out_channels > 0 && kernel_size > 0,
             "invalid conv1d shape");
  IW_REQUIRE(stride > 0, "stride must be positive");
  IW_REQUIRE(padding >= 0, "padding must be non-negative");
  const int64_t tout = (input_length + 2 * padding - kernel_size) / stride + 1;
  IW_REQUIRE(input_length + 2 * padding >= kernel_size, "input too short for the kernel");
  if (batch == 0) return IW_OK;
  IW_REQUIRE(x && weight && out, "null tensor pointer");
  IW_REQUIRE(!has_bias || bias, "has_bias set but bias is null");
  GemmArgs g;
  g.a = x;
  g.conv_tin = input_length;
  g.conv_cin = in_channels;
  g.conv_stride = stride;
  g.conv_pad = padding;
  g.conv_tout = tout;
  g.conv_ksize = kernel_size;
  g.b = weight;
  g.ldb = in_channels * kernel_size;
  g.M = batch * tout;
  g.N = out_channels;
  g.K = in_channels * kernel_size;
  g.epi = EPI_S8;
  g.bias = has_bias ? bias : nullptr;
  g.mult_pc = 0;
  g.scalar_mult = multiplier;
  g.scalar_shift = shift;
  g.out = out;
  g.out_T = tout;
  return gemm_conv(g, false, as_stream(stream));
}

int iw_conv1d_cl(const int8_t *x, const int8_t *weight_kc, const int32_t *bias,
                 uint32_t multiplier, int8_t shift, const uint8_t *lut,
                 const uint8_t *luti_multiplier, const int8_t *luti_shift,
                 const uint8_t *luto_multiplier, const int8_t *luto_shift, int64_t luti_count,
                 int64_t luto_count, const int8_t *pe, const uint16_t *pe_multiplier,
                 const int8_t *pe_shift, int64_t pe_multiplier_count, int64_t pe_shift_count,
                 void *out, int64_t batch, int64_t in_channels, int64_t input_length,
                 int64_t out_channels, int64_t kernel_size, int64_t stride, int64_t padding,
                 bool has_bias, iw_stream_t stream) {
  IW_REQUIRE(batch >= 0 && in_channels > 0 && out_channels > 0 && kernel_size > 0 && stride > 0 &&
                 padding >= 0 && input_length + 2 * padding >= kernel_size,
             "invalid conv1d shape");
  IW_REQUIRE(in_channels % 16 == 0, "channels-last conv needs in_channels % 16 == 0");
  int rc = check_gelu_counts(out_channels, luti_count, luto_count);
  if (rc) return rc;
  const int64_t tout = (input_length + 2 * padding - kernel_size) / stride + 1;
  if (batch == 0) return IW_OK;
  IW_REQUIRE(x && weight_kc && out && lut && luti_multiplier && luti_shift && luto_multiplier &&
                 luto_shift,
             "null tensor pointer");
  IW_REQUIRE(!has_bias || bias, "has_bias set but bias is null");
  GemmArgs g;
  g.a = x;
  g.conv_tin = input_length;
  g.conv_cin = in_channels;
  g.conv_stride = stride;
  g.conv_pad = padding;
  g.conv_tout = tout;
  g.conv_ksize = kernel_size;
  g.b = weight_kc;
  g.ldb = in_channels * kernel_size;
  g.M = batch * tout;
  g.N = out_channels;
  g.K = in_channels * kernel_size;
  g.epi = EPI_S8;
  g.bias = has_bias ? bias : nullptr;
  g.mult_pc = 0;
  g.scalar_mult = multiplier;
  g.scalar_shift = shift;
  g.lut = lut;
  g.luti_m = luti_multiplier;
  g.luti_s = luti_shift;
  g.luto_m = luto_multiplier;
  g.luto_s = luto_shift;
  g.luti_pc = luti_count != 1;
  g.luto_pc = luto_count != 1;
  if (pe) {
    IW_REQUIRE(pe_multiplier && pe_shift, "null positional requant parameters");
    IW_REQUIRE(pe_multiplier_count == 1 || pe_multiplier_count == out_channels,
               "multiplier must contain 1 or C elements");
    IW_REQUIRE(pe_shift_count == 1 || pe_shift_count == out_channels,
               "shift must contain 1 or C elements");
    g.pe = pe;
    g.pe_mult = pe_multiplier;
    g.pe_shift = pe_shift;
    g.pe_mpc = pe_multiplier_count != 1;
    g.pe_spc = pe_shift_count != 1;
    g.pe_T = tout;
  }
  g.out = out;
  g.ldc = out_channels;
  return gemm_conv(g, true, as_stream(stream));
}

int iw_quantize_mel(const float *mel, float alpha, int8_t *out, int64_t batch, int64_t n_mels,
                    int64_t frames, iw_stream_t stream) {
  IW_REQUIRE(batch >= 0 && n_mels > 0 && frames > 0, "invalid mel shape");
  if (batch == 0) return IW_OK;
  IW_REQUIRE(mel && out, "null tensor pointer");
  return launch_quantize_mel(mel, alpha, out, batch, n_mels, frames, as_stream(stream));
}

int iw_qk_requant_rowmax(const int8_t *q, const int8_t *k, const bool *mask, int16_t *qk,
                         int16_t *row_max_plus1, int64_t batch, int64_t heads, int64_t q_length,
                         int64_t k_length, int64_t head_dim, uint8_t multiplier, int32_t shift,
                         bool has_mask, iw_stream_t stream) {
  IW_REQUIRE(batch >= 0 && heads >= 0 && q_length >= 0 && k_length >= 0 && head_dim >= 0,
             "invalid attention shape");
  if (batch * heads * q_length == 0) return IW_OK;
  IW_REQUIRE(q && k && qk && row_max_plus1, "null tensor pointer");
  IW_REQUIRE(!has_mask || mask, "has_mask set but mask is null");
  return launch_qk_requant_rowmax(q, k, has_mask ? reinterpret_cast<const uint8_t *>(mask) : nullptr,
                                  qk, row_max_plus1, batch * heads, q_length, k_length, head_dim,
                                  multiplier, shift, as_stream(stream));
}

int iw_shift_exp(const int16_t *qk, const int16_t *row_max_plus1, const bool *mask, uint8_t *p,
                 int32_t *row_sum, int64_t batch, int64_t heads, int64_t q_length,
                 int64_t k_length, int32_t frac_bits, bool has_mask, iw_stream_t stream) {
  IW_REQUIRE(frac_bits > 0 && frac_bits < 14, "frac_bits must be in [1, 14)");
  IW_REQUIRE(batch >= 0 && heads >= 0 && q_length >= 0 && k_length >= 0,
             "invalid attention shape");
  if (batch * heads * q_length == 0) return IW_OK;
  IW_REQUIRE(qk && row_max_plus1 && p && row_sum, "null tensor pointer");
  IW_REQUIRE(!has_mask || mask, "has_mask set but mask is null");
  return launch_shift_exp(qk, row_max_plus1,
                          has_mask ? reinterpret_cast<const uint8_t *>(mask) : nullptr, p, row_sum,
                          batch * heads, q_length, k_length, frac_bits, as_stream(stream));
}

int iw_pv_norm_requant(const uint8_t *p, const int8_t *v, const int32_t *row_sum,
                       uint8_t av_multiplier, int8_t av_shift, uint32_t rsqrt_offset,
                       int8_t *out, int64_t batch, int64_t heads, int64_t q_length,
                       int64_t k_length, int64_t head_dim, iw_stream_t stream) {
  IW_REQUIRE(rsqrt_offset <= 29, "rsqrt_offset must be in [0,29]");
  IW_REQUIRE(batch >= 0 && heads >= 0 && q_length >= 0 && k_length >= 0 && head_dim >= 0,
             "invalid attention shape");
  if (batch * heads * q_length * head_dim == 0) return IW_OK;
  IW_REQUIRE(p && v && row_sum && out, "null tensor pointer");
  return launch_pv_norm_requant(p, v, row_sum, av_multiplier, av_shift, rsqrt_offset, out, batch,
                                heads, q_length, k_length, head_dim, as_stream(stream));
}

int iw_shift_exp_table(uint8_t *table, int32_t frac_bits, iw_stream_t stream) {
  IW_REQUIRE(frac_bits > 0 && frac_bits < 14, "frac_bits must be in [1, 14)");
  IW_REQUIRE(table, "null table pointer");
  return launch_shift_exp_lut(table, frac_bits, as_stream(stream));
}

int iw_attention(const int8_t *q, int64_t q_sb, int64_t q_st, const int8_t *k, int64_t k_sb,
                 int64_t k_sh, int64_t k_st, const int8_t *vt, int64_t v_sb, int64_t v_sh,
                 int64_t v_sd, int8_t *out, int64_t o_sb, int64_t o_st, const bool *mask,
                 int64_t batch, int64_t heads, int64_t q_length, int64_t k_length,
                 int64_t head_dim, uint8_t qk_multiplier, int8_t qk_shift, int32_t frac_bits,
                 uint8_t av_multiplier, int8_t av_shift, uint32_t rsqrt_offset,
                 const uint8_t *table, bool decode, iw_stream_t stream) {
  IW_REQUIRE(frac_bits > 0 && frac_bits < 14, "frac_bits must be in [1, 14)");
  IW_REQUIRE(rsqrt_offset <= 29, "rsqrt_offset must be in [0,29]");
  IW_REQUIRE(head_dim > 0 && head_dim <= 128 && head_dim % 16 == 0,
             "fused attention needs head_dim % 16 == 0 and head_dim <= 128");
  IW_REQUIRE(batch >= 0 && heads > 0 && q_length >= 0 && k_length >= 0, "invalid attention shape");
  IW_REQUIRE(batch <= 0x7fffffff && q_length <= 0x7fffffff && k_length <= 0x7fffffff,
             "attention shape too large");
  if (batch * q_length == 0) return IW_OK;
  IW_REQUIRE(q && k && vt && out, "null tensor pointer");
  IW_REQUIRE(v_sd % 16 == 0 && v_sd >= ((k_length + 15) / 16) * 16,
             "transposed V rows must be 16-byte multiples covering k_length");
  const uintptr_t align = reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k) |
                          reinterpret_cast<uintptr_t>(vt) | (uintptr_t)q_sb | (uintptr_t)q_st |
                          (uintptr_t)k_sb | (uintptr_t)k_sh | (uintptr_t)k_st | (uintptr_t)v_sb |
                          (uintptr_t)v_sh;
  IW_REQUIRE((align & 15) == 0, "fused attention operands must be 16-byte aligned");
  AttnArgs a;
  a.q = q;
  a.q_sb = q_sb;
  a.q_st = q_st;
  a.k = k;
  a.k_sb = k_sb;
  a.k_sh = k_sh;
  a.k_st = k_st;
  a.vt = vt;
  a.v_sb = v_sb;
  a.v_sh = v_sh;
  a.v_sd = v_sd;
  a.vt_ld = v_sd;
  a.out = out;
  a.o_sb = o_sb;
  a.o_st = o_st;
  a.mask = reinterpret_cast<const uint8_t *>(mask);
  a.B = (int32_t)batch;
  a.H = (int32_t)heads;
  a.Tq = (int32_t)q_length;
  a.Tk = (int32_t)k_length;
  a.D = (int32_t)head_dim;
  a.qk_m = qk_multiplier;
  a.qk_s = (uint32_t)(qk_shift > 0 ? qk_shift : 0);
  a.frac_bits = frac_bits;
  a.av_m = av_multiplier;
  a.av_s = (uint32_t)(av_shift < 0 ? 0 : (av_shift > 32 ? 32 : av_shift));
  a.rsqrt_off = rsqrt_offset;
  a.lut = table;
  if (decode) {
    IW_REQUIRE(q_length <= 8, "decode attention handles at most 8 query rows");
    return launch_attn_decode(a, as_stream(stream));
  }
  IW_REQUIRE(table, "prefill attention needs the shift-exp table");
  IW_REQUIRE(v_sh == head_dim * v_sd && v_sb == heads * head_dim * v_sd,
             "prefill attention expects V^T as [B,H,D,v_sd]");
  int dev = 0, cus = 256;
  if (hipGetDevice(&dev) == hipSuccess) {
    int v = 0;
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && v > 0)
      cus = v;
  }
  return launch_attn_prefill(a, cus * (head_dim <= 64 ? 4 : 3), as_stream(stream));
}

int iw_transpose_heads(const int8_t *src, int64_t src_sb, int64_t src_st, int8_t *dst,
                       int64_t dst_sb, int64_t dst_sh, int64_t dst_sd, int64_t dst_sq, int64_t t_offset,
                       int64_t batch, int64_t positions, int64_t heads, int64_t head_dim,
                       iw_stream_t stream) {
  IW_REQUIRE(batch >= 0 && positions >= 0 && heads > 0 && head_dim > 0 && t_offset >= 0,
             "invalid transpose shape");
  IW_REQUIRE(dst_sq == 4 || (dst_sd == 4 && dst_sq >= 4 * head_dim),
             "dst_sq == 4 (transposed rows) or dst_sd == 4 with dst_sq >= 4 * head_dim (key quads)");
  IW_REQUIRE(batch <= 65535, "batch too large for the transpose grid");
  if (batch * positions == 0) return IW_OK;
  IW_REQUIRE(src && dst, "null tensor pointer");
  return launch_transpose_heads(src, src_sb, src_st, dst, dst_sb, dst_sh, dst_sd, dst_sq, t_offset, batch,
                                positions, heads, head_dim, as_stream(stream));
}

int iw_gather_heads(const int8_t *src, int64_t src_sb, int64_t src_st, int8_t *dst, int64_t dst_sb,
                    int64_t dst_sh, int64_t dst_st, int64_t t_offset, int64_t batch,
                    int64_t positions, int64_t heads, int64_t head_dim, iw_stream_t stream) {
  IW_REQUIRE(batch >= 0 && positions >= 0 && heads > 0 && head_dim > 0 && t_offset >= 0,
             "invalid gather shape");
  IW_REQUIRE(head_dim % 16 == 0, "gather_heads needs head_dim % 16 == 0");
  if (batch * positions == 0) return IW_OK;
  IW_REQUIRE(src && dst, "null tensor pointer");
  const uintptr_t align = reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst) |
                          (uintptr_t)src_sb | (uintptr_t)src_st | (uintptr_t)dst_sb |
                          (uintptr_t)dst_sh | (uintptr_t)dst_st;
  IW_REQUIRE((align & 15) == 0, "gather_heads operands must be 16-byte aligned");
  return launch_gather_heads(src, src_sb, src_st, dst, dst_sb, dst_sh, dst_st, t_offset, batch,
                             positions, heads, head_dim, as_stream(stream));
}

int iw_copy_rows(const int8_t *src, int64_t src_sb, int64_t src_st, int8_t *dst, int64_t dst_sb,
                 int64_t dst_st, int64_t t_offset, int64_t batch, int64_t positions,
                 int64_t channels, iw_stream_t stream) {
  IW_REQUIRE(batch >= 0 && positions >= 0 && channels > 0 && t_offset >= 0, "invalid copy shape");
  if (batch * positions == 0) return IW_OK;
  IW_REQUIRE(src && dst, "null tensor pointer");
  return launch_copy_rows(src, src_sb, src_st, dst, dst_sb, dst_st, t_offset, batch, positions,
                          channels, as_stream(stream));
}

int iw_linear8_qkv_cache(const int8_t *x, const int8_t *weight, const int32_t *bias,
                         const int8_t *weight_zero, const uint32_t *multiplier, const int8_t *shift,
                         int64_t M, int64_t K, bool has_bias, bool asymmetric, int8_t *q_out,
                         int64_t q_ld, int8_t *k_cache, int64_t k_sb, int64_t k_sh, int64_t k_st,
                         int8_t *v_cache, int64_t v_sb, int64_t v_sh, int64_t v_sd, int64_t v_sq,
                         int64_t channels, int64_t head_dim, int64_t tokens_per_row_group,
                         int64_t cache_positions, const int32_t *pos, iw_stream_t stream) {
  GemmArgs g;
  SkinnyScatter sc;
  int rc = qkv_cache_args(x, weight, bias, weight_zero, multiplier, shift, M, K, has_bias, asymmetric, q_out,
                          q_ld, k_cache, k_sb, k_sh, k_st, v_cache, v_sb, v_sh, v_sd, v_sq, channels, head_dim,
                          tokens_per_row_group, cache_positions, pos, &g, &sc);
  if (rc || M == 0) return rc;
  IW_REQUIRE(gemm_skinny_eligible(g), "QKV projection needs K % 16 == 0 and 16-byte aligned operands");
  return gemm_skinny(g, &sc, as_stream(stream));
}

int iw_attention_decode_cache(const int8_t *q, int64_t q_sb, const int8_t *k, int64_t k_sb,
                              int64_t k_sh, int64_t k_st, const int8_t *vt, int64_t v_sb,
                              int64_t v_sh, int64_t v_sd, int64_t v_sq, int8_t *out, int64_t o_sb,
                              int64_t batch, int64_t heads, int64_t head_dim, int64_t k_length,
                              const int32_t *pos, int64_t max_keys, uint8_t qk_multiplier,
                              int8_t qk_shift, int32_t frac_bits, uint8_t av_multiplier,
                              int8_t av_shift, uint32_t rsqrt_offset, iw_stream_t stream) {
  return attention_decode_cache_entry(q, q_sb, k, k_sb, k_sh, k_st, vt, v_sb, v_sh, v_sd, v_sq, out, o_sb, batch,
                                      heads,
                                      head_dim, k_length, pos, max_keys, qk_multiplier, qk_shift, frac_bits,
                                      av_multiplier, av_shift, rsqrt_offset, false, stream);
}

int iw_embed_tokens(const int64_t *tokens, const int8_t *table, const int8_t *pe,
                    int64_t pe_rows, const int32_t *pos, const uint16_t *multiplier,
                    const int8_t *shift, int16_t *out, int64_t batch, int64_t channels,
                    iw_stream_t stream) {
  IW_REQUIRE(batch >= 0 && channels > 0 && pe_rows > 0, "invalid embedding shape");
  if (batch == 0) return IW_OK;
  IW_REQUIRE(tokens && table && pe && pos && multiplier && shift && out, "null tensor pointer");
  return launch_add_requant15(table, tokens, pe, multiplier, shift, out, batch, 1, channels, 0, 0,
                              as_stream(stream), pos, pe_rows);
}

int iw_greedy_advance(const int8_t *logits, int64_t rows, int64_t cols, int64_t ld,
                      int64_t *next_tokens, int64_t *history, int64_t history_ld,
                      int64_t history_cols, int32_t *step, int32_t *pos, int32_t pos_increment,
                      iw_stream_t stream) {
  IW_REQUIRE(rows >= 0 && cols > 0 && cols < (1 << 23) && ld >= cols && history_cols > 0 &&
                 history_ld >= history_cols,
             "invalid greedy step shape (at most 2^23 - 1 columns)");
  IW_REQUIRE(logits && next_tokens && history && step && pos, "null tensor pointer");
  return launch_greedy_step(logits, rows, cols, ld, next_tokens, history, history_ld, history_cols, step,
                            pos, pos_increment, as_stream(stream));
}

int iw_greedy_advance_filtered(const int8_t *logits, int64_t rows, int64_t cols, int64_t ld,
                               int64_t *next_tokens, int64_t *history, int64_t history_ld,
                               int64_t history_cols, int32_t *step, int32_t *pos,
                               int32_t pos_increment, const uint32_t *suppress,
                               const uint32_t *suppress_first, const int64_t *prev0, int32_t eot,
                               int32_t timestamp_begin, int32_t max_initial_timestamp,
                               float logit_scale, float *sum_logprobs, int32_t *eot_count,
                               iw_stream_t stream) {
  IW_REQUIRE(rows >= 0 && cols > 0 && cols < (1 << 23) && ld >= cols && history_cols > 0 &&
                 history_ld >= history_cols,
             "invalid greedy step shape (at most 2^23 - 1 columns)");
  IW_REQUIRE(logits && next_tokens && history && step && pos, "null tensor pointer");
  IW_REQUIRE(timestamp_begin < 0 || eot >= 0, "the timestamp rules need the EOT id");
  IW_REQUIRE((timestamp_begin < 0 && !sum_logprobs) || logit_scale > 0.f, "logit_scale must be positive");
  return launch_greedy_step_filtered(logits, rows, cols, ld, next_tokens, history, history_ld, history_cols,
                                     step, pos, pos_increment, suppress, suppress_first, prev0, eot,
                                     timestamp_begin, max_initial_timestamp, logit_scale, sum_logprobs,
                                     eot_count, as_stream(stream));
}

int iw_greedy_update(const uint16_t *row_max, int64_t tiles, const int8_t *logits, int64_t ld, int64_t rows,
                     int64_t cols, int64_t *next_tokens, int64_t *history, int64_t history_ld,
                     int64_t history_cols, int32_t *step, int32_t *pos, int32_t pos_increment, int32_t eot,
                     const int64_t *prev0, float *sum_logprobs, float logit_scale, int32_t *eot_count,
                     uint32_t *arrive, iw_stream_t stream) {
  IW_REQUIRE(rows >= 0 && rows < (1LL << 31) && cols > 0 && cols < (1 << 23) && history_cols > 0 &&
                 history_ld >= history_cols,
             "invalid greedy step shape (at most 2^23 - 1 columns)");
  IW_REQUIRE(!row_max || tiles == (cols + 31) / 32, "tiles must be ceil(cols / 32)");
  IW_REQUIRE((row_max || logits) && (!logits || ld >= cols), "the row maxima or the logits are needed");
  IW_REQUIRE(!sum_logprobs || (logits && logit_scale > 0.f), "log-probabilities need the logits and a positive scale");
  IW_REQUIRE(next_tokens && history && step && pos && arrive, "null tensor pointer");
  if (rows == 0) return IW_OK;
  return launch_greedy_update(row_max, tiles, logits, ld, rows, cols, next_tokens, history, history_ld,
                              history_cols, step, pos, pos_increment, eot, prev0, sum_logprobs, logit_scale,
                              eot_count, arrive, as_stream(stream));
}

int iw_token_prob(const int8_t *logits, int64_t rows, int64_t cols, int64_t ld, int64_t token, float logit_scale,
                  float *out, iw_stream_t stream) {
  IW_REQUIRE(rows >= 0 && cols > 0 && cols < (1 << 30) && ld >= cols, "invalid logits shape");
  IW_REQUIRE(token >= 0 && token < cols, "token outside the vocabulary");
  IW_REQUIRE(logit_scale > 0.f, "logit_scale must be positive");
  if (rows == 0) return IW_OK;
  IW_REQUIRE(logits && out, "null tensor pointer");
  return launch_token_prob(logits, rows, cols, ld, token, logit_scale, out, as_stream(stream));
}


int iw_log_mel(const float *audio, int64_t batch, int64_t n_samples, int64_t audio_ld, const float *twiddle,
               const float *window, const int32_t *filter_start, const int32_t *filter_len,
               const int32_t *filter_offset, const float *filter_weights, int32_t n_taps, int32_t n_mels,
               float *out, int64_t out_batch_stride, float *workspace, iw_stream_t stream) {
  int rc = check_log_mel(audio, batch, n_samples, audio_ld, twiddle, window, filter_start, filter_len,
                         filter_offset, filter_weights, n_taps, n_mels, out, out_batch_stride);
  if (rc != IW_OK || batch == 0) return rc;
  IW_REQUIRE(workspace, "null tensor pointer");
  return launch_log_mel(audio, batch, n_samples, audio_ld, twiddle, window, filter_start, filter_len,
                        filter_offset, filter_weights, n_taps, n_mels, out, out_batch_stride, workspace,
                        as_stream(stream));
}

int64_t iw_log_mel_scratch_floats(int64_t batch, int64_t n_samples) {
  if (batch < 0 || n_samples < 0) return -1;
  return batch * ((n_samples / 160 + 63) / 64);
}

int iw_log_mel_noalloc(const float *audio, int64_t batch, int64_t n_samples, int64_t audio_ld,
                       const float *twiddle, const float *window, const int32_t *filter_start,
                       const int32_t *filter_len, const int32_t *filter_offset, const float *filter_weights,
                       int32_t n_taps, int32_t n_mels, float *out, int64_t out_batch_stride,
                       iw_stream_t stream) {
  int rc = check_log_mel(audio, batch, n_samples, audio_ld, twiddle, window, filter_start, filter_len,
                         filter_offset, filter_weights, n_taps, n_mels, out, out_batch_stride);
  if (rc != IW_OK || batch == 0) return rc;
  IW_REQUIRE(iw_log_mel_scratch_floats(batch, n_samples) <= IW_LOG_MEL_SCRATCH_FLOATS,
             "iw_log_mel_noalloc: batch * ceil((n_samples / 160) / 64) exceeds the fixed scratch of "
             "IW_LOG_MEL_SCRATCH_FLOATS (65536) block maxima; use iw_log_mel with a workspace");
  float *blockmax = nullptr;
  rc = log_mel_scratch(as_stream(stream), &blockmax);
  if (rc != IW_OK) return rc;
  // every block of the transform kernel writes its own maximum before the
  // finishing kernel reads it, so nothing needs clearing between calls
  return launch_log_mel(audio, batch, n_samples, audio_ld, twiddle, window, filter_start, filter_len,
                        filter_offset, filter_weights, n_taps, n_mels, out, out_batch_stride, blockmax,
                        as_stream(stream));
}

int iw_dtw(const float *x, int64_t rows, int64_t cols, int64_t ld, int8_t *trace, int64_t trace_ld,
           iw_stream_t stream) {
  IW_REQUIRE(rows > 0 && rows < 1024 && cols > 0 && cols < (1 << 30) && ld >= cols && trace_ld >= cols + 1,
             "invalid DTW shape (1 <= rows < 1024)");
  IW_REQUIRE(x && trace, "null tensor pointer");
  return launch_dtw(x, rows, cols, ld, trace, trace_ld, as_stream(stream));
}

int iw_median_filter(const float *x, int64_t rows, int64_t cols, int64_t ld, int32_t width, float *y,
                     int64_t y_ld, iw_stream_t stream) {
  IW_REQUIRE(width > 0 && width % 2 == 1 && width <= 31, "filter width must be odd and at most 31");
  IW_REQUIRE(rows >= 0 && cols > width / 2 && cols < (1 << 30) && ld >= cols && y_ld >= cols,
             "invalid median filter shape (the row must be longer than width / 2)");
  if (rows == 0) return IW_OK;
  IW_REQUIRE(x && y, "null tensor pointer");
  return launch_median_filter(x, rows, cols, ld, width, y, y_ld, as_stream(stream));
}

int iw_argmax_rows(const int8_t *x, int64_t rows, int64_t cols, int64_t ld, int64_t *out,
                   iw_stream_t stream) {
  IW_REQUIRE(rows >= 0 && cols > 0 && cols < (1 << 23) && ld >= cols,
             "invalid argmax shape (at most 2^23 - 1 columns)");
  if (rows == 0) return IW_OK;
  IW_REQUIRE(x && out, "null tensor pointer");
  return launch_argmax_rows(x, rows, cols, ld, out, as_stream(stream));
}

// ---- fragment-major decode operands ----

int64_t iw_frag_bytes(int64_t rows, int64_t cols) {
  if (rows < 0 || cols < 0 || cols > kFragMaxK) return 0;
  return frag_rpad(rows) * frag_kpad(cols);
}

int iw_frag_pack(const int8_t *src, int64_t rows, int64_t cols, int64_t ld, int8_t *dst, iw_stream_t stream) {
  IW_REQUIRE(rows >= 0 && cols >= 0 && cols <= kFragMaxK, "fragment-major matrices have at most 5120 columns");
  IW_REQUIRE(ld >= cols, "ld must be at least cols");
  if (rows == 0 || cols == 0) return IW_OK;
  IW_REQUIRE(src && dst, "null tensor pointer");
  IW_REQUIRE((reinterpret_cast<uintptr_t>(dst) & 15) == 0, "dst must be 16-byte aligned");
  return launch_frag_pack(src, rows, cols, ld, dst, as_stream(stream));
}

int iw_linear8_frag(const int8_t *x, const int8_t *weight, const int32_t *bias, const int8_t *weight_zero,
                    const uint32_t *multiplier, const int8_t *shift, int8_t *out, int64_t M, int64_t K, int64_t N,
                    bool has_bias, bool asymmetric, bool out_frag, iw_stream_t stream) {
  int rc = check_linear(x, weight, bias, weight_zero, multiplier, shift, out, M, K, N, has_bias, asymmetric);
  if (rc || M == 0) return rc;
  rc = check_frag(x, weight, M, K, N);
  if (rc) return rc;
  IW_REQUIRE(!out_frag || N <= kFragMaxK, "a fragment-major output has at most 5120 columns");
  GemmArgs g = linear_args(x, weight, bias, weight_zero, multiplier, shift, out, M, K, N, has_bias, asymmetric,
                           EPI_L8);
  if (out_frag) g.ldc = frag_kpad(N);
  return gemm_frag(g, nullptr, out_frag, as_stream(stream));
}

int iw_linear8_gelu_frag(const int8_t *x, const int8_t *weight, const int32_t *bias, const int8_t *weight_zero,
                         const uint32_t *multiplier, const int8_t *shift, const uint8_t *lut,
                         const uint8_t *luti_multiplier, const int8_t *luti_shift, const uint8_t *luto_multiplier,
                         const int8_t *luto_shift, int64_t luti_count, int64_t luto_count, int8_t *out, int64_t M,
                         int64_t K, int64_t N, bool has_bias, bool asymmetric, bool out_frag,
                         const int8_t *next_weight, int64_t next_n, int64_t next_k, iw_stream_t stream) {
  int rc = check_linear(x, weight, bias, weight_zero, multiplier, shift, out, M, K, N, has_bias, asymmetric);
  if (rc) return rc;
  rc = check_gelu_counts(N, luti_count, luto_count);
  if (rc || M == 0) return rc;
  rc = check_frag(x, weight, M, K, N);
  if (rc) return rc;
  FragPrefetch pf;
  rc = frag_prefetch_args(next_weight, next_n, next_k, &pf);
  if (rc) return rc;
  IW_REQUIRE(!out_frag || N <= kFragMaxK, "a fragment-major output has at most 5120 columns");
  IW_REQUIRE(lut && luti_multiplier && luti_shift && luto_multiplier && luto_shift, "null GeLU parameter pointer");
  GemmArgs g = linear_args(x, weight, bias, weight_zero, multiplier, shift, out, M, K, N, has_bias, asymmetric,
                           EPI_L8);
  g.lut = lut;
  g.luti_m = luti_multiplier;
  g.luti_s = luti_shift;
  g.luto_m = luto_multiplier;
  g.luto_s = luto_shift;
  g.luti_pc = luti_count != 1;
  g.luto_pc = luto_count != 1;
  g.pf = pf;
  if (out_frag) g.ldc = frag_kpad(N);
  return gemm_frag(g, nullptr, out_frag, as_stream(stream));
}

int iw_linear32_residual15_frag(const int8_t *x, const int8_t *weight, const int32_t *bias,
                                const int8_t *weight_zero, const uint32_t *multiplier, const int8_t *shift,
                                const int16_t *residual, uint16_t residual_multiplier, int16_t *out, int64_t M,
                                int64_t K, int64_t N, bool has_bias, bool asymmetric, iw_stream_t stream) {
  int rc = check_linear(x, weight, bias, weight_zero, multiplier, shift, out, M, K, N, has_bias, asymmetric);
  if (rc || M == 0) return rc;
  rc = check_frag(x, weight, M, K, N);
  if (rc) return rc;
  IW_REQUIRE(residual, "null residual pointer");
  GemmArgs g = linear_args(x, weight, bias, weight_zero, multiplier, shift, out, M, K, N, has_bias, asymmetric,
                           EPI_L32RES);
  g.res = residual;
  g.ldres = N;
  g.res_mult = residual_multiplier;
  return gemm_frag(g, nullptr, false, as_stream(stream));
}

int iw_linear8_qkv_cache_frag(const int8_t *x, const int8_t *weight, const int32_t *bias,
                              const int8_t *weight_zero, const uint32_t *multiplier, const int8_t *shift,
                              int64_t M, int64_t K, bool has_bias, bool asymmetric, int8_t *q_out, int64_t q_ld,
                              int8_t *k_cache, int64_t k_sb, int64_t k_sh, int64_t k_st, int8_t *v_cache,
                              int64_t v_sb, int64_t v_sh, int64_t v_sd, int64_t v_sq, int64_t channels,
                              int64_t head_dim, int64_t tokens_per_row_group, int64_t cache_positions,
                              const int32_t *pos, iw_stream_t stream) {
  GemmArgs g;
  SkinnyScatter sc;
  int rc = qkv_cache_args(x, weight, bias, weight_zero, multiplier, shift, M, K, has_bias, asymmetric, q_out,
                          q_ld, k_cache, k_sb, k_sh, k_st, v_cache, v_sb, v_sh, v_sd, v_sq, channels, head_dim,
                          tokens_per_row_group, cache_positions, pos, &g, &sc);
  if (rc || M == 0) return rc;
  rc = check_frag(x, weight, M, K, 3 * channels);
  if (rc) return rc;
  return gemm_frag(g, &sc, false, as_stream(stream));
}

int iw_layernorm32_frag(const int16_t *x, const int8_t *weight, const int32_t *bias, uint8_t ln_multiplier,
                        int8_t ln_shift, uint32_t out_multiplier, int8_t out_shift, uint32_t rsqrt_offset,
                        int8_t *out, int64_t rows, int64_t hidden, bool has_bias, const int8_t *next_weight,
                        int64_t next_n, int64_t next_k, iw_stream_t stream) {
  FragPrefetch pf;
  const int rc = frag_prefetch_args(next_weight, next_n, next_k, &pf);
  if (rc) return rc;
  return layernorm32_entry(x, weight, bias, ln_multiplier, ln_shift, out_multiplier, out_shift, rsqrt_offset, out,
                           rows, hidden, has_bias, true, stream, &pf);
}

int iw_attention_decode_cache_frag(const int8_t *q, int64_t q_sb, const int8_t *k, int64_t k_sb, int64_t k_sh,
                                   int64_t k_st, const int8_t *vt, int64_t v_sb, int64_t v_sh, int64_t v_sd,
                                   int64_t v_sq, int8_t *out, int64_t batch, int64_t heads, int64_t head_dim,
                                   int64_t k_length, const int32_t *pos, int64_t max_keys, uint8_t qk_multiplier,
                                   int8_t qk_shift, int32_t frac_bits, uint8_t av_multiplier, int8_t av_shift,
                                   uint32_t rsqrt_offset, const int8_t *next_weight, int64_t next_n,
                                   int64_t next_k, iw_stream_t stream) {
  FragPrefetch pf;
  const int rc = frag_prefetch_args(next_weight, next_n, next_k, &pf);
  if (rc) return rc;
  return attention_decode_cache_entry(q, q_sb, k, k_sb, k_sh, k_st, vt, v_sb, v_sh, v_sd, v_sq, out, 0, batch,
                                      heads, head_dim, k_length, pos, max_keys, qk_multiplier, qk_shift, frac_bits,
                                      av_multiplier, av_shift, rsqrt_offset, true, stream, &pf);
}

int iw_attention_decode_cross_lnq(const int16_t *x, int64_t x_ld, const int8_t *ln_weight, const int32_t *ln_bias,
                                  uint8_t ln_multiplier, int8_t ln_shift, uint32_t ln_out_multiplier,
                                  int8_t ln_out_shift, uint32_t ln_rsqrt_offset, bool ln_has_bias,
                                  const int8_t *q_weight, const int32_t *q_bias, const int8_t *q_weight_zero,
                                  const uint32_t *q_multiplier, const int8_t *q_shift, bool q_has_bias,
                                  bool q_asymmetric, const int8_t *k, int64_t k_sb, int64_t k_sh, int64_t k_st,
                                  const int8_t *vt, int64_t v_sb, int64_t v_sh, int64_t v_sd, int8_t *out,
                                  int64_t batch, int64_t heads, int64_t head_dim, int64_t k_length,
                                  uint8_t qk_multiplier, int8_t qk_shift, int32_t frac_bits, uint8_t av_multiplier,
                                  int8_t av_shift, uint32_t rsqrt_offset, iw_stream_t stream) {
  IW_REQUIRE(frac_bits > 0 && frac_bits < 14, "frac_bits must be in [1, 14)");
  IW_REQUIRE(rsqrt_offset <= 29, "rsqrt_offset must be in [0,29]");
  IW_REQUIRE(head_dim == 64, "the fused cross-attention takes head_dim 64");
  const int64_t C = heads * head_dim;
  const int code = layernorm_width_code(C);
  IW_REQUIRE(code >= 0, "unsupported LayerNorm hidden size: " + std::to_string(C));
  IW_REQUIRE(batch >= 0 && batch <= kSkinnyMaxRows && k_length > 0 && k_length <= 2048,
             "the fused cross-attention takes at most 128 rows and 1 .. 2048 keys");
  IW_REQUIRE(x_ld >= C, "x_ld must be at least heads * head_dim");
  IW_REQUIRE(v_sd % 16 == 0 && v_sd >= ((k_length + 15) / 16) * 16,
             "transposed V rows must be 16-byte multiples covering k_length");
  if (batch == 0) return IW_OK;
  IW_REQUIRE(x && ln_weight && q_weight && q_multiplier && q_shift && k && vt && out, "null tensor pointer");
  IW_REQUIRE(!ln_has_bias || ln_bias, "ln_has_bias set but ln_bias is null");
  IW_REQUIRE(!q_has_bias || q_bias, "q_has_bias set but q_bias is null");
  IW_REQUIRE(!q_asymmetric || q_weight_zero, "q_asymmetric set but q_weight_zero is null");
  const uintptr_t align = reinterpret_cast<uintptr_t>(q_weight) | reinterpret_cast<uintptr_t>(k) |
                          reinterpret_cast<uintptr_t>(vt) | (uintptr_t)k_sb | (uintptr_t)k_sh | (uintptr_t)k_st |
                          (uintptr_t)v_sb | (uintptr_t)v_sh;
  IW_REQUIRE((align & 15) == 0, "decode attention operands must be 16-byte aligned");
  IW_REQUIRE((reinterpret_cast<uintptr_t>(x) & 1) == 0, "x must be 2-byte aligned");
  AttnArgs a;
  a.k = k;
  a.k_sb = k_sb;
  a.k_sh = k_sh;
  a.k_st = k_st;
  a.vt = vt;
  a.v_sb = v_sb;
  a.v_sh = v_sh;
  a.v_sd = v_sd;
  a.v_sq = 4;
  a.vt_ld = v_sd;
  a.out = out;
  a.B = (int32_t)batch;
  a.H = (int32_t)heads;
  a.Tq = 1;
  a.Tk = (int32_t)k_length;
  a.D = (int32_t)head_dim;
  a.qk_m = qk_multiplier;
  a.qk_s = (uint32_t)(qk_shift > 0 ? qk_shift : 0);
  a.frac_bits = frac_bits;
  a.av_m = av_multiplier;
  a.av_s = (uint32_t)(av_shift < 0 ? 0 : (av_shift > 32 ? 32 : av_shift));
  a.rsqrt_off = rsqrt_offset;
  a.max_tk = (int32_t)k_length;
  a.o_frag_kp = frag_kpad(C);
  LnQueryArgs lq;
  lq.x = x;
  lq.ldx = x_ld;
  lq.gamma = ln_weight;
  lq.beta = ln_has_bias ? ln_bias : nullptr;
  lq.ln_m = ln_multiplier;
  lq.ln_s = ln_shift;
  lq.out_m = ln_out_multiplier;
  lq.out_s = ln_out_shift;
  lq.rsqrt_off = ln_rsqrt_offset;
  lq.code = code;
  lq.hidden = (int32_t)C;
  lq.wq = q_weight;
  lq.kp = frag_kpad(C);
  lq.bias = q_has_bias ? q_bias : nullptr;
  lq.wz = q_asymmetric ? q_weight_zero : nullptr;
  lq.mult = q_multiplier;
  lq.shift = q_shift;
  return launch_attn_decode_cross_lnq(a, lq, as_stream(stream));
}

int iw_classifier_argmax_frag(const int8_t *x, const int8_t *weight, uint32_t multiplier, int8_t shift,
                              int8_t *out, uint16_t *row_max, int64_t M, int64_t K, int64_t N,
                              iw_stream_t stream) {
  IW_REQUIRE(K > 0, "hidden size must be positive");
  IW_REQUIRE(N > 0 && N < (1 << 23), "vocabulary size must be in 1 .. 2^23 - 1");
  IW_REQUIRE(M >= 0, "invalid row count");
  if (M == 0) return IW_OK;
  IW_REQUIRE(x && weight && row_max, "null tensor pointer");
  int rc = check_frag(x, weight, M, K, N);
  if (rc) return rc;
  GemmArgs g;
  g.a = x;
  g.b = weight;
  g.M = M;
  g.N = N;
  g.K = K;
  g.epi = EPI_S8;
  g.mult_pc = 0;
  g.out = out;
  g.ldc = N;
  g.scalar_mult = multiplier;
  g.scalar_shift = shift;
  g.amax = row_max;
  g.amax_ld = (N + 31) / 32;
  return gemm_frag(g, nullptr, false, as_stream(stream));
}

int iw_classifier_frag(const int8_t *x, const int8_t *weight, uint32_t multiplier, int8_t shift, int8_t *out,
                       int64_t M, int64_t K, int64_t N, iw_stream_t stream) {
  IW_REQUIRE(K > 0, "hidden size must be positive");
  IW_REQUIRE(N > 0, "vocabulary size must be positive");
  IW_REQUIRE(M >= 0, "invalid row count");
  if (M == 0) return IW_OK;
  IW_REQUIRE(x && weight && out, "null tensor pointer");
  int rc = check_frag(x, weight, M, K, N);
  if (rc) return rc;
  GemmArgs g;
  g.a = x;
  g.b = weight;
  g.M = M;
  g.N = N;
  g.K = K;
  g.epi = EPI_S8;
  g.mult_pc = 0;
  g.out = out;
  g.ldc = N;
  g.scalar_mult = multiplier;
  g.scalar_shift = shift;
  return gemm_frag(g, nullptr, false, as_stream(stream));
}

}  // extern "C"
