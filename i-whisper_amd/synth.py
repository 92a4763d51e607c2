"""Synthetic inputs and a synthetic integer checkpoint for the benchmark workloads.

* ``synthetic_mel``: seeded 30 s log-mel, values ~ N(-0.5, 0.4) clipped to
  [-1.5, 1.5], float32 [B, n_mels, frames].
* ``calibrated_int_params``: random-init float Whisper weights (N(0, 0.02) for
  every linear / conv / embedding weight and bias, LayerNorm gamma = 1 and
  beta = 0, sinusoidal encoder positions), a float calibration forward on
  seeded synthetic mels and prompt tokens, then conversion to the integer
  parameters of ``Whisper_int`` (reference state-dict names and dtypes).

The conversion restates the structure of the reference's offline quantiser
(i_whisper/model_quant.py): activation scales alpha = range / absmax from the
calibration pass, per-output-channel asymmetric int8 weights with zero points
(model_quant.py:670-735), and every requantisation multiplier / shift derived
with frexp (model_quant.py:170-193, 357-394, 1187-1200). The exact search and
EMA choices of the reference calibration are not reproduced (they only decide
which integers the checkpoint holds; both the HIP path and the oracle consume
the same integers).
"""
from __future__ import annotations

import math
from typing import Dict, Optional, Sequence

import numpy as np
import torch

from .model_int import ModelDimensions

PROMPT = (50258, 50259, 50359)  # <|startoftranscript|><|en|><|transcribe|>


def synthetic_mel(batch: int, n_mels: int, frames: int, seed: int) -> np.ndarray:
    r = np.random.default_rng(seed)
    return np.clip(r.normal(-0.5, 0.4, size=(batch, n_mels, frames)), -1.5, 1.5).astype(np.float32)


def prompt_tokens(batch: int, n_vocab: int, seed: Optional[int] = None, length: int = 3) -> np.ndarray:
    """The Whisper start prompt (ids folded into the vocabulary of small test
    models), or uniform random ids in [0, n_vocab) when a seed is given."""
    if seed is not None:
        return np.random.default_rng(seed).integers(0, n_vocab, size=(batch, length)).astype(np.int64)
    base = np.array([t % n_vocab for t in PROMPT[:length]], np.int64)
    return np.tile(base, (batch, 1))


# ---------------------------------------------------------------------------
# float reference model (CPU, float32) used for calibration only
# ---------------------------------------------------------------------------

def _sinusoids(length: int, channels: int, max_timescale: float = 10000.0) -> torch.Tensor:
    inc = math.log(max_timescale) / (channels // 2 - 1)
    inv = torch.exp(-inc * torch.arange(channels // 2))
    t = torch.arange(length)[:, None] * inv[None, :]
    return torch.cat([torch.sin(t), torch.cos(t)], dim=1)


class _Gen:
    def __init__(self, seed: int):
        self.r = np.random.default_rng(seed)

    def normal(self, *shape, std=0.02):
        a = self.r.standard_normal(shape, dtype=np.float32)
        a *= np.float32(std)
        return torch.from_numpy(a)


def float_weights(dims: ModelDimensions, seed: int, decoder_mlp_scale: float = 1.0) -> Dict[str, torch.Tensor]:
    """Random-init float weights. ``decoder_mlp_scale`` scales the decoder MLPs'
    output weights and FC1 biases (1 = plain N(0, 0.02)): a random decoder's
    MLP adds the same direction to every position, so its greedy argmax hardly
    depends on the input; a small scale lets the argmax follow the input."""
    g = _Gen(seed)
    W: Dict[str, torch.Tensor] = {}
    d, dt = dims.n_audio_state, dims.n_text_state
    W["encoder.conv1.weight"] = g.normal(d, dims.n_mels, 3)
    W["encoder.conv1.bias"] = g.normal(d)
    W["encoder.conv2.weight"] = g.normal(d, d, 3)
    W["encoder.conv2.bias"] = g.normal(d)
    W["encoder.positional_embedding"] = _sinusoids(dims.n_audio_ctx, d)

    def block(p, n, cross):
        for ln in ["attn_ln", "mlp_ln"] + (["cross_attn_ln"] if cross else []):
            W[f"{p}.{ln}.weight"] = torch.ones(n)
            W[f"{p}.{ln}.bias"] = torch.zeros(n)
        for a in ["attn"] + (["cross_attn"] if cross else []):
            for lin in ("query", "key", "value", "out"):
                W[f"{p}.{a}.{lin}.weight"] = g.normal(n, n)
                if lin != "key":
                    W[f"{p}.{a}.{lin}.bias"] = g.normal(n)
        W[f"{p}.mlp.0.weight"] = g.normal(4 * n, n)
        W[f"{p}.mlp.0.bias"] = g.normal(4 * n)
        W[f"{p}.mlp.2.weight"] = g.normal(n, 4 * n)
        W[f"{p}.mlp.2.bias"] = g.normal(n)

    for i in range(dims.n_audio_layer):
        block(f"encoder.blocks.{i}", d, False)
    W["encoder.ln_post.weight"] = torch.ones(d)
    W["encoder.ln_post.bias"] = torch.zeros(d)
    W["decoder.token_embedding.weight"] = g.normal(dims.n_vocab, dt)
    W["decoder.positional_embedding"] = g.normal(dims.n_text_ctx, dt)
    for i in range(dims.n_text_layer):
        block(f"decoder.blocks.{i}", dt, True)
        if decoder_mlp_scale != 1.0:
            for k in ("mlp.0.bias", "mlp.2.weight", "mlp.2.bias"):
                W[f"decoder.blocks.{i}.{k}"] *= decoder_mlp_scale
    W["decoder.ln.weight"] = torch.ones(dt)
    W["decoder.ln.bias"] = torch.zeros(dt)
    return W


class _Stats:
    """absmax of every calibration point (max over all calibration batches)."""

    def __init__(self):
        self.v: Dict[str, float] = {}

    def __call__(self, name: str, t: torch.Tensor) -> torch.Tensor:
        m = float(t.detach().abs().max())
        self.v[name] = max(self.v.get(name, 0.0), m, 1e-8)
        return t


def _gelu(x):
    return x * torch.sigmoid(1.702 * x)


def _ln(x, W, p):
    return torch.nn.functional.layer_norm(x, x.shape[-1:], W[p + ".weight"], W[p + ".bias"])


def _attn(x, xa, W, p, n_head, st: _Stats, causal: bool):
    q = x @ W[p + ".query.weight"].T + W[p + ".query.bias"]
    src = x if xa is None else xa
    k = src @ W[p + ".key.weight"].T
    v = src @ W[p + ".value.weight"].T + W[p + ".value.bias"]
    st(p + ".q", q), st(p + ".k", k), st(p + ".v", v)
    B, T, C = q.shape
    D = C // n_head
    qh = q.view(B, T, n_head, D).transpose(1, 2)
    kh = k.view(B, -1, n_head, D).transpose(1, 2)
    vh = v.view(B, -1, n_head, D).transpose(1, 2)
    logits = qh @ kh.transpose(-1, -2) / math.sqrt(D)
    if causal:
        Tk = kh.shape[2]
        mask = torch.ones(T, Tk, dtype=torch.bool).triu(1 + Tk - T)
        logits = logits.masked_fill(mask, float("-inf"))
    st(p + ".qk", logits.masked_fill(torch.isinf(logits), 0.0))
    o = (torch.softmax(logits, -1) @ vh).transpose(1, 2).reshape(B, T, C)
    st(p + ".wv", o)
    return o @ W[p + ".out.weight"].T + W[p + ".out.bias"]


def _block(x, xa, W, p, n_head, st, causal):
    st(p + ".in", x)
    x = x + _attn(st(p + ".attn_ln.out", _ln(x, W, p + ".attn_ln")), None, W, p + ".attn", n_head,
                  st, causal)
    st(p + ".mid", x)
    if xa is not None:
        x = x + _attn(st(p + ".cross_attn_ln.out", _ln(x, W, p + ".cross_attn_ln")), xa, W,
                      p + ".cross_attn", n_head, st, False)
        st(p + ".mid2", x)
    h = st(p + ".mlp_ln.out", _ln(x, W, p + ".mlp_ln"))
    h = st(p + ".fc1", h @ W[p + ".mlp.0.weight"].T + W[p + ".mlp.0.bias"])
    h = st(p + ".gelu", _gelu(h))
    x = x + h @ W[p + ".mlp.2.weight"].T + W[p + ".mlp.2.bias"]
    return st(p + ".out", x)


@torch.no_grad()
def _calibrate(dims: ModelDimensions, W, mels: torch.Tensor, tokens: torch.Tensor) -> _Stats:
    st = _Stats()
    ctx = mels.shape[-1] // 2
    st("encoder.mel", mels)
    c1 = torch.nn.functional.conv1d(mels, W["encoder.conv1.weight"], W["encoder.conv1.bias"], padding=1)
    st("encoder.conv1", c1)
    g1 = st("encoder.gelu1", _gelu(c1))
    c2 = torch.nn.functional.conv1d(g1, W["encoder.conv2.weight"], W["encoder.conv2.bias"], stride=2,
                                    padding=1)
    st("encoder.conv2", c2)
    g2 = st("encoder.gelu2", _gelu(c2)).permute(0, 2, 1)
    x = g2 + W["encoder.positional_embedding"][:ctx]
    for i in range(dims.n_audio_layer):
        x = _block(x, None, W, f"encoder.blocks.{i}", dims.n_audio_head, st, False)
    xa = st("encoder.ln_post.out", _ln(x, W, "encoder.ln_post"))
    T = tokens.shape[1]
    y = W["decoder.token_embedding.weight"][tokens] + W["decoder.positional_embedding"][:T]
    for i in range(dims.n_text_layer):
        y = _block(y, xa, W, f"decoder.blocks.{i}", dims.n_text_head, st, True)
    h = st("decoder.ln.out", _ln(y, W, "decoder.ln"))
    st("decoder.logits", h @ W["decoder.token_embedding.weight"].T)
    return st


# ---------------------------------------------------------------------------
# float -> integer conversion
# ---------------------------------------------------------------------------

def _frexp(r: float, bits: int):
    """(m, e) with r ~= m * 2^(e - bits), m in [2^(bits-1), 2^bits)."""
    f, e = math.frexp(r)
    m = int(round(f * (1 << bits)))
    if m >= (1 << bits):
        m >>= 1
        e += 1
    return m, e


def _mulh_shift(r: float):
    """uint32 multiplier and right shift with mulh(acc, m) >> s ~= acc * r (r < 1)."""
    m, e = _frexp(r, 32)
    s = -e
    if s < 0:  # gain >= 1 is not representable: saturate the gain to ~1
        return 0xFFFFFFFF, 0
    return m, min(s, 31)


def _mulh_lshift(r: float):
    """uint32 multiplier and left shift with mulh(acc, m) << s ~= acc * r."""
    m, e = _frexp(r, 32)
    if e >= 0:
        return m, min(e, 31)
    return max(1, int(round(m * 2.0 ** e))), 0


def _mul8_shift(r: float, trunc: bool = False):
    """uint8 multiplier m in [64,128) and shift s >= 0 with (x*m) >> s ~= x * r
    (model_quant.py:1187-1200 form)."""
    f, e = math.frexp(r)
    m = int(f * 128) if trunc else int(round(f * 128))
    if m >= 128:
        m //= 2
        e += 1
    return max(1, m), int(min(max(7 - e, 0), 32))


def _mul16_shift(r: float):
    f, e = math.frexp(r)
    m = int(round(f * 65536))
    if m >= 65536:
        m //= 2
        e += 1
    return m, int(min(max(16 - e, 0), 32))


def _alpha(st: _Stats, name: str, rng: float = 127.0) -> float:
    return rng / st.v[name]


def _quant_w_per_channel(w: torch.Tensor):
    """Asymmetric per-output-channel int8: w ~= s_n * (w_int - wz_n)."""
    w = w.reshape(w.shape[0], -1).double()
    lo, hi = w.min(1).values, w.max(1).values
    scale = ((hi - lo) / 254.0).clamp_min(1e-12)
    centre = (hi + lo) / 2
    w_int = torch.round((w - centre[:, None]) / scale[:, None]).clamp(-127, 127)
    wz = torch.round(-centre / scale).clamp(-128, 127)
    w_int = (w_int + wz[:, None]).clamp(-128, 127)
    return w_int.to(torch.int8), wz.to(torch.int8), 1.0 / scale


def _np(t, dtype):
    return np.ascontiguousarray(t.cpu().numpy().astype(dtype))


def _gelu_params(alpha_in: float, alpha_out: float, ch_in: int, ch_out: int, prefix: str, P):
    delta = 0.5  # LUT step in float units: indices -8..7 cover [-4, 3.5]
    lut = np.array([round(255.0 / (1.0 + math.exp(-1.702 * (i - 8) * delta))) for i in range(16)],
                   np.uint8)
    im, is_ = _mul8_shift(1.0 / (alpha_in * delta))
    om, os_ = _mul8_shift(alpha_out / (alpha_in * 255.0))
    P[prefix + ".lut"] = lut
    P[prefix + ".luti_req_multiplier"] = np.full(ch_in, im, np.uint8)
    P[prefix + ".luti_req_shiftmount"] = np.full(ch_in, is_, np.int8)
    P[prefix + ".luto_req_multiplier"] = np.full(ch_out, om, np.uint8)
    P[prefix + ".luto_req_shiftmount"] = np.full(ch_out, os_, np.int8)
    P[prefix + ".de_smooth_vec"] = np.ones(ch_in, np.uint8)


def _linear(W, P, src: str, dst: str, alpha_in: float, alpha_out: float, kind: str,
            has_bias: bool = True):
    w_int, wz, aw = _quant_w_per_channel(W[src + ".weight"])
    P[dst + ".weight"] = _np(w_int, np.int8)
    P[dst + ".wgt_zeros"] = _np(wz, np.int8)
    if has_bias:
        b = torch.round(W[src + ".bias"].double() * alpha_in * aw).clamp(-2**31, 2**31 - 1)
        P[dst + ".bias"] = _np(b, np.int32)
    # vectorised _mulh_shift / _mulh_lshift over the output channels
    r = alpha_out / (alpha_in * aw.cpu().numpy().astype(np.float64))
    f, e = np.frexp(r)
    m = np.round(f * 2.0 ** 32)
    over = m >= 2.0 ** 32
    m = np.where(over, m / 2, m)
    e = e + over.astype(e.dtype)
    if kind == "l8":
        s = -e
        sat = s < 0
        m = np.where(sat, 2.0 ** 32 - 1, m)
        s = np.minimum(np.where(sat, 0, s), 31)
    else:
        neg = e < 0
        m = np.where(neg, np.maximum(1.0, np.round(m * 2.0 ** np.minimum(e, 0))), m)
        s = np.where(neg, 0, np.minimum(e, 31))
    P[dst + ".req_multiplier"] = m.astype(np.uint64).astype(np.uint32)
    P[dst + ".req_shiftmount"] = s.astype(np.int8)


def _layernorm(W, P, p: str, alpha_out: float):
    g = W[p + ".weight"].double()
    ag = 127.0 / max(float(g.abs().max()), 1e-8)
    P[p + ".weight"] = _np(torch.round(g * ag).clamp(-127, 127), np.int8)
    P[p + ".bias"] = _np(torch.round(W[p + ".bias"].double() * 2048 * ag), np.int32)
    # int15 stage holds z * 2^11: ln_m * 2^(13 - ln_s) = 2^11
    P[p + ".ln_req_multiplier"] = np.array([128], np.uint8)
    P[p + ".ln_req_shiftmount"] = np.array([9], np.int8)
    m, s = _mulh_shift(alpha_out / (2048 * ag))
    P[p + ".out_req_multiplier"] = np.array([m], np.uint32)
    P[p + ".out_req_shiftmount"] = np.array([s], np.int8)


def _attention(W, P, st, p: str, n_head: int, alpha_in: float, alpha_kv_in: float, x_alpha_in: float,
               x_alpha_out: float):
    aq, ak, av = _alpha(st, p + ".q"), _alpha(st, p + ".k"), _alpha(st, p + ".v")
    ao = _alpha(st, p + ".wv")
    _linear(W, P, p + ".query", p + ".query", alpha_in, aq, "l8")
    _linear(W, P, p + ".key", p + ".key", alpha_kv_in, ak, "l8", has_bias=False)
    _linear(W, P, p + ".value", p + ".value", alpha_kv_in, av, "l8")
    _linear(W, P, p + ".out", p + ".out", ao, x_alpha_out * 32768.0, "l32")
    C = W[p + ".query.weight"].shape[0]
    D = C // n_head
    max_logit = st.v[p + ".qk"]
    f = int(min(max(15 - math.ceil(math.log2(max_logit + 1.0)), 1), 13))
    qm, qs = _mul8_shift((2.0 ** f) / (math.sqrt(D) * aq * ak), trunc=True)
    am, as_ = _mul8_shift(ao / av, trunc=True)
    P[p + ".qk_req_multiplier"] = np.array([qm], np.uint8)
    P[p + ".qk_req_shiftmount"] = np.array([qs], np.int8)
    P[p + ".av_req_multiplier"] = np.array([am], np.uint8)
    P[p + ".av_req_shiftmount"] = np.array([as_], np.int8)
    P[p + ".qk_frac_bits"] = np.array(f, np.int32)


def _res_mult(a_new: float, a_old: float) -> int:
    return int(min(max(round(32768.0 * a_new / a_old), 1), 65535))


def _blocks(W, P, st, prefix: str, n_layer: int, n_head: int, x_alpha: float, cross: bool,
            xa_alpha: Optional[float]):
    for i in range(n_layer):
        p = f"{prefix}.blocks.{i}"
        a_in = x_alpha
        a_mid = min(16383.0 / st.v[p + ".mid"], a_in)
        a_ln = _alpha(st, p + ".attn_ln.out")
        _layernorm(W, P, p + ".attn_ln", a_ln)
        _attention(W, P, st, p + ".attn", n_head, a_ln, a_ln, a_in, a_mid)
        P[p + ".attn_res_req_multiplier"] = np.array([_res_mult(a_mid, a_in)], np.uint16)
        a_cur = a_mid
        if cross:
            a_mid2 = min(16383.0 / st.v[p + ".mid2"], a_cur)
            a_cln = _alpha(st, p + ".cross_attn_ln.out")
            _layernorm(W, P, p + ".cross_attn_ln", a_cln)
            _attention(W, P, st, p + ".cross_attn", n_head, a_cln, xa_alpha, a_cur, a_mid2)
            P[p + ".cross_attn_res_req_multiplier"] = np.array([_res_mult(a_mid2, a_cur)], np.uint16)
            a_cur = a_mid2
        else:
            P[p + ".cross_attn_res_req_multiplier"] = np.array([1], np.uint16)
        a_out = min(16383.0 / st.v[p + ".out"], a_cur)
        a_mln = _alpha(st, p + ".mlp_ln.out")
        a_fc1 = _alpha(st, p + ".fc1")
        a_gelu = _alpha(st, p + ".gelu")
        _layernorm(W, P, p + ".mlp_ln", a_mln)
        _linear(W, P, p + ".mlp.0", p + ".mlp.0", a_mln, a_fc1, "l8")
        n_mlp = W[p + ".mlp.0.weight"].shape[0]
        _gelu_params(a_fc1, a_gelu, n_mlp, n_mlp, p + ".mlp.1", P)
        _linear(W, P, p + ".mlp.2", p + ".mlp.2", a_gelu, a_out * 32768.0, "l32")
        P[p + ".mlp_res_req_multiplier"] = np.array([_res_mult(a_out, a_cur)], np.uint16)
        x_alpha = a_out
    return x_alpha


def calibrated_int_params(dims: ModelDimensions, seed: int = 0, n_calib: int = 8,
                          calib_ctx: Optional[int] = None, calib_tokens: int = 16,
                          verbose: bool = False, decoder_mlp_scale: float = 1.0) -> Dict[str, np.ndarray]:
    """Integer parameters of ``Whisper_int`` (reference state-dict keys and dtypes),
    calibrated on ``n_calib`` seeded mels of 2 * min(n_audio_ctx, calib_ctx or 300)
    frames."""
    torch_threads = torch.get_num_threads()
    W = float_weights(dims, seed, decoder_mlp_scale)
    ctx = min(dims.n_audio_ctx, calib_ctx or 300)
    mels = torch.from_numpy(synthetic_mel(n_calib, dims.n_mels, 2 * ctx, seed + 1))
    toks = np.concatenate([prompt_tokens(n_calib, dims.n_vocab),
                           np.random.default_rng(seed + 2).integers(
                               0, dims.n_vocab, size=(n_calib, max(calib_tokens - 3, 0)))], 1)
    toks = torch.from_numpy(toks[:, :min(calib_tokens, dims.n_text_ctx)])
    st = _calibrate(dims, W, mels, toks)
    if verbose:
        print(f"calibrated on {n_calib} mels x {2 * ctx} frames ({torch_threads} threads)")
    P: Dict[str, np.ndarray] = {}
    d = dims.n_audio_state
    # --- encoder front end ---
    a_mel = _alpha(st, "encoder.mel")
    P["encoder.input_alpha"] = np.array([a_mel], np.float32)
    a_c1, a_g1 = _alpha(st, "encoder.conv1"), _alpha(st, "encoder.gelu1")
    a_c2, a_g2 = _alpha(st, "encoder.conv2"), _alpha(st, "encoder.gelu2")
    for name, a_in, a_out in (("conv1", a_mel, a_c1), ("conv2", a_g1, a_c2)):
        w = W[f"encoder.{name}.weight"]
        aw = 127.0 / float(w.abs().max())
        # weight flattened [Cout, Cin*K] with the kernel index fastest (model_int.py:559-561)
        P[f"encoder.{name}.weight"] = _np(torch.round(w.double() * aw).clamp(-127, 127)
                                          .reshape(w.shape[0], -1), np.int8)
        P[f"encoder.{name}.bias"] = _np(torch.round(W[f"encoder.{name}.bias"].double() * a_in * aw),
                                        np.int32)
        m, s = _mulh_shift(a_out / (a_in * aw))
        P[f"encoder.{name}.req_multiplier"] = np.array([m], np.uint32)
        P[f"encoder.{name}.req_shiftmount"] = np.array([s], np.int8)
    _gelu_params(a_c1, a_g1, 1, 1, "encoder.gelu1", P)
    _gelu_params(a_c2, a_g2, 1, d, "encoder.gelu2", P)
    pe = W["encoder.positional_embedding"].double()
    P["encoder.positional_embedding"] = _np(torch.round(pe * a_g2).clamp(-127, 127), np.int8)
    x0max = max(st.v["encoder.blocks.0.in"] if dims.n_audio_layer else st.v["encoder.gelu2"], 1e-8)
    a_x = 16383.0 / x0max
    m16, s16 = _mul16_shift(a_x / a_g2)
    P["encoder.req_multiplier"] = np.full(d, m16, np.uint16)
    P["encoder.req_shiftmount"] = np.full(d, s16, np.int8)
    a_x = _blocks(W, P, st, "encoder", dims.n_audio_layer, dims.n_audio_head, a_x, False, None)
    a_enc = _alpha(st, "encoder.ln_post.out")
    _layernorm(W, P, "encoder.ln_post", a_enc)
    # --- decoder ---
    E = W["decoder.token_embedding.weight"].double()
    aE = 127.0 / float(E.abs().max())
    P["decoder.token_embedding.weight"] = _np(torch.round(E * aE).clamp(-127, 127), np.int8)
    P["decoder.positional_embedding"] = _np(
        torch.round(W["decoder.positional_embedding"].double() * aE).clamp(-127, 127), np.int8)
    y0max = st.v["decoder.blocks.0.in"] if dims.n_text_layer else 1.0
    a_y = 16383.0 / y0max
    m8, s8 = _mul8_shift(a_y / aE)
    P["decoder.req_multiplier"] = np.array([m8], np.uint8)
    P["decoder.req_shiftmount"] = np.array([s8], np.int8)
    _blocks(W, P, st, "decoder", dims.n_text_layer, dims.n_text_head, a_y, True, a_enc)
    a_dln = _alpha(st, "decoder.ln.out")
    _layernorm(W, P, "decoder.ln", a_dln)
    a_logit = _alpha(st, "decoder.logits")
    cm, cs = _mulh_shift(a_logit / (a_dln * aE))
    P["decoder.clf_req_multiplier"] = np.array([cm], np.uint32)
    P["decoder.clf_req_shiftmount"] = np.array([cs], np.int8)
    P["decoder.act_logits_alpha"] = np.array([a_logit], np.float32)
    return P


def param_bytes(params: Dict[str, np.ndarray]) -> int:
    return int(sum(v.nbytes for v in params.values()))


def shapes_of(params: Dict[str, np.ndarray]) -> Dict[str, Sequence[int]]:
    return {k: tuple(v.shape) for k, v in params.items()}
