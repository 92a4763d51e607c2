"""Synthetic inputs and a synthetic integer checkpoint for the benchmark workloads.

* ``synthetic_mel``: seeded 30 s log-mel, values ~ N(-0.5, 0.4) clipped to
  [-1.5, 1.5], float32 [B, n_mels, frames].
* ``calibrated_int_params``: random-init float Whisper weights, a float
  calibration run on seeded full-length synthetic mels (the encoder, then a
  greedy decode from the start prompt, as quantize.py:395-407 calibrates with
  ``decode`` on padded 30 s audio), then conversion to the integer parameters
  of ``Whisper_int`` (reference state-dict names and dtypes).

The conversion follows the integer forms of the reference's offline quantiser
(i_whisper/model_quant.py), parameter by parameter:

* Linear8 and Conv1d requant: ``frexp`` mantissa x 2^31 truncated, shift
  ``-e - 1`` clamped to [0, 32] (model_quant.py:637-642, 907-913); the
  out-projections and FC2 (Linear32): the same multiplier, left shift ``e``
  clamped to [0, 32], targeting the next LayerNorm's input scale x 2^16
  (model_quant.py:638-640, 1184, 1512-1527);
* LayerNorm: input scale 16383 / max|x| (the int16 residual stream),
  ``ln_req`` = mantissa x 2^7 rounded with shift ``-e + 7 + 13``, gamma per
  tensor to int8, beta at ``ln_alpha * wgt_alpha``, output requant mantissa
  x 2^31 rounded with shift ``-e - 1`` (model_quant.py:357-394, 400-420);
* residual15 multipliers ``round(alpha_next * 2^15 / alpha_prev)`` clamped
  to uint16 (model_quant.py:1534-1545);
* attention ``qk_frac_bits = 15 - (floor(log2 max|qk|) + 1)`` and the qk / av
  multipliers as mantissa x 2^7 truncated, shift ``-e + 7``
  (model_quant.py:1186-1198, 1318-1343);
* GeLU: the 16-entry sigmoid table over [-6, 6) in steps of 0.75 with the
  ends pinned to 0 and 255, luti / luto as mantissa x 2^7 rounded, shift
  ``-e + 7`` (model_quant.py:107-122, 170-190); the input step is scaled by
  1.702 so that the table approximates x * sigmoid(1.702 x), the float
  model's GeLU;
* encoder input requant: mantissa x 2^15 rounded, shift ``-e + 15``; decoder
  embedding requant: mantissa x 2^7 rounded, shift ``-e + 7``
  (model_quant.py:1838-1842, 2089-2093); classifier: mantissa x 2^31 rounded,
  shift ``-e - 1`` clamped to [0, 31] (model_quant.py:2029-2033);
* Linear weights per output channel, asymmetric: alpha = 254 / (max - min),
  zero point ``trunc(-(max + min) / 2 * alpha)`` (model_quant.py:670-735,
  without the reference's +-1e-4 range search); biases at
  ``wgt_alpha * act_alpha``.

So every Linear / conv multiplier lies in [2^30, 2^31) and every rounded
31-bit multiplier in [2^30, 2^31]: the range a reference checkpoint holds.

The random weights are shaped so that greedy decoding follows its input
instead of repeating one token (``shaped``): with plain N(0, 0.02) weights every
block adds a large input-independent vector (its biases, the mean of the GeLU
output through FC2, attention that averages its keys almost uniformly), which
builds up over the layers until it alone decides the argmax. Shaping scales
every block's biases by 0.1, centres each FC2 row, scales the out-projections
and FC2 by 1 / sqrt(2 * layers) (the scaled residual initialisation of GPT-2),
and in the decoder scales the self- and cross-attention query and key weights
by 4 (a selective softmax) and the positional embedding by 4. Shapes, dtypes
and the work per step are unchanged.
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
# float model (float32, on the GPU when there is one) used for calibration only
# ---------------------------------------------------------------------------

def _sinusoids(length: int, channels: int, max_timescale: float = 10000.0) -> torch.Tensor:
    inc = math.log(max_timescale) / (channels // 2 - 1)
    inv = torch.exp(-inc * torch.arange(channels // 2))
    t = torch.arange(length)[:, None] * inv[None, :]
    return torch.cat([torch.sin(t), torch.cos(t)], dim=1)


class _Gen:
    def __init__(self, seed: int):
        self.r = np.random.default_rng(seed)

    def normal(self, *shape, std=0.02, mean=0.0):
        a = self.r.standard_normal(shape, dtype=np.float32)
        a *= np.float32(std)
        if mean:
            a += np.float32(mean)
        return torch.from_numpy(a)


def float_weights(dims: ModelDimensions, seed: int, decoder_mlp_scale: float = 1.0,
                  shaped: bool = True) -> Dict[str, torch.Tensor]:
    """Random-init float weights: N(0, 0.02) for every linear / conv / embedding
    weight and bias, LayerNorm gamma ~ N(1, 0.1) and beta ~ N(0, 0.02),
    sinusoidal encoder positions. ``decoder_mlp_scale`` scales the decoder
    MLPs' output weights and FC1 biases; ``shaped`` applies the shaping
    described in the module docstring."""
    g = _Gen(seed)
    W: Dict[str, torch.Tensor] = {}
    d, dt = dims.n_audio_state, dims.n_text_state
    W["encoder.conv1.weight"] = g.normal(d, dims.n_mels, 3)
    W["encoder.conv1.bias"] = g.normal(d)
    W["encoder.conv2.weight"] = g.normal(d, d, 3)
    W["encoder.conv2.bias"] = g.normal(d)
    W["encoder.positional_embedding"] = _sinusoids(dims.n_audio_ctx, d)

    def ln(p, n):
        W[f"{p}.weight"] = g.normal(n, std=0.1, mean=1.0)
        W[f"{p}.bias"] = g.normal(n)

    def block(p, n, cross, n_layer):
        for name in ["attn_ln", "mlp_ln"] + (["cross_attn_ln"] if cross else []):
            ln(f"{p}.{name}", n)
        attns = ["attn"] + (["cross_attn"] if cross else [])
        for a in attns:
            for lin in ("query", "key", "value", "out"):
                W[f"{p}.{a}.{lin}.weight"] = g.normal(n, n)
                if lin != "key":
                    W[f"{p}.{a}.{lin}.bias"] = g.normal(n)
        W[f"{p}.mlp.0.weight"] = g.normal(4 * n, n)
        W[f"{p}.mlp.0.bias"] = g.normal(4 * n)
        W[f"{p}.mlp.2.weight"] = g.normal(n, 4 * n)
        W[f"{p}.mlp.2.bias"] = g.normal(n)
        if not shaped:
            return
        for k in [k for k in W if k.startswith(p + ".") and k.endswith(".bias") and "_ln." not in k]:
            W[k] *= 0.1
        w2 = W[f"{p}.mlp.2.weight"]
        W[f"{p}.mlp.2.weight"] = w2 - w2.mean(1, keepdim=True)
        res = 1.0 / math.sqrt(2.0 * n_layer)
        for k in [f"{a}.out.weight" for a in attns] + ["mlp.2.weight"]:
            W[f"{p}.{k}"] *= res
        if cross:
            for a in attns:
                W[f"{p}.{a}.query.weight"] *= 4.0
                W[f"{p}.{a}.key.weight"] *= 4.0

    for i in range(dims.n_audio_layer):
        block(f"encoder.blocks.{i}", d, False, dims.n_audio_layer)
    ln("encoder.ln_post", d)
    W["decoder.token_embedding.weight"] = g.normal(dims.n_vocab, dt)
    W["decoder.positional_embedding"] = g.normal(dims.n_text_ctx, dt)
    if shaped:
        W["decoder.positional_embedding"] *= 4.0
    for i in range(dims.n_text_layer):
        p = f"decoder.blocks.{i}"
        block(p, dt, True, dims.n_text_layer)
        if decoder_mlp_scale != 1.0:
            for k in ("mlp.0.bias", "mlp.2.weight", "mlp.2.bias"):
                W[f"{p}.{k}"] *= decoder_mlp_scale
    ln("decoder.ln", dt)
    return W


class _Stats:
    """max |x| of every calibration point (over all calibration steps)."""

    def __init__(self):
        self.v: Dict[str, float] = {}

    def __call__(self, name: str, t: torch.Tensor) -> torch.Tensor:
        m = float(t.detach().abs().max())
        self.v[name] = max(self.v.get(name, 0.0), m, 1e-8)
        return t

    def __getitem__(self, name: str) -> float:
        return self.v[name]


def _gelu(x):
    return x * torch.sigmoid(1.702 * x)


def _ln(x, W, p, st: _Stats):
    """LayerNorm recording its input, normalised and output maxima."""
    st(p + ".x", x)
    mean = x.mean(-1, keepdim=True)
    z = (x - mean) * torch.rsqrt(((x - mean) ** 2).mean(-1, keepdim=True) + 1e-5)
    st(p + ".norm", z)
    return st(p + ".out", z * W[p + ".weight"] + W[p + ".bias"])


def _heads(t, n_head):
    B, T, C = t.shape
    return t.view(B, T, n_head, C // n_head).transpose(1, 2).contiguous()


def _attn(x, W, p, n_head, st: _Stats, kv=None, cache=None):
    """Multi-head attention of queries ``x``. Self-attention when ``kv`` is None:
    the new keys / values are appended to ``cache`` (a dict) and the queries
    see the cached positions and the causal part of their own block.
    Cross-attention: ``kv`` = the precomputed (k, v) heads of the audio."""
    q = st(p + ".q", x @ W[p + ".query.weight"].T + W[p + ".query.bias"])
    qh = _heads(q, n_head)
    T = x.shape[1]
    if kv is None:
        k = st(p + ".k", x @ W[p + ".key.weight"].T)
        v = st(p + ".v", x @ W[p + ".value.weight"].T + W[p + ".value.bias"])
        kh, vh = _heads(k, n_head), _heads(v, n_head)
        if cache is not None:
            if "k" in cache:
                kh = torch.cat([cache["k"], kh], 2)
                vh = torch.cat([cache["v"], vh], 2)
            cache["k"], cache["v"] = kh, vh
        causal = True
    else:
        kh, vh = kv
        causal = False
    D = qh.shape[-1]
    logits = (qh @ kh.transpose(-1, -2).contiguous()) / math.sqrt(D)
    st(p + ".qk", logits)
    if causal and T > 1:
        Tk = kh.shape[2]
        mask = torch.ones(T, Tk, dtype=torch.bool, device=x.device).triu(1 + Tk - T)
        logits = logits.masked_fill(mask, float("-inf"))
    o = (torch.softmax(logits, -1) @ vh).transpose(1, 2).reshape(x.shape[0], T, -1)
    st(p + ".wv", o)
    return o @ W[p + ".out.weight"].T + W[p + ".out.bias"]


def _cross_kv(xa, W, p, n_head, st: _Stats):
    k = st(p + ".k", xa @ W[p + ".key.weight"].T)
    v = st(p + ".v", xa @ W[p + ".value.weight"].T + W[p + ".value.bias"])
    return _heads(k, n_head), _heads(v, n_head)


def _mlp(x, W, p, st: _Stats):
    h = _ln(x, W, p + ".mlp_ln", st)
    h = st(p + ".fc1", h @ W[p + ".mlp.0.weight"].T + W[p + ".mlp.0.bias"])
    h = st(p + ".gelu", _gelu(h))
    return x + h @ W[p + ".mlp.2.weight"].T + W[p + ".mlp.2.bias"]


def _encoder(dims: ModelDimensions, W, mels: torch.Tensor, st: _Stats) -> torch.Tensor:
    st("encoder.mel", mels)
    c1 = st("encoder.conv1", torch.nn.functional.conv1d(mels, W["encoder.conv1.weight"],
                                                        W["encoder.conv1.bias"], padding=1))
    g1 = st("encoder.gelu1", _gelu(c1))
    c2 = st("encoder.conv2", torch.nn.functional.conv1d(g1, W["encoder.conv2.weight"], W["encoder.conv2.bias"],
                                                        stride=2, padding=1))
    x = st("encoder.gelu2", _gelu(c2)).permute(0, 2, 1)
    x = x + W["encoder.positional_embedding"][:x.shape[1]]
    for i in range(dims.n_audio_layer):
        p = f"encoder.blocks.{i}"
        x = x + _attn(_ln(x, W, p + ".attn_ln", st), W, p + ".attn", dims.n_audio_head, st)
        x = _mlp(x, W, p, st)
    return _ln(x, W, "encoder.ln_post", st)


def _greedy_calibration(dims: ModelDimensions, W, xa: torch.Tensor, prompt: torch.Tensor, steps: int,
                        st: _Stats) -> torch.Tensor:
    """Greedy decoding over a key/value cache (decoding.py:684-712 without the
    logit filters), every step recorded in ``st``. Returns the tokens."""
    L, H = dims.n_text_layer, dims.n_text_head
    cross = [_cross_kv(xa, W, f"decoder.blocks.{i}.cross_attn", H, st) for i in range(L)]
    caches = [dict() for _ in range(L)]
    E = W["decoder.token_embedding.weight"]
    tokens, new, offset = prompt, prompt, 0
    for _ in range(max(steps, 1)):  # the decoding loop's sample_len forwards
        T = new.shape[1]
        y = E[new] + W["decoder.positional_embedding"][offset:offset + T]
        for i in range(L):
            p = f"decoder.blocks.{i}"
            y = y + _attn(_ln(y, W, p + ".attn_ln", st), W, p + ".attn", H, st, cache=caches[i])
            y = y + _attn(_ln(y, W, p + ".cross_attn_ln", st), W, p + ".cross_attn", H, st, kv=cross[i])
            y = _mlp(y, W, p, st)
        logits = st("decoder.logits", _ln(y, W, "decoder.ln", st) @ E.T)
        offset += T
        new = logits[:, -1].argmax(-1, keepdim=True)
        tokens = torch.cat([tokens, new], 1)
    return tokens


# ---------------------------------------------------------------------------
# float -> integer conversion, in the reference quantiser's parameter forms
# ---------------------------------------------------------------------------

def _frexp(r):
    f, e = np.frexp(np.asarray(r, np.float64))
    return f, e.astype(np.int64)


def _req_l8(r):
    """Linear8 / Conv1d: trunc(f * 2^31), right shift -e - 1 in [0, 32]."""
    f, e = _frexp(r)
    return np.trunc(f * 2.0 ** 31).astype(np.uint32), np.clip(-e - 1, 0, 32).astype(np.int8)


def _req_out(r):
    """Linear32 (out-projection, FC2): trunc(f * 2^31), left shift e in [0, 32]."""
    f, e = _frexp(r)
    return np.trunc(f * 2.0 ** 31).astype(np.uint32), np.clip(e, 0, 32).astype(np.int8)


def _req_round31(r, smax: int):
    """LayerNorm output / classifier: round(f * 2^31), right shift -e - 1 in [0, smax]."""
    f, e = _frexp(r)
    m = np.clip(np.round(f * 2.0 ** 31), 0, 2.0 ** 32 - 1)
    return m.astype(np.uint32), np.clip(-e - 1, 0, smax).astype(np.int8)


def _req_u8(r, trunc: bool, extra: int = 0, smax: int = 32):
    """uint8 multiplier f * 2^7 (truncated or rounded), shift -e + 7 + extra."""
    f, e = _frexp(r)
    m = np.trunc(f * 128.0) if trunc else np.round(f * 128.0)
    return np.clip(m, 0, 255).astype(np.uint8), np.clip(-e + 7 + extra, 0, smax).astype(np.int8)


def _req_u16(r):
    """uint16 multiplier round(f * 2^15), shift -e + 15 in [0, 31]."""
    f, e = _frexp(r)
    return np.clip(np.round(f * 32768.0), 0, 65535).astype(np.uint16), np.clip(-e + 15, 0, 31).astype(np.int8)


def _a8(st: _Stats, name: str) -> float:
    """int8 activation scale 127 / max|x|."""
    return 127.0 / st[name]


def _a15(st: _Stats, ln: str) -> float:
    """int16 residual-stream scale at a LayerNorm's input: 16383 / max|x|."""
    return 16383.0 / st[ln + ".x"]


def _np(t, dtype):
    return np.ascontiguousarray(t.detach().cpu().numpy().astype(dtype))


def _quant_w_per_channel(w: torch.Tensor):
    """Asymmetric per-output-channel int8 (model_quant.py:670-735 without the
    range search): alpha = 254 / (max - min), zero = trunc(-(max + min) / 2 *
    alpha), w_int = round(w * alpha + zero) in [-127, 127]."""
    w = w.reshape(w.shape[0], -1).double().cpu()
    hi, lo = w.max(1).values, w.min(1).values
    alpha = 254.0 / (hi - lo).clamp_min(1e-12)
    zero = torch.trunc(-(hi + lo) / 2.0 * alpha)
    w_int = torch.round(w * alpha[:, None] + zero[:, None]).clamp(-127, 127)
    return w_int.to(torch.int8), zero.to(torch.int8), alpha.numpy()


GELU_LUT_STEP = 0.75  # model_quant.py:114-119: 16 entries over [-6, 6)


def _gelu_params(alpha_in: float, alpha_out: float, ch_in: int, ch_out: int, prefix: str, P):
    lut = np.round(1.0 / (1.0 + np.exp(-np.arange(-6.0, 6.0, GELU_LUT_STEP))) * 255.0)
    lut[0], lut[-1] = 0, 255
    im, is_ = _req_u8(1.702 / (alpha_in * GELU_LUT_STEP), trunc=False)
    om, os_ = _req_u8(alpha_out / (alpha_in * 255.0), trunc=False)
    P[prefix + ".lut"] = lut.astype(np.uint8)
    P[prefix + ".luti_req_multiplier"] = np.full(ch_in, im, np.uint8)
    P[prefix + ".luti_req_shiftmount"] = np.full(ch_in, is_, np.int8)
    P[prefix + ".luto_req_multiplier"] = np.full(ch_out, om, np.uint8)
    P[prefix + ".luto_req_shiftmount"] = np.full(ch_out, os_, np.int8)
    P[prefix + ".de_smooth_vec"] = np.ones(ch_in, np.uint8)


def _linear(W, P, src: str, dst: str, alpha_in: float, alpha_out: float, kind: str, has_bias: bool = True):
    w_int, wz, aw = _quant_w_per_channel(W[src + ".weight"])
    P[dst + ".weight"] = _np(w_int, np.int8)
    P[dst + ".wgt_zeros"] = _np(wz, np.int8)
    if has_bias:
        b = np.round(W[src + ".bias"].double().cpu().numpy() * aw * alpha_in)
        P[dst + ".bias"] = np.clip(b, -2.0 ** 31, 2.0 ** 31 - 1).astype(np.int32)
    r = alpha_out / (aw * alpha_in)
    m, s = _req_l8(r) if kind == "l8" else _req_out(r)
    P[dst + ".req_multiplier"] = m
    P[dst + ".req_shiftmount"] = s


def _layernorm(W, P, st: _Stats, p: str, alpha_out: float):
    ln_alpha = 16383.0 / st[p + ".norm"]
    g = W[p + ".weight"].double().cpu()
    ag = 127.0 / max(float(g.abs().max()), 1e-8)
    P[p + ".weight"] = _np(torch.round(g * ag).clamp(-127, 127), np.int8)
    b = torch.round(W[p + ".bias"].double().cpu() * ln_alpha * ag).clamp(-(2.0 ** 30 - 1), 2.0 ** 30 - 1)
    P[p + ".bias"] = _np(b, np.int32)
    m, s = _req_u8(ln_alpha, trunc=False, extra=13, smax=31)
    P[p + ".ln_req_multiplier"] = m.reshape(1)
    P[p + ".ln_req_shiftmount"] = s.reshape(1)
    m, s = _req_round31(alpha_out / (ln_alpha * ag), 32)
    P[p + ".out_req_multiplier"] = m.reshape(1)
    P[p + ".out_req_shiftmount"] = s.reshape(1)


def _attention(W, P, st: _Stats, p: str, n_head: int, alpha_in: float, alpha_kv_in: float, alpha_next: float):
    aq, ak, av, ao = _a8(st, p + ".q"), _a8(st, p + ".k"), _a8(st, p + ".v"), _a8(st, p + ".wv")
    _linear(W, P, p + ".query", p + ".query", alpha_in, aq, "l8")
    _linear(W, P, p + ".key", p + ".key", alpha_kv_in, ak, "l8", has_bias=False)
    _linear(W, P, p + ".value", p + ".value", alpha_kv_in, av, "l8")
    _linear(W, P, p + ".out", p + ".out", ao, alpha_next * 65536.0, "l32")
    D = W[p + ".query.weight"].shape[0] // n_head
    f = int(np.clip(15 - (math.floor(math.log2(st[p + ".qk"])) + 1), 1, 13))
    qm, qs = _req_u8((2.0 ** f) / (math.sqrt(D) * aq * ak), trunc=True)
    am, as_ = _req_u8(ao / av, trunc=True)
    P[p + ".qk_req_multiplier"] = qm.reshape(1)
    P[p + ".qk_req_shiftmount"] = qs.reshape(1)
    P[p + ".av_req_multiplier"] = am.reshape(1)
    P[p + ".av_req_shiftmount"] = as_.reshape(1)
    P[p + ".qk_frac_bits"] = np.array(f, np.int32)


def _res_mult(a_next: float, a_prev: float) -> np.ndarray:
    return np.array([min(max(round(a_next * 32768.0 / a_prev), 0), 65535)], np.uint16)


def _blocks(W, P, st: _Stats, prefix: str, n_layer: int, n_head: int, final_ln: str, cross: bool,
            xa_alpha: Optional[float]):
    for i in range(n_layer):
        p = f"{prefix}.blocks.{i}"
        nxt = f"{prefix}.blocks.{i + 1}.attn_ln" if i + 1 < n_layer else final_ln
        a_in = _a15(st, p + ".attn_ln")
        a_mid = _a15(st, p + (".cross_attn_ln" if cross else ".mlp_ln"))
        a_ln = _a8(st, p + ".attn_ln.out")
        _layernorm(W, P, st, p + ".attn_ln", a_ln)
        _attention(W, P, st, p + ".attn", n_head, a_ln, a_ln, a_mid)
        P[p + ".attn_res_req_multiplier"] = _res_mult(a_mid, a_in)
        a_cur = a_mid
        if cross:
            a_mid2 = _a15(st, p + ".mlp_ln")
            a_cln = _a8(st, p + ".cross_attn_ln.out")
            _layernorm(W, P, st, p + ".cross_attn_ln", a_cln)
            _attention(W, P, st, p + ".cross_attn", n_head, a_cln, xa_alpha, a_mid2)
            P[p + ".cross_attn_res_req_multiplier"] = _res_mult(a_mid2, a_cur)
            a_cur = a_mid2
        else:
            P[p + ".cross_attn_res_req_multiplier"] = np.array([1], np.uint16)
        a_out = _a15(st, nxt)
        a_mln, a_fc1, a_gelu = _a8(st, p + ".mlp_ln.out"), _a8(st, p + ".fc1"), _a8(st, p + ".gelu")
        _layernorm(W, P, st, p + ".mlp_ln", a_mln)
        _linear(W, P, p + ".mlp.0", p + ".mlp.0", a_mln, a_fc1, "l8")
        n_mlp = W[p + ".mlp.0.weight"].shape[0]
        _gelu_params(a_fc1, a_gelu, n_mlp, n_mlp, p + ".mlp.1", P)
        _linear(W, P, p + ".mlp.2", p + ".mlp.2", a_gelu, a_out * 65536.0, "l32")
        P[p + ".mlp_res_req_multiplier"] = _res_mult(a_out, a_cur)


def _device(device):
    if device is not None:
        return torch.device(device)
    return torch.device("cuda") if torch.cuda.is_available() else torch.device("cpu")


def calibrated_int_params(dims: ModelDimensions, seed: int = 0, n_calib: int = 8,
                          calib_ctx: Optional[int] = None, calib_tokens: Optional[int] = None,
                          verbose: bool = False, decoder_mlp_scale: float = 1.0,
                          shaped: bool = True, device=None) -> Dict[str, np.ndarray]:
    """Integer parameters of ``Whisper_int`` (reference state-dict keys and dtypes).

    Calibration: ``n_calib`` seeded mels of 2 * min(n_audio_ctx, calib_ctx)
    frames (default: the full 30 s), the encoder, then ``calib_tokens``
    greedy steps (default n_text_ctx // 2, the reference decoder's default
    sample length) from the start prompt. The float model runs on the GPU
    when there is one (``device``), otherwise on the CPU."""
    dev = _device(device)
    W = {k: v.to(dev) for k, v in float_weights(dims, seed, decoder_mlp_scale, shaped).items()}
    ctx = min(dims.n_audio_ctx, calib_ctx or dims.n_audio_ctx)
    steps = calib_tokens if calib_tokens is not None else dims.n_text_ctx // 2
    steps = max(0, min(steps, dims.n_text_ctx - len(PROMPT)))
    st = _Stats()
    with torch.no_grad():
        mels = torch.from_numpy(synthetic_mel(n_calib, dims.n_mels, 2 * ctx, seed + 1)).to(dev)
        xa = _encoder(dims, W, mels, st)
        prompt = torch.from_numpy(prompt_tokens(n_calib, dims.n_vocab)).to(dev)
        toks = _greedy_calibration(dims, W, xa, prompt, steps, st)
    if verbose:
        print(f"calibrated on {n_calib} mels x {2 * ctx} frames + {steps} greedy steps on {dev}; "
              f"row 0 tokens {toks[0, 3:11].tolist()} ...")
    del xa, mels
    P: Dict[str, np.ndarray] = {}
    d = dims.n_audio_state
    # --- encoder front end ---
    a_mel = _a8(st, "encoder.mel")
    P["encoder.input_alpha"] = np.array([a_mel], np.float32)
    a_c1, a_g1, a_c2 = _a8(st, "encoder.conv1"), _a8(st, "encoder.gelu1"), _a8(st, "encoder.conv2")
    pe = W["encoder.positional_embedding"].double().cpu()
    a_g2 = min(_a8(st, "encoder.gelu2"), 127.0 / max(float(pe.abs().max()), 1e-8))
    for name, a_in, a_out in (("conv1", a_mel, a_c1), ("conv2", a_g1, a_c2)):
        w = W[f"encoder.{name}.weight"].double().cpu()
        aw = 127.0 / float(w.abs().max())
        # weight flattened [Cout, Cin*K] with the kernel index fastest (model_int.py:559-561)
        P[f"encoder.{name}.weight"] = _np(torch.round(w * aw).clamp(-127, 127).reshape(w.shape[0], -1), np.int8)
        P[f"encoder.{name}.bias"] = _np(torch.round(W[f"encoder.{name}.bias"].double().cpu() * a_in * aw),
                                        np.int32)
        m, s = _req_l8(a_out / (a_in * aw))
        P[f"encoder.{name}.req_multiplier"] = m.reshape(1)
        P[f"encoder.{name}.req_shiftmount"] = s.reshape(1)
    _gelu_params(a_c1, a_g1, 1, 1, "encoder.gelu1", P)
    _gelu_params(a_c2, a_g2, 1, d, "encoder.gelu2", P)
    P["encoder.positional_embedding"] = _np(torch.round(pe * a_g2).clamp(-127, 127), np.int8)
    first = "encoder.blocks.0.attn_ln" if dims.n_audio_layer else "encoder.ln_post"
    m16, s16 = _req_u16(_a15(st, first) / a_g2)
    P["encoder.req_multiplier"] = np.full(d, m16, np.uint16)
    P["encoder.req_shiftmount"] = np.full(d, s16, np.int8)
    _blocks(W, P, st, "encoder", dims.n_audio_layer, dims.n_audio_head, "encoder.ln_post", False, None)
    a_enc = _a8(st, "encoder.ln_post.out")
    _layernorm(W, P, st, "encoder.ln_post", a_enc)
    # --- decoder ---
    E = W["decoder.token_embedding.weight"].double().cpu()
    Pd = W["decoder.positional_embedding"].double().cpu()
    # one scale for both tables: the embedding sum is formed in int8 units (model_int.py:1411-1421)
    aE = 127.0 / max(float(E.abs().max()), float(Pd.abs().max()))
    P["decoder.token_embedding.weight"] = _np(torch.round(E * aE).clamp(-127, 127), np.int8)
    P["decoder.positional_embedding"] = _np(torch.round(Pd * aE).clamp(-127, 127), np.int8)
    first = "decoder.blocks.0.attn_ln" if dims.n_text_layer else "decoder.ln"
    m8, s8 = _req_u8(_a15(st, first) / aE, trunc=False, smax=31)
    P["decoder.req_multiplier"] = m8.reshape(1)
    P["decoder.req_shiftmount"] = s8.reshape(1)
    _blocks(W, P, st, "decoder", dims.n_text_layer, dims.n_text_head, "decoder.ln", True, a_enc)
    a_cf = _a8(st, "decoder.ln.out")
    _layernorm(W, P, st, "decoder.ln", a_cf)
    a_logit = _a8(st, "decoder.logits")
    cm, cs = _req_round31(a_logit / (aE * a_cf), 31)
    P["decoder.clf_req_multiplier"] = cm.reshape(1)
    P["decoder.clf_req_shiftmount"] = cs.reshape(1)
    P["decoder.act_logits_alpha"] = np.array([a_logit], np.float32)
    del W
    if dev.type == "cuda":
        torch.cuda.empty_cache()
    return P


def param_bytes(params: Dict[str, np.ndarray]) -> int:
    return int(sum(v.nbytes for v in params.values()))


def shapes_of(params: Dict[str, np.ndarray]) -> Dict[str, Sequence[int]]:
    return {k: tuple(v.shape) for k, v in params.items()}
