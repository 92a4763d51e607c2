"""Batched encoder and greedy-decoder runners over a ``Whisper_int`` model.

These drive the same gfx950 kernels as the layer API with the data layout
chosen for the MI355X instead of the reference's per-call tensors:

* Q/K/V (and cross-attention K/V) projections run as one GEMM over the
  concatenated weights; the key projection has no bias, which equals a zero
  bias in the concatenation.
* The residual stream is one int16 buffer updated in place by the fused
  Linear32 + residual15 kernels.
* The decoder keeps preallocated per-head KV caches: self-attention K as
  [B, H, n_ctx, D] and V in key quads [B, H, n_ctx16 / 4, D, 4] (head_dim 64;
  V transposed per head [B, H, D, n_ctx16] for other head sizes);
  cross-attention K as [B, H, n_audio_ctx, D] and V transposed per head,
  projected once per utterance. This replaces
  the reference's hook-based ``torch.cat`` cache (model_int.py:1587-1618) with
  identical values.
* Greedy decoding feeds the last token each step (decoding.py:148-179,
  684-712) and takes the first maximum of the int8 logits for a fixed number
  of steps, optionally after the decoding task's logit filters
  (``LogitFilters``, applied on the device).

The runners copy (and for the one-token step, repack) the model's weights
when they are built: a runner built before ``load_state_dict`` keeps the old
weights, so build a new runner after loading new weights.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import List, Optional, Sequence

import numpy as np
import torch

from . import _lib
from .model_int import AudioEncoder_int, ResidualAttentionBlock_int, TextDecoder_int, Whisper_int


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _ptr(t):
    return None if t is None else t.data_ptr()


class _FusedLinear:
    """Several LinearBase layers sharing an input, as one [sum N, K] GEMM."""

    def __init__(self, layers):
        dev = layers[0].weight.device
        self.K = layers[0].in_features
        self.N = sum(l.out_features for l in layers)
        self.weight = torch.cat([l.weight for l in layers]).contiguous()
        biases = []
        for l in layers:
            biases.append(l.bias if l.bias is not None else
                          torch.zeros(l.out_features, dtype=torch.int32, device=dev))
        self.bias = torch.cat(biases).contiguous()
        self.wz = torch.cat([l.wgt_zeros for l in layers]).contiguous()
        self.mult = torch.cat([l.req_multiplier for l in layers]).contiguous()
        self.shift = torch.cat([l.req_shiftmount for l in layers]).contiguous()

    def linear8(self, x: torch.Tensor, M: int, out: torch.Tensor) -> torch.Tensor:
        _lib.call("iw_linear8", x.data_ptr(), self.weight.data_ptr(), self.bias.data_ptr(),
                  self.wz.data_ptr(), self.mult.data_ptr(), self.shift.data_ptr(), out.data_ptr(), M,
                  self.K, self.N, True, True, _stream())
        return out


def _lin8(layer, x_ptr: int, M: int, out: torch.Tensor):
    b, z = layer.bias, layer.wgt_zeros if layer.asym else None
    _lib.call("iw_linear8", x_ptr, layer.weight.data_ptr(), _ptr(b), _ptr(z),
              layer.req_multiplier.data_ptr(), layer.req_shiftmount.data_ptr(), out.data_ptr(), M,
              layer.in_features, layer.out_features, b is not None, z is not None, _stream())
    return out


def _lin32_res(layer, x_ptr: int, M: int, res: torch.Tensor, res_mult: int):
    b, z = layer.bias, layer.wgt_zeros if layer.asym else None
    _lib.call("iw_linear32_residual15", x_ptr, layer.weight.data_ptr(), _ptr(b), _ptr(z),
              layer.req_multiplier.data_ptr(), layer.req_shiftmount.data_ptr(), res.data_ptr(),
              res_mult, res.data_ptr(), M, layer.in_features, layer.out_features, b is not None,
              z is not None, _stream())


def _ln(ln, x: torch.Tensor, rows: int, out: torch.Tensor):
    s = ln._scalars()
    _lib.call("iw_layernorm32", x.data_ptr(), ln.weight.data_ptr(), _ptr(ln.bias), s["lm"], s["ls"],
              s["om"], s["os"], ln.offset, out.data_ptr(), rows, ln.normalized_shape[0],
              ln.bias is not None, _stream())
    return out


def _gelu_args(gelu) -> tuple:
    """GeLU parameter pointers and counts for the fused FC1 + GeLU GEMM. A
    per-channel parameter whose values are all equal is passed as a single
    value (count 1): the same results, and the large-M GEMM then applies GeLU
    as a table of the int8 value. Reads the parameters once (a device sync),
    so runners call it when they are built."""
    lut, im, is_, om, os_, ci, co = gelu.gelu_ptrs()

    def uniform(t: torch.Tensor) -> bool:
        return t.numel() > 1 and bool((t == t.reshape(-1)[0]).all())

    if uniform(gelu.luti_req_multiplier) and uniform(gelu.luti_req_shiftmount):
        ci = 1
    if uniform(gelu.luto_req_multiplier) and uniform(gelu.luto_req_shiftmount):
        co = 1
    return lut, im, is_, om, os_, ci, co


def _mlp_gelu(block: ResidualAttentionBlock_int, x_ptr: int, M: int, out: torch.Tensor,
              gelu_args: Optional[tuple] = None):
    fc1, gelu = block.mlp[0], block.mlp[1]
    lut, im, is_, om, os_, ci, co = gelu_args if gelu_args is not None else gelu.gelu_ptrs()
    _lib.call("iw_linear8_gelu", x_ptr, fc1.weight.data_ptr(), _ptr(fc1.bias),
              _ptr(fc1.wgt_zeros), fc1.req_multiplier.data_ptr(), fc1.req_shiftmount.data_ptr(),
              lut, im, is_, om, os_, ci, co, out.data_ptr(), M, fc1.in_features, fc1.out_features,
              fc1.bias is not None, fc1.wgt_zeros is not None, _stream())
    return out


def _frag_pack(w: torch.Tensor) -> torch.Tensor:
    """Fragment-major image of a row-major int8 [R, K] matrix (zero padded)."""
    R, K = w.shape
    out = torch.zeros(_lib.value("iw_frag_bytes", R, K), dtype=torch.int8, device=w.device)
    _lib.call("iw_frag_pack", w.data_ptr(), R, K, w.stride(0), out.data_ptr(), _stream())
    return out


def _frag_buffer(rows: int, cols: int, dev) -> torch.Tensor:
    """A zeroed fragment-major [rows, cols] activation buffer: producers write
    only the real rows and columns, so the padding stays zero."""
    return torch.zeros(_lib.value("iw_frag_bytes", rows, cols), dtype=torch.int8, device=dev)


_NO_PREFETCH = (None, 0, 0)


def _pf_args(nxt: Optional["_FragLinear"]):
    """The prefetch-hint arguments naming ``nxt``'s weight (or none)."""
    return nxt.pf() if nxt is not None else _NO_PREFETCH


def _ln_frag(ln, x: torch.Tensor, rows: int, out: torch.Tensor, nxt: Optional["_FragLinear"] = None):
    """LayerNorm into a fragment-major operand; ``nxt``: the GEMM that reads it,
    whose weight tiles the launch reads into L2 on the way."""
    s = ln._scalars()
    _lib.call("iw_layernorm32_frag", x.data_ptr(), ln.weight.data_ptr(), _ptr(ln.bias), s["lm"],
              s["ls"], s["om"], s["os"], ln.offset, out.data_ptr(), rows, ln.normalized_shape[0],
              ln.bias is not None, *_pf_args(nxt), _stream())
    return out


class _FragLinear:
    """A LinearBase layer (or a _FusedLinear) with its weight packed
    fragment-major for the one-token decode GEMMs."""

    def __init__(self, layer):
        fused = isinstance(layer, _FusedLinear)
        self.K = layer.K if fused else layer.in_features
        self.N = layer.N if fused else layer.out_features
        self.w = _frag_pack(layer.weight)
        self.bias = layer.bias
        self.wz = layer.wz if fused else (layer.wgt_zeros if layer.asym else None)
        self.mult = layer.mult if fused else layer.req_multiplier
        self.shift = layer.shift if fused else layer.req_shiftmount

    def args(self):
        return (self.w.data_ptr(), _ptr(self.bias), _ptr(self.wz), self.mult.data_ptr(),
                self.shift.data_ptr())

    def pf(self):
        """The prefetch-hint arguments naming this GEMM's weight."""
        return (self.w.data_ptr(), self.N, self.K)

    def linear8(self, xf: torch.Tensor, M: int, out: torch.Tensor, out_frag: bool = False):
        _lib.call("iw_linear8_frag", xf.data_ptr(), *self.args(), out.data_ptr(), M, self.K, self.N,
                  self.bias is not None, self.wz is not None, out_frag, _stream())

    def linear32_res(self, xf: torch.Tensor, M: int, res: torch.Tensor, res_mult: int):
        _lib.call("iw_linear32_residual15_frag", xf.data_ptr(), *self.args(), res.data_ptr(), res_mult,
                  res.data_ptr(), M, self.K, self.N, self.bias is not None, self.wz is not None,
                  _stream())


class EncoderRunner:
    """AudioEncoder_int forward for a fixed batch with preallocated activations."""

    def __init__(self, encoder: AudioEncoder_int, batch: int):
        self.enc = encoder
        self.B = batch
        C, H, T = encoder.n_state, encoder.n_head, encoder.n_ctx
        self.C, self.H, self.T, self.D = C, H, T, C // H
        self.M = batch * T
        dev = encoder.positional_embedding.device
        self.qkv = [_FusedLinear([b.attn.query, b.attn.key, b.attn.value]) for b in encoder.blocks]
        self.tp = (T + 15) // 16 * 16
        self.h8 = torch.empty((self.M, C), dtype=torch.int8, device=dev)
        self.qkv_buf = torch.empty((self.M, 3 * C), dtype=torch.int8, device=dev)
        self.vt = torch.empty((batch, H, self.D, self.tp), dtype=torch.int8, device=dev)
        self.wv = torch.empty((self.M, C), dtype=torch.int8, device=dev)
        self.f8 = torch.empty((self.M, 4 * C), dtype=torch.int8, device=dev)
        self.out = torch.empty((batch, T, C), dtype=torch.int8, device=dev)
        self.tables = [b.attn.shift_exp_table() for b in encoder.blocks]
        self.gelu_args = [_gelu_args(b.mlp[1]) for b in encoder.blocks]
        # Optional per-launch timing: a list receiving (kind, ops, start, end)
        # HIP events recorded on the launch stream around GEMM / attention calls.
        self.timer: Optional[list] = None

    def _tick(self, kind: str, ops: float):
        if self.timer is None:
            return None
        e = torch.cuda.Event(enable_timing=True)
        e.record()
        return kind, ops, e

    def _tock(self, tok):
        if tok is not None:
            e = torch.cuda.Event(enable_timing=True)
            e.record()
            self.timer.append((*tok, e))

    def block(self, i: int, x16: torch.Tensor):
        blk = self.enc.blocks[i]
        att = blk.attn
        s = att._scalars()
        sc = blk._scalars()
        B, C, H, D, T, M = self.B, self.C, self.H, self.D, self.T, self.M
        _ln(blk.attn_ln, x16, M, self.h8)
        t = self._tick("gemm", 2.0 * M * 3 * C * C)
        self.qkv[i].linear8(self.h8, M, self.qkv_buf)
        self._tock(t)
        q = self.qkv_buf.data_ptr()
        _lib.call("iw_transpose_heads", q + 2 * C, T * 3 * C, 3 * C, self.vt.data_ptr(),
                  H * D * self.tp, D * self.tp, self.tp, 4, 0, B, T, H, D, _stream())
        t = self._tick("attention", 4.0 * B * H * T * T * D)
        _lib.call("iw_attention", q, T * 3 * C, 3 * C, q + C, T * 3 * C, D, 3 * C,
                  self.vt.data_ptr(), H * D * self.tp, D * self.tp, self.tp, self.wv.data_ptr(),
                  T * C, C, None, B, H, T, T, D, s["qm"], s["qs"], s["f"], s["am"], s["as_"],
                  att.rsqrt_offset, self.tables[i].data_ptr(), False, _stream())
        self._tock(t)
        t = self._tick("gemm", 2.0 * M * C * C)
        _lin32_res(att.out, self.wv.data_ptr(), M, x16, sc["a"])
        self._tock(t)
        _ln(blk.mlp_ln, x16, M, self.h8)
        t = self._tick("gemm", 2.0 * M * 4 * C * C)
        _mlp_gelu(blk, self.h8.data_ptr(), M, self.f8, self.gelu_args[i])
        self._tock(t)
        t = self._tick("gemm", 2.0 * M * 4 * C * C)
        _lin32_res(blk.mlp[2], self.f8.data_ptr(), M, x16, sc["m"])
        self._tock(t)

    def __call__(self, mel: torch.Tensor) -> torch.Tensor:
        want = (self.B, self.enc.n_mels, 2 * self.T)
        if tuple(mel.shape) != want:
            raise ValueError(f"mel batch of shape {tuple(mel.shape)}; this runner takes {want}")
        if mel.dtype not in (torch.float32, torch.int8):
            raise ValueError(f"mel must be float32 or int8, not {mel.dtype}")
        x16 = self.enc.frontend(mel)
        for i in range(len(self.enc.blocks)):
            self.block(i, x16)
        _ln(self.enc.ln_post, x16, self.M, self.out)
        return self.out


@dataclass
class LogitFilters:
    """The decoding task's logit filters (decoding.py:410-509, built as in
    DecodingTask, :556-572) and the EOT freeze of GreedyDecoder.update
    (:290), applied on the device inside the greedy step.

    ``suppress_tokens``: SuppressTokens ids; ``suppress_blank``: SuppressBlank
    ids (``tokenizer.encode(" ") + [eot]``), empty = no SuppressBlank;
    ``timestamp_begin`` >= 0 turns ApplyTimestampRules on, with
    ``no_timestamps`` and ``max_initial_timestamp_index`` (< 0 = None) and the
    logits' dequantisation scale ``logit_scale`` (None = the decoder's
    1 / act_logits_alpha)."""
    eot: int
    suppress_tokens: Sequence[int] = ()
    suppress_blank: Sequence[int] = ()
    timestamp_begin: int = -1
    no_timestamps: int = -1
    max_initial_timestamp_index: int = -1
    logit_scale: Optional[float] = None


def _bitmask(ids, n: int, dev) -> torch.Tensor:
    words = np.zeros((n + 31) // 32, np.uint32)
    for i in ids:
        i = int(i)
        if not 0 <= i < n:
            raise ValueError(f"token id {i} outside the vocabulary")
        words[i >> 5] |= np.uint32(1) << np.uint32(i & 31)
    return torch.from_numpy(words).to(dev)


class DecoderRunner:
    """Greedy TextDecoder_int steps over preallocated self/cross KV caches.

    Caches are per layer and per head contiguous: self-attention K
    [B, H, n_ctx, D] and V transposed [B, H, D, n_ctx16]; cross-attention K
    [B, H, n_audio_ctx, D] and V transposed [B, H, D, n_audio_ctx16], projected
    once per utterance. The prompt step runs eagerly; every later step is one
    token per utterance and runs a fixed kernel sequence whose cache position
    lives in device memory, so it is captured once as a HIP graph and
    replayed (``use_graph``).
    """

    def __init__(self, decoder: TextDecoder_int, batch: int, n_audio_ctx: int,
                 max_steps: Optional[int] = None, use_graph: bool = True,
                 filters: Optional[LogitFilters] = None, frag: bool = True, prefetch: bool = True,
                 eot: Optional[int] = None, logprobs: bool = True, no_speech: Optional[int] = None,
                 sot_index: int = 0, fuse_cross: bool = True):
        """``eot``: the EOT id for GreedyDecoder.update's EOT freeze and the
        all-finished count without filters (the filters carry their own);
        ``logprobs``: accumulate each row's sum of log-probabilities
        (``sum_logprobs``); ``no_speech``: the no-speech token id, whose
        probability at the prompt position ``sot_index`` the prompt step
        records (``no_speech_probs``); ``fuse_cross``: the one-token step runs
        each cross-attention's LayerNorm and query projection inside the
        cross-attention kernel (head_dim 64), instead of as two launches."""
        self.dec = decoder
        self.B = batch
        C, H = decoder.n_state, decoder.n_head
        self.C, self.H, self.D = C, H, C // H
        self.Tcap = decoder.n_ctx
        self.tcap16 = (self.Tcap + 15) // 16 * 16
        self.Ta = n_audio_ctx
        self.ta16 = (n_audio_ctx + 15) // 16 * 16
        self.use_graph = use_graph
        dev = decoder.positional_embedding.device
        L, D = decoder.n_layer, self.D
        i8 = dict(dtype=torch.int8, device=dev)
        self.self_qkv = [_FusedLinear([b.attn.query, b.attn.key, b.attn.value]) for b in decoder.blocks]
        self.cross_kv = [_FusedLinear([b.cross_attn.key, b.cross_attn.value]) for b in decoder.blocks]
        self.k_self = [torch.zeros((batch, H, self.Tcap, D), **i8) for _ in range(L)]
        # V of the self-attention in key quads [B, H, Tcap/4, D, 4] (one
        # token's append is 4 D contiguous bytes per head) where the decode
        # attention reads them (head_dim 64), else transposed [B, H, D, Tcap]
        self.v_quads = D == 64
        if self.v_quads:
            self.v_self = [torch.zeros((batch, H, self.tcap16 // 4, 4 * D), **i8) for _ in range(L)]
            self.v_strides = (H * self.tcap16 * D, self.tcap16 * D, 4, 4 * D)
        else:
            self.v_self = [torch.zeros((batch, H, D, self.tcap16), **i8) for _ in range(L)]
            self.v_strides = (H * D * self.tcap16, D * self.tcap16, self.tcap16, 4)
        self.k_cross = [torch.zeros((batch, H, n_audio_ctx, D), **i8) for _ in range(L)]
        self.vt_cross = [torch.zeros((batch, H, D, self.ta16), **i8) for _ in range(L)]
        self.kv_tmp = torch.empty((batch * n_audio_ctx, 2 * C), **i8)
        self.self_tables = [b.attn.shift_exp_table() for b in decoder.blocks]
        self.cross_tables = [b.cross_attn.shift_exp_table() for b in decoder.blocks]
        # one-token step buffers
        self.x16 = torch.empty((batch, C), dtype=torch.int16, device=dev)
        self.h8 = torch.empty((batch, C), **i8)
        self.q8 = torch.empty((batch, C), **i8)
        self.wv = torch.empty((batch, C), **i8)
        self.f8 = torch.empty((batch, 4 * C), **i8)
        self.logits = torch.empty((batch, decoder.n_vocab), **i8)
        # fragment-major weights and activations of the one-token step
        self.frag = frag and batch <= 128 and 4 * C <= 5120
        # each LayerNorm (and FC1) of the one-token step reads the next
        # GEMM's weight tiles into L2 (a hint; results do not depend on it)
        self.prefetch = prefetch
        self.fuse_cross = fuse_cross and self.frag and self.D == 64 and n_audio_ctx <= 2048
        if self.frag:
            self.f_qkv = [_FragLinear(f) for f in self.self_qkv]
            self.f_out = [_FragLinear(b.attn.out) for b in decoder.blocks]
            self.f_cq = [_FragLinear(b.cross_attn.query) for b in decoder.blocks]
            self.f_co = [_FragLinear(b.cross_attn.out) for b in decoder.blocks]
            self.f_fc1 = [_FragLinear(b.mlp[0]) for b in decoder.blocks]
            self.f_fc2 = [_FragLinear(b.mlp[2]) for b in decoder.blocks]
            self.f_emb = _frag_pack(decoder.token_embedding.weight)
            self.h8f = _frag_buffer(batch, C, dev)
            self.wvf = _frag_buffer(batch, C, dev)
            self.f8f = _frag_buffer(batch, 4 * C, dev)
        # device-side decode state
        self.pos = torch.zeros(1, dtype=torch.int32, device=dev)   # tokens in the self caches
        self.step_no = torch.zeros(1, dtype=torch.int32, device=dev)
        self.tokens = torch.zeros(batch, dtype=torch.int64, device=dev)
        self.hist_cols = max_steps or decoder.n_ctx
        self.history = torch.zeros((batch, self.hist_cols), dtype=torch.int64, device=dev)
        self.graph = None
        self.graph_multi = None  # GRAPH_STEPS steps in one graph
        self.graph_stream = None
        self.prev0 = torch.zeros(batch, dtype=torch.int64, device=dev)  # the prompt's last token
        # GreedyDecoder.update's bookkeeping on the device: the per-tile row
        # maxima of the fused classifier, the rows' log-probability sums, the
        # number of rows whose token is EOT at each step, the arrival counter
        # of the update kernel's blocks (0 between launches)
        V = decoder.n_vocab
        self.tiles = (V + 31) // 32
        self.row_max = torch.zeros((batch, self.tiles), dtype=torch.uint16, device=dev)
        self.eot = filters.eot if filters is not None else (-1 if eot is None else int(eot))
        if filters is not None and eot is not None and int(eot) != filters.eot:
            raise ValueError("eot differs from the filters' EOT id")
        self.logprobs = logprobs
        self.sum_logprobs = torch.zeros(batch, dtype=torch.float32, device=dev)
        self.eot_count = torch.zeros(self.hist_cols, dtype=torch.int32, device=dev)
        self.arrive = torch.zeros(1, dtype=torch.int32, device=dev)
        self.no_speech = no_speech
        self.sot_index = sot_index
        self.no_speech_probs = torch.full((batch,), float("nan"), dtype=torch.float32, device=dev)
        self.steps_done = 0
        self.logit_scale = 1.0 / float(decoder.act_logits_alpha.detach().reshape(-1)[0].item())
        self.filters = filters
        if filters is not None:
            V = decoder.n_vocab
            ts_on = filters.timestamp_begin >= 0
            always = list(filters.suppress_tokens) + ([filters.no_timestamps]
                                                       if ts_on and filters.no_timestamps >= 0 else [])
            self.f_mask = _bitmask(always, V, dev) if always else None
            self.f_first = _bitmask(always + list(filters.suppress_blank), V, dev) \
                if filters.suppress_blank else None
            scale = filters.logit_scale
            if scale is None:
                scale = 1.0 / float(decoder.act_logits_alpha.detach().reshape(-1)[0].item())
            if ts_on and not scale > 0:
                raise ValueError("the timestamp rules need a positive logit scale")
            self.f_scale = float(scale)

    # ---- per utterance ----
    def set_audio(self, xa: torch.Tensor):
        """Project the cross-attention K/V of the encoder output once per utterance."""
        want = (self.B, self.Ta, self.C)
        if tuple(xa.shape) != want or xa.dtype != torch.int8:
            raise ValueError(f"audio features {tuple(xa.shape)} {xa.dtype}; this runner takes int8 {want}")
        if not xa.is_cuda:
            raise ValueError("audio features must be on the GPU")
        xa = xa.contiguous()
        B, Ta, C, H, D = self.B, self.Ta, self.C, self.H, self.D
        kv = self.kv_tmp
        for l in range(self.dec.n_layer):
            self.cross_kv[l].linear8(xa, B * Ta, kv)
            _lib.call("iw_gather_heads", kv.data_ptr(), Ta * 2 * C, 2 * C, self.k_cross[l].data_ptr(),
                      H * Ta * D, Ta * D, D, 0, B, Ta, H, D, _stream())
            _lib.call("iw_transpose_heads", kv.data_ptr() + C, Ta * 2 * C, 2 * C,
                      self.vt_cross[l].data_ptr(), H * D * self.ta16, D * self.ta16, self.ta16, 4, 0, B,
                      Ta, H, D, _stream())

    def reset(self):
        self.pos.zero_()
        self.step_no.zero_()
        self.sum_logprobs.zero_()
        self.eot_count.zero_()
        self.no_speech_probs.fill_(float("nan"))

    # ---- shared pieces ----
    def _cross_attend(self, att, l, q_ptr, q_sb, q_st, Tq, out, table):
        s = att._scalars()
        H, D, Ta = self.H, self.D, self.Ta
        if Tq <= 8:
            # the streaming decode kernel with every query position of a head
            # sharing its pass over the cached K/V, where the prefill kernel
            # would do the work of a whole 128-row query tile
            _lib.call("iw_attention", q_ptr, q_sb, q_st, self.k_cross[l].data_ptr(), H * Ta * D, Ta * D, D,
                      self.vt_cross[l].data_ptr(), H * D * self.ta16, D * self.ta16, self.ta16, out.data_ptr(),
                      Tq * self.C, self.C, None, self.B, H, Tq, Ta, D, s["qm"], s["qs"], s["f"], s["am"],
                      s["as_"], att.rsqrt_offset, None, True, _stream())
        else:
            _lib.call("iw_attention", q_ptr, q_sb, q_st, self.k_cross[l].data_ptr(), H * Ta * D,
                      Ta * D, D, self.vt_cross[l].data_ptr(), H * D * self.ta16, D * self.ta16,
                      self.ta16, out.data_ptr(), Tq * self.C, self.C, None, self.B, H, Tq, Ta, D,
                      s["qm"], s["qs"], s["f"], s["am"], s["as_"], att.rsqrt_offset,
                      table.data_ptr(), False, _stream())

    def cross_attention(self, layer: int, q: torch.Tensor, out: torch.Tensor):
        """One decode-step cross-attention of ``layer`` over this utterance's
        cached K/V: q and out are [B, C] int8 (launched on the current stream)."""
        att = self.dec.blocks[layer].cross_attn
        self._cross_attend(att, layer, q.data_ptr(), self.C, self.C, 1, out, None)

    def cross_attention_lnq(self, layer: int, out: torch.Tensor):
        """The one-token step's fused cross-attention of ``layer`` (its
        LayerNorm and query projection computed in the kernel) on the current
        residual rows (``x16``): out is the fragment-major [B, C] image (launched
        on the current stream; needs ``fuse_cross``)."""
        if not self.fuse_cross:
            raise ValueError("this runner does not fuse the cross-attention")
        self._cross_lnq(layer, out)

    def _cross_lnq(self, l: int, out: torch.Tensor):
        blk = self.dec.blocks[l]
        B, C, H, D, Ta = self.B, self.C, self.H, self.D, self.Ta
        s = blk.cross_attn._scalars()
        ln, cq = blk.cross_attn_ln, self.f_cq[l]
        lsc = ln._scalars()
        _lib.call("iw_attention_decode_cross_lnq", self.x16.data_ptr(), C, ln.weight.data_ptr(), _ptr(ln.bias),
                  lsc["lm"], lsc["ls"], lsc["om"], lsc["os"], ln.offset, ln.bias is not None,
                  cq.w.data_ptr(), _ptr(cq.bias), _ptr(cq.wz), cq.mult.data_ptr(), cq.shift.data_ptr(),
                  cq.bias is not None, cq.wz is not None, self.k_cross[l].data_ptr(), H * Ta * D, Ta * D, D,
                  self.vt_cross[l].data_ptr(), H * D * self.ta16, D * self.ta16, self.ta16, out.data_ptr(), B, H,
                  D, Ta, s["qm"], s["qs"], s["f"], s["am"], s["as_"], blk.cross_attn.rsqrt_offset, _stream())

    def _finish(self, x_last: torch.Tensor, pos_inc: int):
        """Final LayerNorm of the last position, classifier (with the row maxima
        fused into its epilogue on the fragment-major path), then one
        GreedyDecoder.update: token, EOT freeze, log-probability sum, EOT count,
        history, counters."""
        dec = self.dec
        sc = dec.scalars()
        f = self.filters
        fused = self.frag and f is None
        if self.frag:
            _ln_frag(dec.ln, x_last, self.B, self.h8f)
            if fused:
                _lib.call("iw_classifier_argmax_frag", self.h8f.data_ptr(), self.f_emb.data_ptr(), sc["cm"],
                          sc["cs"], self.logits.data_ptr(), self.row_max.data_ptr(), self.B, self.C,
                          dec.n_vocab, _stream())
            else:
                _lib.call("iw_classifier_frag", self.h8f.data_ptr(), self.f_emb.data_ptr(), sc["cm"], sc["cs"],
                          self.logits.data_ptr(), self.B, self.C, dec.n_vocab, _stream())
        else:
            _ln(dec.ln, x_last, self.B, self.h8)
            _lib.call("iw_classifier", self.h8.data_ptr(), dec.token_embedding.weight.data_ptr(),
                      sc["cm"], sc["cs"], self.logits.data_ptr(), self.B, self.C, dec.n_vocab,
                      _stream())
        lp = self.sum_logprobs.data_ptr() if self.logprobs else None
        if f is None:
            _lib.call("iw_greedy_update", self.row_max.data_ptr() if fused else None, self.tiles,
                      self.logits.data_ptr(), dec.n_vocab, self.B, dec.n_vocab, self.tokens.data_ptr(),
                      self.history.data_ptr(), self.hist_cols, self.hist_cols, self.step_no.data_ptr(),
                      self.pos.data_ptr(), pos_inc, self.eot, self.prev0.data_ptr(), lp, self.logit_scale,
                      self.eot_count.data_ptr() if self.eot >= 0 else None, self.arrive.data_ptr(), _stream())
        else:
            _lib.call("iw_greedy_advance_filtered", self.logits.data_ptr(), self.B, dec.n_vocab,
                      dec.n_vocab, self.tokens.data_ptr(), self.history.data_ptr(), self.hist_cols,
                      self.hist_cols, self.step_no.data_ptr(), self.pos.data_ptr(), pos_inc,
                      _ptr(self.f_mask), _ptr(self.f_first), self.prev0.data_ptr(), f.eot,
                      f.timestamp_begin, f.max_initial_timestamp_index, self.f_scale, lp,
                      self.eot_count.data_ptr(), _stream())

    # ---- the prompt (several tokens, cache empty) ----
    def prompt_step(self, tokens: torch.Tensor):
        dec = self.dec
        B, C, H, D = self.B, self.C, self.H, self.D
        P = tokens.shape[1]
        if P > self.Tcap:
            raise ValueError("prompt longer than n_text_ctx")
        if self.no_speech is not None and not 0 <= self.sot_index < P:
            raise ValueError("sot_index outside the prompt")
        M = B * P
        dev = tokens.device
        x16 = dec.embed(tokens.view(B, P), 0).view(M, C)
        h8 = torch.empty((M, C), dtype=torch.int8, device=dev)
        qkv = torch.empty((M, 3 * C), dtype=torch.int8, device=dev)
        wv = torch.empty((M, C), dtype=torch.int8, device=dev)
        qc = torch.empty((M, C), dtype=torch.int8, device=dev)
        f8 = torch.empty((M, 4 * C), dtype=torch.int8, device=dev)
        mask = dec.mask[:P, :P].contiguous()
        # the prompt's V transposed for the prefill attention (the cache may
        # hold key quads)
        p16 = (P + 15) // 16 * 16
        vt = torch.empty((B, H, D, p16), dtype=torch.int8, device=dev) if self.v_quads else None
        for l, blk in enumerate(dec.blocks):
            sc = blk._scalars()
            _ln(blk.attn_ln, x16, M, h8)
            self.self_qkv[l].linear8(h8, M, qkv)
            q = qkv.data_ptr()
            _lib.call("iw_gather_heads", q + C, P * 3 * C, 3 * C, self.k_self[l].data_ptr(),
                      H * self.Tcap * D, self.Tcap * D, D, 0, B, P, H, D, _stream())
            _lib.call("iw_transpose_heads", q + 2 * C, P * 3 * C, 3 * C, self.v_self[l].data_ptr(),
                      *self.v_strides, 0, B, P, H, D, _stream())
            if vt is not None:
                _lib.call("iw_transpose_heads", q + 2 * C, P * 3 * C, 3 * C, vt.data_ptr(), H * D * p16,
                          D * p16, p16, 4, 0, B, P, H, D, _stream())
                vt_args = (vt.data_ptr(), H * D * p16, D * p16, p16)
            else:
                vt_args = (self.v_self[l].data_ptr(), *self.v_strides[:3])
            s = blk.attn._scalars()
            _lib.call("iw_attention", q, P * 3 * C, 3 * C, self.k_self[l].data_ptr(), H * self.Tcap * D,
                      self.Tcap * D, D, *vt_args, wv.data_ptr(), P * C, C, mask.data_ptr(), B, H, P,
                      P, D, s["qm"], s["qs"], s["f"], s["am"], s["as_"], blk.attn.rsqrt_offset,
                      self.self_tables[l].data_ptr(), False, _stream())
            _lin32_res(blk.attn.out, wv.data_ptr(), M, x16, sc["a"])
            _ln(blk.cross_attn_ln, x16, M, h8)
            _lin8(blk.cross_attn.query, h8.data_ptr(), M, qc)
            self._cross_attend(blk.cross_attn, l, qc.data_ptr(), P * C, C, P, wv, self.cross_tables[l])
            _lin32_res(blk.cross_attn.out, wv.data_ptr(), M, x16, sc["c"])
            _ln(blk.mlp_ln, x16, M, h8)
            _mlp_gelu(blk, h8.data_ptr(), M, f8)
            _lin32_res(blk.mlp[2], f8.data_ptr(), M, x16, sc["m"])
        if self.no_speech is not None:
            # the no-speech probability at the start-of-transcript position
            # (decoding.py:690-695): softmax of that position's logits
            sot = x16.view(B, P, C)[:, self.sot_index].contiguous()
            h = torch.empty((B, C), dtype=torch.int8, device=dev)
            lg = torch.empty((B, dec.n_vocab), dtype=torch.int8, device=dev)
            _ln(dec.ln, sot, B, h)
            sc0 = dec.scalars()
            _lib.call("iw_classifier", h.data_ptr(), dec.token_embedding.weight.data_ptr(), sc0["cm"], sc0["cs"],
                      lg.data_ptr(), B, C, dec.n_vocab, _stream())
            _lib.call("iw_token_prob", lg.data_ptr(), B, dec.n_vocab, dec.n_vocab, self.no_speech,
                      self.logit_scale, self.no_speech_probs.data_ptr(), _stream())
        last = x16.view(B, P, C)[:, P - 1].contiguous()
        self._finish(last, P)

    # ---- one token per utterance (graph-capturable) ----
    def decode_step(self):
        dec = self.dec
        B, C, H, D = self.B, self.C, self.H, self.D
        sc0 = dec.scalars()
        _lib.call("iw_embed_tokens", self.tokens.data_ptr(), dec.token_embedding.weight.data_ptr(),
                  dec.positional_embedding.data_ptr(), dec.n_ctx, self.pos.data_ptr(),
                  sc0["m16"].data_ptr(), sc0["s"].data_ptr(), self.x16.data_ptr(), B, C, _stream())
        if self.frag:
            self._decode_layers_frag()
            self._finish(self.x16, 1)
            return
        x16, h8, q8, wv, f8 = self.x16, self.h8, self.q8, self.wv, self.f8
        for l, blk in enumerate(dec.blocks):
            sc = blk._scalars()
            fq = self.self_qkv[l]
            _ln(blk.attn_ln, x16, B, h8)
            _lib.call("iw_linear8_qkv_cache", h8.data_ptr(), fq.weight.data_ptr(), fq.bias.data_ptr(),
                      fq.wz.data_ptr(), fq.mult.data_ptr(), fq.shift.data_ptr(), B, C, True, True,
                      q8.data_ptr(), C, self.k_self[l].data_ptr(), H * self.Tcap * D, self.Tcap * D, D,
                      self.v_self[l].data_ptr(), *self.v_strides, C, D, 1, self.Tcap, self.pos.data_ptr(),
                      _stream())
            s = blk.attn._scalars()
            _lib.call("iw_attention_decode_cache", q8.data_ptr(), C, self.k_self[l].data_ptr(),
                      H * self.Tcap * D, self.Tcap * D, D, self.v_self[l].data_ptr(), *self.v_strides,
                      wv.data_ptr(), C, B, H, D, 1,
                      self.pos.data_ptr(), self.Tcap, s["qm"], s["qs"], s["f"], s["am"], s["as_"],
                      blk.attn.rsqrt_offset, _stream())
            _lin32_res(blk.attn.out, wv.data_ptr(), B, x16, sc["a"])
            _ln(blk.cross_attn_ln, x16, B, h8)
            _lin8(blk.cross_attn.query, h8.data_ptr(), B, q8)
            self._cross_attend(blk.cross_attn, l, q8.data_ptr(), C, C, 1, wv, None)
            _lin32_res(blk.cross_attn.out, wv.data_ptr(), B, x16, sc["c"])
            _ln(blk.mlp_ln, x16, B, h8)
            _mlp_gelu(blk, h8.data_ptr(), B, f8)
            _lin32_res(blk.mlp[2], f8.data_ptr(), B, x16, sc["m"])
        self._finish(x16, 1)

    def _decode_layers_frag(self):
        """The decoder blocks of one token step on fragment-major operands: each
        LayerNorm, attention and FC1 writes the operand image its GEMM reads."""
        dec = self.dec
        B, C, H, D = self.B, self.C, self.H, self.D
        x16, q8, h8f, wvf, f8f = self.x16, self.q8, self.h8f, self.wvf, self.f8f
        pf = (lambda f: f) if self.prefetch else (lambda f: None)
        for l, blk in enumerate(dec.blocks):
            sc = blk._scalars()
            fq = self.f_qkv[l]
            _ln_frag(blk.attn_ln, x16, B, h8f, pf(fq))
            _lib.call("iw_linear8_qkv_cache_frag", h8f.data_ptr(), *fq.args(), B, C, True, True,
                      q8.data_ptr(), C, self.k_self[l].data_ptr(), H * self.Tcap * D, self.Tcap * D, D,
                      self.v_self[l].data_ptr(), *self.v_strides, C, D, 1, self.Tcap, self.pos.data_ptr(),
                      _stream())
            s = blk.attn._scalars()
            _lib.call("iw_attention_decode_cache_frag", q8.data_ptr(), C, self.k_self[l].data_ptr(),
                      H * self.Tcap * D, self.Tcap * D, D, self.v_self[l].data_ptr(), *self.v_strides,
                      wvf.data_ptr(), B, H, D, 1,
                      self.pos.data_ptr(), self.Tcap, s["qm"], s["qs"], s["f"], s["am"], s["as_"],
                      blk.attn.rsqrt_offset, *_pf_args(pf(self.f_out[l])), _stream())
            self.f_out[l].linear32_res(wvf, B, x16, sc["a"])
            s = blk.cross_attn._scalars()
            Ta = self.Ta
            if self.fuse_cross:
                self._cross_lnq(l, wvf)
            else:
                _ln_frag(blk.cross_attn_ln, x16, B, h8f, pf(self.f_cq[l]))
                self.f_cq[l].linear8(h8f, B, q8)
                _lib.call("iw_attention_decode_cache_frag", q8.data_ptr(), C, self.k_cross[l].data_ptr(),
                          H * Ta * D, Ta * D, D, self.vt_cross[l].data_ptr(), H * D * self.ta16,
                          D * self.ta16, self.ta16, 4, wvf.data_ptr(), B, H, D, Ta, None, Ta, s["qm"], s["qs"],
                          s["f"], s["am"], s["as_"], blk.cross_attn.rsqrt_offset, *_NO_PREFETCH, _stream())
            self.f_co[l].linear32_res(wvf, B, x16, sc["c"])
            f1, f2 = self.f_fc1[l], self.f_fc2[l]
            _ln_frag(blk.mlp_ln, x16, B, h8f, pf(f1))
            lut, im, is_, om, os_, ci, co = blk.mlp[1].gelu_ptrs()
            nxt = pf(f2)
            _lib.call("iw_linear8_gelu_frag", h8f.data_ptr(), *f1.args(), lut, im, is_, om, os_, ci, co,
                      f8f.data_ptr(), B, f1.K, f1.N, f1.bias is not None, f1.wz is not None, True,
                      *_pf_args(nxt), _stream())
            f2.linear32_res(f8f, B, x16, sc["m"])

    # Steps per replay of the multi-step graph: every graph launch leaves a
    # gap of ~9 us before its first kernel, so n steps run as n // 8 replays of
    # an 8-step graph and the rest as replays of the one-step graph.
    GRAPH_STEPS = 8

    def _replay(self, n: int):
        if n <= 0:
            return
        if not self.use_graph:
            for _ in range(n):
                self.decode_step()
            return
        if self.graph is None:
            # one eager step on the capture stream loads every kernel before
            # capture
            s = torch.cuda.Stream()
            s.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(s):
                self.decode_step()
            n -= 1
            s.synchronize()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=s):
                self.decode_step()
            self.graph, self.graph_stream = g, s
        if n >= self.GRAPH_STEPS and self.graph_multi is None:
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=self.graph_stream):
                for _ in range(self.GRAPH_STEPS):
                    self.decode_step()
            self.graph_multi = g
        if self.graph_multi is not None:
            for _ in range(n // self.GRAPH_STEPS):
                self.graph_multi.replay()
            n %= self.GRAPH_STEPS
        for _ in range(n):
            self.graph.replay()

    def run(self, prompt: torch.Tensor, steps: int, keep_logits: bool = False, stop_on_eot: bool = False):
        """Greedy tokens [B, steps] after ``prompt`` (and the int8 logits of every step).
        With ``stop_on_eot`` (needs an EOT id) decoding ends once every row's
        latest token is EOT (DecodingTask._main_loop's ``completed``,
        decoding.py:710), checked after each graph replay; the tokens then end
        at that step. ``steps_done`` holds the number of steps taken."""
        if prompt.dim() != 2 or prompt.shape[0] != self.B or prompt.shape[1] < 1:
            raise ValueError(f"prompt of shape {tuple(prompt.shape)}; this runner takes [{self.B}, P >= 1]")
        if prompt.dtype != torch.int64 or not prompt.is_cuda:
            raise ValueError("prompt must be an int64 tensor on the GPU")
        if steps < 1:
            raise ValueError("steps must be at least 1")
        if prompt.shape[1] + steps > self.Tcap:
            raise ValueError(f"prompt + steps exceeds n_text_ctx ({self.Tcap})")
        if steps > self.hist_cols:
            raise ValueError("more steps than the history holds")
        if stop_on_eot and self.eot < 0:
            raise ValueError("stop_on_eot needs the EOT id (eot= or filters)")
        self.reset()
        self.prev0.copy_(prompt[:, -1])
        logits = []
        self.prompt_step(prompt.contiguous())
        done = 1
        if keep_logits:
            logits.append(self.logits.clone())
            while done < steps and not (stop_on_eot and self._all_eot(done)):
                self.decode_step()
                logits.append(self.logits.clone())
                done += 1
        elif not stop_on_eot:
            self._replay(steps - 1)
            done = steps
        else:
            while done < steps and not self._all_eot(done):
                n = min(self.GRAPH_STEPS, steps - done)
                self._replay(n)
                done += n
            # the replays past the finishing step only repeat EOT; end at it
            cnt = self.eot_count[:done].cpu()
            fin = (cnt == self.B).nonzero()
            if len(fin):
                done = int(fin[0]) + 1
        self.steps_done = done
        toks = self.history[:, :done]
        if keep_logits:
            return toks, torch.stack(logits, 1)
        return toks

    def _all_eot(self, done: int) -> bool:
        """Whether every row's token of step ``done - 1`` is EOT (one read of the device count)."""
        return int(self.eot_count[done - 1]) == self.B

    def run_forced(self, prompt: torch.Tensor, forced: torch.Tensor):
        """Teacher-forced steps: the prompt step, then one step per column of
        ``forced`` [B, n] fed as the next input token instead of the previous
        step's choice (eager launches). Returns the first-index argmax of every
        step's int8 logits [B, n + 1] and those logits [B, n + 1, vocab]."""
        if self.filters is not None:
            raise ValueError("teacher forcing takes a runner built without logit filters")
        if forced.dim() != 2 or forced.shape[0] != self.B or forced.dtype != torch.int64:
            raise ValueError(f"forced tokens must be int64 [{self.B}, n]")
        n = forced.shape[1]
        if n + 1 > self.hist_cols or prompt.shape[1] + n > self.Tcap:
            raise ValueError("too many forced steps for this runner")
        if n and (int(forced.min()) < 0 or int(forced.max()) >= self.dec.n_vocab):
            raise ValueError("forced token id out of range")
        self.run(prompt, 1, keep_logits=True)
        logits = [self.logits.clone()]
        for i in range(n):
            self.tokens.copy_(forced[:, i])
            self.decode_step()
            logits.append(self.logits.clone())
        return self.history[:, :n + 1].clone(), torch.stack(logits, 1)


@dataclass
class GreedyResult:
    """What DecodingTask._main_loop returns for greedy decoding
    (decoding.py:684-712): the tokens, each row's sum of log-probabilities of
    its sampled tokens (up to its EOT) and the no-speech probability at the
    start-of-transcript position (NaN without a no-speech id)."""
    tokens: torch.Tensor           # int64 [B, prompt_len + steps]
    sum_logprobs: torch.Tensor     # float32 [B]
    no_speech_probs: torch.Tensor  # float32 [B]
    steps: int                     # greedy steps taken (fewer than asked when all rows ended)


def greedy_decode(model: Whisper_int, audio_features: torch.Tensor, prompt: torch.Tensor,
                  steps: int, runner: Optional[DecoderRunner] = None,
                  keep_logits: bool = False, filters: Optional[LogitFilters] = None,
                  eot: Optional[int] = None, no_speech: Optional[int] = None, stop_on_eot: bool = False,
                  return_result: bool = False):
    """Greedy decoding; returns int64 tokens [B, prompt_len + steps] (and the int8 logits of
    every step [B, steps, vocab] when ``keep_logits``), or a GreedyResult with
    ``return_result``. With ``filters`` the decoding task's logit filters and the EOT freeze
    apply at every step on the device; without them the choice is the plain first-index argmax
    (with the EOT freeze when ``eot`` is given). ``stop_on_eot`` ends decoding once every row
    has emitted EOT. A given ``runner`` must have been built with the same filters, EOT and
    no-speech ids."""
    B, P = prompt.shape
    dec = model.decoder
    if P + steps > dec.n_ctx:
        raise ValueError(f"prompt + steps exceeds n_text_ctx ({dec.n_ctx})")
    if int(prompt.min()) < 0 or int(prompt.max()) >= dec.n_vocab:
        raise ValueError("prompt token id out of range")
    if steps <= 0:
        return prompt.clone()
    if runner is None:
        runner = DecoderRunner(dec, B, audio_features.shape[1], use_graph=not keep_logits,
                               filters=filters, eot=eot, no_speech=no_speech)
    else:
        if runner.filters is not filters:
            raise ValueError("the runner was built with other logit filters (pass the runner's own "
                             "filters, or None for a runner built without filters)")
        if (eot is not None and int(eot) != runner.eot) or (no_speech is not None and no_speech != runner.no_speech):
            raise ValueError("the runner was built with another EOT or no-speech id")
    runner.set_audio(audio_features)
    res = runner.run(prompt, steps, keep_logits=keep_logits, stop_on_eot=stop_on_eot)
    logits = None
    if keep_logits:
        res, logits = res
    toks = torch.cat([prompt, res], 1)
    if return_result:
        out = GreedyResult(toks, runner.sum_logprobs.clone(), runner.no_speech_probs.clone(), runner.steps_done)
        return (out, logits) if keep_logits else out
    return (toks, logits) if keep_logits else toks
