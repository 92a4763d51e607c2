"""End-to-end CPU oracle of the integer Whisper (TEST INFRASTRUCTURE ONLY).

Composes the oracle ops (oracle/iw_oracle.c) along the reference dataflow,
unfused and in the reference's tensor layouts:
  encoder       model_int.py:1260-1316  (AudioEncoder_int.forward)
  block         model_int.py:1112-1174  (ResidualAttentionBlock_int.forward)
  attention     model_int.py:713-1040   (MultiHeadAttention_int.forward / qkv_attention)
  decoder       model_int.py:1398-1484  (TextDecoder_int.forward)
  KV cache      model_int.py:1587-1618  (hooks concatenating key/value outputs)
  greedy        decoding.py:684-712 with GreedyDecoder.update (:280-296), as a fixed
                number of steps without logit filters; argmax over the int8 logits
                (dequantisation by a positive scale keeps the order).
Parameters are the integer state dict (name -> numpy array).
"""
from __future__ import annotations

import numpy as np

from .oracle import Oracle


class OracleWhisper:
    def __init__(self, dims, params, threads: int = 8, kind: str = "oracle"):
        """``kind`` "oracle" composes oracle/iw_oracle.c; "ref" composes the reference's
        own scalar kernels (oracle/_ref, where built) along the same dataflow."""
        self.d = dims
        self.P = params
        self.o = Oracle(kind, threads=threads)
        n = dims.n_text_ctx
        self.mask = np.triu(np.ones((n, n), dtype=bool), 1)

    # ---- layers ----
    def _lin8(self, x, p):
        P = self.P
        return self.o.linear8(x, P[p + ".weight"], P.get(p + ".bias"), P.get(p + ".wgt_zeros"),
                              P[p + ".req_multiplier"], P[p + ".req_shiftmount"])

    def _lin32(self, x, p):
        P = self.P
        return self.o.linear32(x, P[p + ".weight"], P.get(p + ".bias"), P.get(p + ".wgt_zeros"),
                               P[p + ".req_multiplier"], P[p + ".req_shiftmount"])

    def _ln(self, x, p):
        P = self.P
        return self.o.layernorm32(x, P[p + ".weight"], P.get(p + ".bias"),
                                  int(P[p + ".ln_req_multiplier"][0]),
                                  int(P[p + ".ln_req_shiftmount"][0]),
                                  int(P[p + ".out_req_multiplier"][0]),
                                  int(P[p + ".out_req_shiftmount"][0]))

    def _gelu(self, x, p):
        P = self.P
        return self.o.gelu(x, P[p + ".lut"], P[p + ".luti_req_multiplier"],
                           P[p + ".luti_req_shiftmount"], P[p + ".luto_req_multiplier"],
                           P[p + ".luto_req_shiftmount"])

    def _conv(self, x, p, stride):
        P = self.P
        return self.o.conv1d(x, P[p + ".weight"], P.get(p + ".bias"), int(P[p + ".req_multiplier"][0]),
                             int(P[p + ".req_shiftmount"][0]), stride, 1)

    def _mha(self, x, xa, mask, cache, p, n_head):
        P = self.P
        q = self._lin8(x, p + ".query")
        if cache is None or xa is None or (p + ".key") not in cache:
            k = self._lin8(x if xa is None else xa, p + ".key")
            v = self._lin8(x if xa is None else xa, p + ".value")
            if cache is not None:  # hook semantics (model_int.py:1596-1602)
                for name, t in ((p + ".key", k), (p + ".value", v)):
                    if name not in cache or t.shape[1] > self.d.n_text_ctx:
                        cache[name] = t
                    else:
                        cache[name] = np.concatenate([cache[name], t], axis=1)
                    if name.endswith("key"):
                        k = cache[name]
                    else:
                        v = cache[name]
        else:
            k, v = cache[p + ".key"], cache[p + ".value"]
        B, Tq, C = q.shape
        Tk = k.shape[1]
        D = C // n_head
        attn_mask = None
        if mask is not None:
            off = Tk - Tq
            attn_mask = np.ascontiguousarray(mask[off:off + Tq, :Tk])
        qh = q.reshape(B, Tq, n_head, D).transpose(0, 2, 1, 3)
        kh = k.reshape(B, Tk, n_head, D).transpose(0, 2, 1, 3)
        vh = v.reshape(B, Tk, n_head, D).transpose(0, 2, 3, 1)
        wv = self.o.attention(qh, kh, vh, attn_mask, int(P[p + ".qk_req_multiplier"][0]),
                              int(P[p + ".qk_req_shiftmount"][0]), int(P[p + ".qk_frac_bits"]),
                              int(P[p + ".av_req_multiplier"][0]), int(P[p + ".av_req_shiftmount"][0]),
                              16)
        return self._lin32(wv, p + ".out")

    def _block(self, x, xa, mask, cache, p, n_head, cross):
        P = self.P
        h = self._mha(self._ln(x, p + ".attn_ln"), None, mask, cache, p + ".attn", n_head)
        x = self.o.residual15(h, x, int(P[p + ".attn_res_req_multiplier"][0]))
        if cross:
            h = self._mha(self._ln(x, p + ".cross_attn_ln"), xa, None, cache, p + ".cross_attn", n_head)
            x = self.o.residual15(h, x, int(P[p + ".cross_attn_res_req_multiplier"][0]))
        h = self._gelu(self._lin8(self._ln(x, p + ".mlp_ln"), p + ".mlp.0"), p + ".mlp.1")
        h = self._lin32(h, p + ".mlp.2")
        return self.o.residual15(h, x, int(P[p + ".mlp_res_req_multiplier"][0]))

    # ---- model ----
    def encoder_input(self, mel):
        """round(mel * input_alpha) (fp32 multiply, round half to even), clamp +-127."""
        a = np.float32(self.P["encoder.input_alpha"].reshape(-1)[0])
        return np.clip(np.rint(mel.astype(np.float32) * a), -127, 127).astype(np.int8)

    def encoder_frontend(self, mel):
        P = self.P
        x = self.encoder_input(mel) if mel.dtype != np.int8 else mel
        x = self._gelu(self._conv(x, "encoder.conv1", 1), "encoder.gelu1")
        x = self._conv(x, "encoder.conv2", 2)
        x = self._gelu(np.ascontiguousarray(x.transpose(0, 2, 1)), "encoder.gelu2")
        return self.o.add_requant15(x, P["encoder.positional_embedding"], P["encoder.req_multiplier"],
                                    P["encoder.req_shiftmount"])

    def encoder(self, mel, layers: int = None):
        x = self.encoder_frontend(mel)
        n = self.d.n_audio_layer if layers is None else layers
        for i in range(n):
            x = self._block(x, None, None, None, f"encoder.blocks.{i}", self.d.n_audio_head, False)
        return self._ln(x, "encoder.ln_post")

    def decoder_logits(self, tokens, xa, cache=None):
        """int8 logits before dequant for every position of ``tokens``."""
        P = self.P
        offset = next(iter(cache.values())).shape[1] if cache else 0
        T = tokens.shape[1]
        emb = P["decoder.token_embedding.weight"][tokens]
        x = self.o.add_requant15(emb, P["decoder.positional_embedding"][offset:offset + T],
                                 P["decoder.req_multiplier"].astype(np.uint16),
                                 P["decoder.req_shiftmount"])
        for i in range(self.d.n_text_layer):
            x = self._block(x, xa, self.mask, cache, f"decoder.blocks.{i}", self.d.n_text_head, True)
        h = self._ln(x, "decoder.ln")
        return self.o.classifier(h, P["decoder.token_embedding.weight"],
                                 int(P["decoder.clf_req_multiplier"][0]),
                                 int(P["decoder.clf_req_shiftmount"][0]))

    def greedy(self, xa, prompt, steps: int, return_logits: bool = False):
        tokens = np.array(prompt, dtype=np.int64)
        cache = {}
        last = []
        for i in range(steps):
            inp = tokens if i == 0 else tokens[:, -1:]
            logits = self.decoder_logits(inp, xa, cache)[:, -1]
            last.append(logits)
            nxt = np.argmax(logits, axis=-1).astype(np.int64)
            tokens = np.concatenate([tokens, nxt[:, None]], axis=1)
        if return_logits:
            return tokens, np.stack(last, 1)
        return tokens

    def forced(self, xa, prompt, forced):
        """Teacher-forced decoding over the cache: the prompt step, then one step
        per column of ``forced`` [B, n] fed as the next input token. Returns the
        argmax of every step's last-position int8 logits [B, n + 1] and those
        logits [B, n + 1, vocab]."""
        tokens = np.array(prompt, dtype=np.int64)
        forced = np.asarray(forced, dtype=np.int64)
        cache = {}
        last = [self.decoder_logits(tokens, xa, cache)[:, -1]]
        for i in range(forced.shape[1]):
            last.append(self.decoder_logits(forced[:, i:i + 1], xa, cache)[:, -1])
        logits = np.stack(last, 1)
        return np.argmax(logits, axis=-1).astype(np.int64), logits
