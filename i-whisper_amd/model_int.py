"""Integer Whisper layers on gfx950: the counterpart of i_whisper/model_int.py.

Class names, constructor arguments, parameter / buffer names, dtypes and
forward signatures follow the reference (model_int.py:50-1622) so a reference
integer checkpoint loads with a strict ``load_state_dict`` and callers switch
by setting ``backend = "hip"`` (the only backend here; see linear.py).

Inside the layers the reference's op chains are fused where the result is
identical element for element: FC1 with GeLU, out-projection / FC2 with the
residual15 merge, conv with GeLU (and the encoder's positional
add_requant15), and the three attention ops (qk_requant_rowmax, shift_exp,
pv_norm_requant) in one kernel.
"""
from __future__ import annotations

import base64
import gzip
from dataclasses import dataclass
from logging import Logger
from typing import Dict, Iterable, List, Optional, Union

import numpy as np
import torch
import torch.nn.functional as F  # noqa: F401  (kept for API parity with the reference)
from torch import Tensor, nn

from . import _lib
from .linear import BACKENDS, Linear8, Linear32, check_backend

__all__ = [
    "ModelDimensions", "GELU_int", "LayerNorm_int", "Conv1d_int", "MultiHeadAttention_int",
    "ResidualAttentionBlock_int", "AudioEncoder_int", "TextDecoder_int", "Whisper_int",
]


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _ptr(t: Optional[Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _item(t: Tensor) -> int:
    return int(t.reshape(-1)[0].item())


class _ScalarCache:
    """Caches host copies of one-element quantisation parameters.

    The values are read once (a device sync) and dropped whenever parameters
    are loaded or moved.
    """

    _scal: Optional[dict] = None

    def _scalars(self) -> dict:
        if self._scal is None:
            self._scal = self._read_scalars()
        return self._scal

    def _read_scalars(self) -> dict:  # pragma: no cover - overridden
        return {}

    def _load_from_state_dict(self, *args, **kwargs):
        self._scal = None
        return super()._load_from_state_dict(*args, **kwargs)

    def _apply(self, fn, *args, **kwargs):
        self._scal = None
        return super()._apply(fn, *args, **kwargs)


@dataclass
class ModelDimensions:
    """model_int.py:50-61."""
    n_mels: int
    n_audio_ctx: int
    n_audio_state: int
    n_audio_head: int
    n_audio_layer: int
    n_vocab: int
    n_text_ctx: int
    n_text_state: int
    n_text_head: int
    n_text_layer: int


# ---------------------------------------------------------------------------
# GeLU, LayerNorm, Conv1d
# ---------------------------------------------------------------------------

class GELU_int(nn.Module):
    """Integer GeLU with a 16-entry sigmoid LUT (model_int.py:66-174; gelu_scalar.cpp:10-181)."""

    def __init__(self, channel_num: int = 1, out_channel_num: int = 1, backend: str = "hip"):
        super().__init__()
        check_backend(backend)
        self.channel_num = channel_num
        self.backend = backend
        self.out_channel_num = out_channel_num if channel_num == 1 else channel_num
        self.act_bit, self.lut_index_bit, self.lut_data_bit = 8, 4, 8
        self.act_range, self.lut_upper, self.lut_zero = 127, 15, 8
        self.lut = nn.Parameter(torch.arange(0, 16).to(torch.uint8), requires_grad=False)
        self.luti_req_multiplier = nn.Parameter(torch.ones(channel_num, dtype=torch.uint8),
                                                requires_grad=False)
        self.luti_req_shiftmount = nn.Parameter(torch.zeros(channel_num, dtype=torch.int8),
                                                requires_grad=False)
        self.luto_req_multiplier = nn.Parameter(torch.ones(self.out_channel_num, dtype=torch.uint8),
                                                requires_grad=False)
        self.luto_req_shiftmount = nn.Parameter(torch.zeros(self.out_channel_num, dtype=torch.int8),
                                                requires_grad=False)
        self.de_smooth_vec = nn.Parameter(torch.ones(channel_num, dtype=torch.uint8),
                                          requires_grad=False)

    def gelu_ptrs(self):
        return (self.lut.data_ptr(), self.luti_req_multiplier.data_ptr(),
                self.luti_req_shiftmount.data_ptr(), self.luto_req_multiplier.data_ptr(),
                self.luto_req_shiftmount.data_ptr(), self.luti_req_multiplier.numel(),
                self.luto_req_multiplier.numel())

    def forward(self, x: Tensor) -> Tensor:
        assert x.dtype == torch.int8, "Input tensor must be int8 in integer inference mode!"
        check_backend(self.backend)
        x = x.contiguous()
        C = x.size(-1)
        lut, im, is_, om, os_, ci, co = self.gelu_ptrs()
        if ci not in (1, C) or co not in (1, C):
            raise RuntimeError("luti/luto parameters must be scalar or match input.size(-1)")
        out = torch.empty_like(x)
        if x.numel():
            _lib.call("iw_gelu", x.data_ptr(), lut, im, is_, om, os_, out.data_ptr(), x.numel(), C,
                      ci, co, _stream())
        return out


class LayerNorm_int(_ScalarCache, nn.LayerNorm):
    """LN32 (model_int.py:177-291; layernorm_scalar.cpp:464-624). Returns (int8 out, input clone)."""

    def __init__(self, normalized_shape, eps: float = 1e-5, elementwise_affine: bool = True,
                 device="cpu", backend: str = "hip"):
        nn.LayerNorm.__init__(self, normalized_shape, eps, elementwise_affine, device="meta")
        check_backend(backend)
        self.backend = backend
        self.act_bit, self.wgt_bit, self.norm_out_bit = 15, 8, 8
        self.offset = 13
        self.act_range, self.wgt_range, self.norm_out_range = 16383, 127, 127
        n = self.normalized_shape[0]
        self.weight = nn.Parameter(torch.ones(n, dtype=torch.int8, device=device), requires_grad=False)
        if self.bias is not None:
            self.bias = nn.Parameter(torch.zeros(n, dtype=torch.int32, device=device),
                                     requires_grad=False)
        self.ln_req_multiplier = nn.Parameter(torch.ones(1, dtype=torch.uint8, device=device),
                                              requires_grad=False)
        self.ln_req_shiftmount = nn.Parameter(torch.zeros(1, dtype=torch.int8, device=device),
                                              requires_grad=False)
        self.out_req_multiplier = nn.Parameter(torch.ones(1, dtype=torch.uint32, device=device),
                                               requires_grad=False)
        self.out_req_shiftmount = nn.Parameter(torch.zeros(1, dtype=torch.int8, device=device),
                                               requires_grad=False)

    def _read_scalars(self):
        return dict(lm=_item(self.ln_req_multiplier), ls=_item(self.ln_req_shiftmount),
                    om=_item(self.out_req_multiplier), os=_item(self.out_req_shiftmount))

    def normalize(self, x: Tensor, out: Optional[Tensor] = None) -> Tensor:
        """The int8 output only, optionally into ``out``."""
        check_backend(self.backend)
        if x.dtype != torch.int16:
            raise AssertionError("LayerNorm_int input must be int16")
        x = x.contiguous()
        H = x.size(-1)
        s = self._scalars()
        if out is None:
            out = torch.empty(x.shape, dtype=torch.int8, device=x.device)
        _lib.call("iw_layernorm32", x.data_ptr(), self.weight.data_ptr(), _ptr(self.bias), s["lm"],
                  s["ls"], s["om"], s["os"], self.offset, out.data_ptr(), x.numel() // H, H,
                  self.bias is not None, _stream())
        return out

    def forward(self, x: Tensor):
        return self.normalize(x), x.clone()


class Conv1d_int(_ScalarCache, nn.Conv1d):
    """int8 Conv1d + bias + per-tensor requant (model_int.py:538-673; conv1d_scalar.cpp:186-288).

    ``weight`` is [Cout, Cin*K] with the kernel index fastest, as in the reference.
    """

    def __init__(self, in_channels: int, out_channels: int, kernel_size: int, stride: int = 1,
                 padding: int = 0, dilation: int = 1, groups: int = 1, bias: bool = True,
                 backend: str = "hip"):
        nn.Conv1d.__init__(self, in_channels, out_channels, kernel_size, stride, padding, dilation,
                           groups, bias, device="meta")
        check_backend(backend)
        if dilation != 1 or groups != 1:
            raise NotImplementedError("Conv1d_int supports dilation 1 and groups 1")
        self.act_range = 127
        self.req_multiplier = nn.Parameter(torch.ones(1, dtype=torch.uint32), requires_grad=False)
        self.req_shiftmount = nn.Parameter(torch.zeros(1, dtype=torch.int8), requires_grad=False)
        self.weight = nn.Parameter(
            torch.ones((out_channels, in_channels * self.kernel_size[0]), dtype=torch.int8),
            requires_grad=False)
        if self.bias is not None:
            self.bias = nn.Parameter(torch.ones(out_channels, dtype=torch.int32), requires_grad=False)
        self.backend = backend
        self._wkc = None

    def _read_scalars(self):
        self._wkc = None
        return dict(m=_item(self.req_multiplier), s=_item(self.req_shiftmount))

    def weight_kc(self) -> Tensor:
        """Weight reordered to [Cout, K, Cin] for the channels-last implicit GEMM."""
        self._scalars()
        if self._wkc is None or self._wkc.device != self.weight.device:
            co, ks, ci = self.out_channels, self.kernel_size[0], self.in_channels
            self._wkc = self.weight.view(co, ci, ks).permute(0, 2, 1).contiguous().view(co, ks * ci)
        return self._wkc

    def _conv_forward(self, x: Tensor, weight: Tensor, bias: Optional[Tensor]) -> Tensor:
        assert x.dtype == torch.int8, "Input activation must be int8 in integer inference mode!"
        check_backend(self.backend)
        x = x.contiguous()
        B, Cin, Tin = x.shape
        ks, st, pd = self.kernel_size[0], self.stride[0], self.padding[0]
        tout = (Tin + 2 * pd - ks) // st + 1
        s = self._scalars()
        out = torch.empty((B, self.out_channels, tout), dtype=torch.int8, device=x.device)
        _lib.call("iw_conv1d", x.data_ptr(), weight.data_ptr(), _ptr(bias), s["m"], s["s"],
                  out.data_ptr(), B, Cin, Tin, self.out_channels, ks, st, pd, bias is not None,
                  _stream())
        return out

    def forward_cl(self, x_cl: Tensor, gelu: GELU_int, pe=None, pe_mult=None, pe_shift=None) -> Tensor:
        """Channels-last conv [B,Tin,Cin] -> GeLU -> optional positional add_requant15.

        Returns int8 [B,Tout,Cout], or int16 when ``pe`` is given.
        """
        B, Tin, Cin = x_cl.shape
        ks, st, pd = self.kernel_size[0], self.stride[0], self.padding[0]
        tout = (Tin + 2 * pd - ks) // st + 1
        s = self._scalars()
        wkc = self.weight_kc()
        lut, im, is_, om, os_, ci, co = gelu.gelu_ptrs()
        dt = torch.int8 if pe is None else torch.int16
        out = torch.empty((B, tout, self.out_channels), dtype=dt, device=x_cl.device)
        _lib.call("iw_conv1d_cl", x_cl.data_ptr(), wkc.data_ptr(), _ptr(self.bias), s["m"], s["s"],
                  lut, im, is_, om, os_, ci, co, _ptr(pe), _ptr(pe_mult), _ptr(pe_shift),
                  0 if pe_mult is None else pe_mult.numel(),
                  0 if pe_shift is None else pe_shift.numel(), out.data_ptr(), B, Cin, Tin,
                  self.out_channels, ks, st, pd, self.bias is not None, _stream())
        return out


# ---------------------------------------------------------------------------
# Attention
# ---------------------------------------------------------------------------

def pack_vt(v: Tensor, n_head: int, pad_to: int = 16) -> Tensor:
    """[B, Tk, H*D] int8 -> V^T per head [B, H, D, round_up(Tk, pad_to)] (padding is never read
    with a non-zero weight)."""
    B, Tk, C = v.shape
    D = C // n_head
    tp = (Tk + pad_to - 1) // pad_to * pad_to
    vt = torch.empty((B, n_head, D, tp), dtype=torch.int8, device=v.device)
    _lib.call("iw_transpose_heads", v.data_ptr(), v.stride(0), v.stride(1), vt.data_ptr(),
              n_head * D * tp, D * tp, tp, 4, 0, B, Tk, n_head, D, _stream())
    return vt


class MultiHeadAttention_int(_ScalarCache, nn.Module):
    """model_int.py:677-1060. ``forward`` returns the int32 out-projection as in the reference."""

    def __init__(self, n_state: int, n_head: int, backend: str = "hip"):
        super().__init__()
        check_backend(backend)
        self.n_state = n_state
        self.n_head = n_head
        self.backend = backend
        self.impl = "fused"
        self.act_range = 127
        self.qk_req_multiplier = nn.Parameter(torch.ones(1, dtype=torch.uint8), requires_grad=False)
        self.qk_req_shiftmount = nn.Parameter(torch.zeros(1, dtype=torch.int8), requires_grad=False)
        self.av_req_multiplier = nn.Parameter(torch.ones(1, dtype=torch.uint8), requires_grad=False)
        self.av_req_shiftmount = nn.Parameter(torch.zeros(1, dtype=torch.int8), requires_grad=False)
        self.register_buffer("qk_frac_bits", torch.tensor(7, dtype=torch.int32))
        self.rsqrt_offset = 16
        self.query = Linear8(n_state, n_state)
        self.key = Linear8(n_state, n_state, bias=False)
        self.value = Linear8(n_state, n_state)
        self.out = Linear32(n_state, n_state)
        self._table = None

    def _read_scalars(self):
        self._table = None
        f = _item(self.qk_frac_bits)
        if not 0 < f < 14:
            raise RuntimeError("frac_bits must be in [1, 14)")
        return dict(qm=_item(self.qk_req_multiplier), qs=_item(self.qk_req_shiftmount), f=f,
                    am=_item(self.av_req_multiplier), as_=_item(self.av_req_shiftmount))

    def shift_exp_table(self) -> Tensor:
        s = self._scalars()
        if self._table is None or self._table.device != self.qk_frac_bits.device:
            t = torch.empty(32768, dtype=torch.uint8, device=self.qk_frac_bits.device)
            _lib.call("iw_shift_exp_table", t.data_ptr(), s["f"], _stream())
            self._table = t
        return self._table

    def forward(self, x: Tensor, xa: Optional[Tensor] = None, mask: Optional[Tensor] = None,
                kv_cache: Optional[dict] = None):
        return self.out(self.attend(x, xa, mask, kv_cache))

    def attend(self, x: Tensor, xa: Optional[Tensor] = None, mask: Optional[Tensor] = None,
               kv_cache: Optional[dict] = None) -> Tensor:
        """Q/K/V projections and attention; int8 [B, Tq, n_state] (before the out-projection)."""
        q = self.query(x)
        if kv_cache is None or xa is None or self.key not in kv_cache:
            k = self.key(x if xa is None else xa)
            v = self.value(x if xa is None else xa)
        else:
            k = kv_cache[self.key]
            v = kv_cache[self.value]
        return self.qkv_attention(q, k, v, mask, kv_cache=kv_cache,
                                  is_cross_attention=(xa is not None))

    def qkv_attention(self, q: Tensor, k: Tensor, v: Tensor, mask: Optional[Tensor] = None,
                      kv_cache: Optional[dict] = None, is_cross_attention: bool = False) -> Tensor:
        check_backend(self.backend)
        q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
        B, Tq, C = q.shape
        Tk = k.shape[1]
        H = self.n_head
        D = C // H
        attn_mask = None
        if mask is not None:  # model_int.py:786-799
            q_offset = Tk - Tq
            assert q_offset >= 0
            attn_mask = mask[q_offset:q_offset + Tq, :Tk].contiguous()
        s = self._scalars()
        out = torch.empty((B, Tq, C), dtype=torch.int8, device=q.device)
        if D % 16 == 0 and D <= 128 and Tk <= 4096:
            vt_key = (self.value, "iwhisper_cross_vt_packed")
            if is_cross_attention and kv_cache is not None and vt_key in kv_cache:
                vt = kv_cache[vt_key]
            else:
                vt = pack_vt(v, H)
                if is_cross_attention and kv_cache is not None:
                    kv_cache[vt_key] = vt
            tp = vt.shape[-1]
            decode = Tq <= 8
            table = None if decode else self.shift_exp_table()
            _lib.call("iw_attention", q.data_ptr(), Tq * C, C, k.data_ptr(), Tk * C, D, C,
                      vt.data_ptr(), H * D * tp, D * tp, tp, out.data_ptr(), Tq * C, C,
                      _ptr(attn_mask), B, H, Tq, Tk, D, s["qm"], s["qs"], s["f"], s["am"],
                      s["as_"], self.rsqrt_offset, _ptr(table), decode, _stream())
            return out
        # Other head sizes: the three reference ops, each on the GPU.
        qh = q.view(B, Tq, H, D).permute(0, 2, 1, 3).contiguous()
        kh = k.view(B, Tk, H, D).permute(0, 2, 1, 3).contiguous()
        vh = v.view(B, Tk, H, D).permute(0, 2, 3, 1).contiguous()
        qk = torch.empty((B, H, Tq, Tk), dtype=torch.int16, device=q.device)
        rm = torch.empty((B, H, Tq, 1), dtype=torch.int16, device=q.device)
        p = torch.empty((B, H, Tq, Tk), dtype=torch.uint8, device=q.device)
        rs = torch.empty((B, H, Tq, 1), dtype=torch.int32, device=q.device)
        mp = _ptr(attn_mask)
        _lib.call("iw_qk_requant_rowmax", qh.data_ptr(), kh.data_ptr(), mp, qk.data_ptr(),
                  rm.data_ptr(), B, H, Tq, Tk, D, s["qm"], s["qs"], mp is not None, _stream())
        _lib.call("iw_shift_exp", qk.data_ptr(), rm.data_ptr(), mp, p.data_ptr(), rs.data_ptr(), B,
                  H, Tq, Tk, s["f"], mp is not None, _stream())
        _lib.call("iw_pv_norm_requant", p.data_ptr(), vh.data_ptr(), rs.data_ptr(), s["am"],
                  s["as_"], self.rsqrt_offset, out.data_ptr(), B, H, Tq, Tk, D, _stream())
        return out

    @staticmethod
    def copy_param(quant_layer):
        new = MultiHeadAttention_int(quant_layer.n_state, quant_layer.n_head)
        new.load_state_dict(quant_layer.state_dict())
        return new


class ResidualAttentionBlock_int(_ScalarCache, nn.Module):
    """model_int.py:1064-1211."""

    def __init__(self, n_state: int, n_head: int, cross_attention: bool = False, backend="hip"):
        super().__init__()
        check_backend(backend)
        self.backend = backend
        self.act_attn_bit = self.act_cross_attn_bit = self.act_mlp_bit = 15
        self.act_attn_range = self.act_cross_attn_range = self.act_mlp_range = 16383
        self.attn_res_req_multiplier = nn.Parameter(torch.ones(1, dtype=torch.uint16),
                                                    requires_grad=False)
        self.cross_attn_res_req_multiplier = nn.Parameter(torch.ones(1, dtype=torch.uint16),
                                                          requires_grad=False)
        self.mlp_res_req_multiplier = nn.Parameter(torch.ones(1, dtype=torch.uint16),
                                                   requires_grad=False)
        self.attn = MultiHeadAttention_int(n_state, n_head)
        self.attn_ln = LayerNorm_int(n_state)
        self.cross_attn = MultiHeadAttention_int(n_state, n_head) if cross_attention else None
        self.cross_attn_ln = LayerNorm_int(n_state) if cross_attention else None
        self.n_mlp = n_state * 4
        self.mlp = nn.Sequential(
            Linear8(n_state, self.n_mlp),
            GELU_int(channel_num=self.n_mlp, out_channel_num=self.n_mlp),
            Linear32(self.n_mlp, n_state),
        )
        self.mlp_ln = LayerNorm_int(n_state)

    def _read_scalars(self):
        return dict(a=_item(self.attn_res_req_multiplier),
                    c=_item(self.cross_attn_res_req_multiplier),
                    m=_item(self.mlp_res_req_multiplier))

    def mlp_gelu(self, h: Tensor) -> Tensor:
        """mlp[0] (Linear8) and mlp[1] (GELU_int) in one kernel."""
        fc1, gelu = self.mlp[0], self.mlp[1]
        h, M, (w, b, z, m, s) = fc1._gemm_args(h)
        lut, im, is_, om, os_, ci, co = gelu.gelu_ptrs()
        out = torch.empty((*h.shape[:-1], fc1.out_features), dtype=torch.int8, device=h.device)
        _lib.call("iw_linear8_gelu", h.data_ptr(), w, b, z, m, s, lut, im, is_, om, os_, ci, co,
                  out.data_ptr(), M, fc1.in_features, fc1.out_features, b is not None,
                  z is not None, _stream())
        return out

    def forward(self, x: Tensor, xa: Optional[Tensor] = None, mask: Optional[Tensor] = None,
                kv_cache: Optional[dict] = None):
        check_backend(self.backend)
        assert x.dtype == torch.int16, "residual tensor must be int16 in integer inference mode!"
        sc = self._scalars()
        x = x.contiguous()
        wv = self.attn.attend(self.attn_ln.normalize(x), mask=mask, kv_cache=kv_cache)
        x = self.attn.out.forward_residual15(wv, x, sc["a"])
        if self.cross_attn is not None:
            wv = self.cross_attn.attend(self.cross_attn_ln.normalize(x), xa, kv_cache=kv_cache)
            x = self.cross_attn.out.forward_residual15(wv, x, sc["c"])
        h = self.mlp_gelu(self.mlp_ln.normalize(x))
        return self.mlp[2].forward_residual15(h, x, sc["m"])

    @staticmethod
    def copy_param(quant_layer):
        new = ResidualAttentionBlock_int(quant_layer.attn_ln.normalized_shape[0],
                                         quant_layer.attn.n_head,
                                         cross_attention=quant_layer.cross_attn is not None)
        new.load_state_dict(quant_layer.state_dict())
        return new


# ---------------------------------------------------------------------------
# Encoder / decoder / model
# ---------------------------------------------------------------------------

class AudioEncoder_int(nn.Module):
    """model_int.py:1215-1340."""

    def __init__(self, n_mels: int, n_ctx: int, n_state: int, n_head: int, n_layer: int,
                 backend: str = "hip"):
        super().__init__()
        check_backend(backend)
        self.n_mels, self.n_ctx, self.n_state, self.n_head, self.n_layer = (
            n_mels, n_ctx, n_state, n_head, n_layer)
        self.backend = backend
        self.act_pe_bit = 8
        self.act_pe_range = 127
        self.act_range = 16383
        self.req_multiplier = nn.Parameter(torch.ones(n_state, dtype=torch.uint16), requires_grad=False)
        self.req_shiftmount = nn.Parameter(torch.zeros(n_state, dtype=torch.int8), requires_grad=False)
        self.register_buffer("positional_embedding", torch.zeros((n_ctx, n_state), dtype=torch.int8))
        self.input_alpha = nn.Parameter(torch.ones(1))
        self.gelu1 = GELU_int()
        self.gelu2 = GELU_int(out_channel_num=self.n_state)
        self.conv1 = Conv1d_int(n_mels, n_state, kernel_size=3, padding=1)
        self.conv2 = Conv1d_int(n_state, n_state, kernel_size=3, stride=2, padding=1)
        self.blocks: Iterable[ResidualAttentionBlock_int] = nn.ModuleList(
            [ResidualAttentionBlock_int(n_state, n_head) for _ in range(n_layer)])
        self.ln_post = LayerNorm_int(n_state)
        self._alpha = None

    def _apply(self, fn, *args, **kwargs):
        self._alpha = None
        return super()._apply(fn, *args, **kwargs)

    def _load_from_state_dict(self, *args, **kwargs):
        self._alpha = None
        return super()._load_from_state_dict(*args, **kwargs)

    def quantize_input(self, mel: Tensor) -> Tensor:
        """round(mel * input_alpha) clamped to +-127, channels-last [B, T, n_mels] int8
        (model_int.py:1265-1267)."""
        if self._alpha is None:
            self._alpha = float(self.input_alpha.detach().reshape(-1)[0].item())
        mel = mel.contiguous()
        if mel.dtype != torch.float32:
            raise RuntimeError("mel must be float32 (or int8 already quantised)")
        B, M, T = mel.shape
        out = torch.empty((B, T, M), dtype=torch.int8, device=mel.device)
        _lib.call("iw_quantize_mel", mel.data_ptr(), self._alpha, out.data_ptr(), B, M, T, _stream())
        return out

    def frontend(self, x: Tensor) -> Tensor:
        """mel -> conv1 -> GeLU -> conv2 -> GeLU -> + positional -> int16 [B, n_ctx, n_state]."""
        check_backend(self.backend)
        if x.dtype != torch.int8:
            x_cl = self.quantize_input(x)
        else:
            x_cl = x.permute(0, 2, 1).contiguous()
        if self.n_mels % 16 == 0 and self.n_state % 16 == 0:
            c1 = self.conv1.forward_cl(x_cl, self.gelu1)
            x16 = self.conv2.forward_cl(c1, self.gelu2, self.positional_embedding,
                                        self.req_multiplier, self.req_shiftmount)
        else:  # same ops unfused, NCT layout as in the reference
            c1 = self.gelu1(self.conv1(x_cl.permute(0, 2, 1).contiguous()))
            c2 = self.gelu2(self.conv2(c1).permute(0, 2, 1).contiguous())
            x16 = torch.empty(c2.shape, dtype=torch.int16, device=c2.device)
            B, T, C = c2.shape
            _lib.call("iw_add_requant15", c2.data_ptr(), self.positional_embedding.data_ptr(),
                      self.req_multiplier.data_ptr(), self.req_shiftmount.data_ptr(), x16.data_ptr(),
                      B, T, C, self.req_multiplier.numel(), self.req_shiftmount.numel(), _stream())
        assert x16.shape[1:] == self.positional_embedding.shape, "incorrect audio shape"
        return x16

    def forward(self, x: Tensor) -> Tensor:
        x = self.frontend(x)
        for block in self.blocks:
            x = block(x)
        return self.ln_post.normalize(x)

    @staticmethod
    def copy_param(quant_layer):
        new = AudioEncoder_int(quant_layer.n_mels, quant_layer.n_ctx, quant_layer.n_state,
                               quant_layer.n_head, quant_layer.n_layer)
        new.load_state_dict(quant_layer.state_dict())
        return new


class TextDecoder_int(nn.Module):
    """model_int.py:1344-1508."""

    def __init__(self, n_vocab: int, n_ctx: int, n_state: int, n_head: int, n_layer: int,
                 backend: str = "hip"):
        super().__init__()
        check_backend(backend)
        self.n_vocab, self.n_ctx, self.n_state, self.n_head, self.n_layer = (
            n_vocab, n_ctx, n_state, n_head, n_layer)
        self.backend = backend
        self.dequant_need = True
        self.logit_range = 127
        self.act_range = 16383
        self.req_multiplier = nn.Parameter(torch.ones(1, dtype=torch.uint8), requires_grad=False)
        self.req_shiftmount = nn.Parameter(torch.zeros(1, dtype=torch.int8), requires_grad=False)
        self.clf_req_multiplier = nn.Parameter(torch.ones(1, dtype=torch.uint32), requires_grad=False)
        self.clf_req_shiftmount = nn.Parameter(torch.zeros(1, dtype=torch.int8), requires_grad=False)
        self.act_logits_alpha = nn.Parameter(torch.ones(1))
        self.token_embedding = nn.Embedding(n_vocab, n_state, device="meta")
        self.token_embedding.weight = nn.Parameter(torch.zeros((n_vocab, n_state), dtype=torch.int8),
                                                   requires_grad=False)
        self.positional_embedding = nn.Parameter(torch.zeros((n_ctx, n_state), dtype=torch.int8),
                                                 requires_grad=False)
        self.blocks: Iterable[ResidualAttentionBlock_int] = nn.ModuleList(
            [ResidualAttentionBlock_int(n_state, n_head, cross_attention=True)
             for _ in range(n_layer)])
        self.ln = LayerNorm_int(n_state)
        mask = torch.ones((n_ctx, n_ctx), dtype=torch.bool).triu_(1)
        self.register_buffer("mask", mask, persistent=False)
        self._scal = None

    def _apply(self, fn, *args, **kwargs):
        self._scal = None
        return super()._apply(fn, *args, **kwargs)

    def _load_from_state_dict(self, *args, **kwargs):
        self._scal = None
        return super()._load_from_state_dict(*args, **kwargs)

    def scalars(self) -> dict:
        if self._scal is None:
            dev = self.req_multiplier.device
            self._scal = dict(
                m16=self.req_multiplier.detach().cpu().to(torch.int32).to(torch.uint16).to(dev),
                s=self.req_shiftmount, cm=_item(self.clf_req_multiplier),
                cs=_item(self.clf_req_shiftmount),
                alpha=float(self.act_logits_alpha.detach().reshape(-1)[0].item()))
        return self._scal

    def embed(self, tokens: Tensor, offset: int) -> Tensor:
        """Token gather + positional add_requant15 -> int16 [B, T, n_state] (model_int.py:1411-1439)."""
        if tokens.dtype != torch.int64:
            tokens = tokens.to(torch.int64)
        tokens = tokens.contiguous()
        B, T = tokens.shape
        if offset + T > self.n_ctx:
            raise RuntimeError("sequence longer than n_text_ctx")
        sc = self.scalars()
        out = torch.empty((B, T, self.n_state), dtype=torch.int16, device=tokens.device)
        _lib.call("iw_embed_add_requant15", tokens.data_ptr(), self.token_embedding.weight.data_ptr(),
                  self.positional_embedding.data_ptr(), offset, sc["m16"].data_ptr(),
                  sc["s"].data_ptr(), out.data_ptr(), B, T, self.n_state, _stream())
        return out

    def classify(self, h: Tensor) -> Tensor:
        """int8 logits before dequant (model_int.py:1446-1469; classifier_scalar.cpp:91-142)."""
        sc = self.scalars()
        h = h.contiguous()
        B, T, C = h.shape
        out = torch.empty((B, T, self.n_vocab), dtype=torch.int8, device=h.device)
        _lib.call("iw_classifier", h.data_ptr(), self.token_embedding.weight.data_ptr(), sc["cm"],
                  sc["cs"], out.data_ptr(), B * T, C, self.n_vocab, _stream())
        return out

    def forward(self, x: Tensor, xa: Tensor, kv_cache: Optional[dict] = None):
        check_backend(self.backend)
        offset = next(iter(kv_cache.values())).shape[1] if kv_cache else 0
        if x.numel() and (int(x.min()) < 0 or int(x.max()) >= self.n_vocab):
            raise RuntimeError("token id out of range")
        x = self.embed(x, offset)
        for block in self.blocks:
            x = block(x, xa, mask=self.mask, kv_cache=kv_cache)
        logits = self.classify(self.ln.normalize(x))
        if self.dequant_need:
            return logits.float().div(self.act_logits_alpha.detach())
        return logits

    @staticmethod
    def copy_param(quant_layer):
        new = TextDecoder_int(quant_layer.n_vocab, quant_layer.n_ctx, quant_layer.n_state,
                              quant_layer.n_head, quant_layer.n_layer)
        new.load_state_dict(quant_layer.state_dict())
        return new


QUANT_MODULES = [Conv1d_int, GELU_int, LayerNorm_int, AudioEncoder_int, TextDecoder_int,
                 ResidualAttentionBlock_int, MultiHeadAttention_int]


class Whisper_int(nn.Module):
    """model_int.py:1524-1622."""

    def __init__(self, dims: ModelDimensions):
        super().__init__()
        self.dims = dims
        self.encoder = AudioEncoder_int(dims.n_mels, dims.n_audio_ctx, dims.n_audio_state,
                                        dims.n_audio_head, dims.n_audio_layer)
        self.decoder = TextDecoder_int(dims.n_vocab, dims.n_text_ctx, dims.n_text_state,
                                       dims.n_text_head, dims.n_text_layer)
        all_heads = torch.zeros(dims.n_text_layer, dims.n_text_head, dtype=torch.bool)
        all_heads[dims.n_text_layer // 2:] = True
        self.register_buffer("alignment_heads", all_heads.to_sparse(), persistent=False)

    @classmethod
    def from_params(cls, dims: ModelDimensions, params: Dict[str, np.ndarray]) -> "Whisper_int":
        """Build from a name -> numpy array mapping with the reference's state-dict keys."""
        model = cls(dims)
        sd = {k: torch.from_numpy(np.ascontiguousarray(v)) for k, v in params.items()}
        model.load_state_dict(sd, strict=True)
        return model

    def set_alignment_heads(self, dump: bytes):
        array = np.frombuffer(gzip.decompress(base64.b85decode(dump)), dtype=bool).copy()
        mask = torch.from_numpy(array).reshape(self.dims.n_text_layer, self.dims.n_text_head)
        self.register_buffer("alignment_heads", mask.to_sparse(), persistent=False)

    def embed_audio(self, mel: Tensor):
        return self.encoder(mel)

    def logits(self, tokens: Tensor, audio_features: Tensor):
        return self.decoder(tokens, audio_features)

    def forward(self, mel: Tensor, tokens: Tensor) -> Tensor:
        return self.decoder(tokens, self.encoder(mel))

    @property
    def device(self):
        return next(self.parameters()).device

    @property
    def is_multilingual(self):
        return self.dims.n_vocab >= 51865

    @property
    def num_languages(self):
        return self.dims.n_vocab - 51765 - int(self.is_multilingual)

    def install_kv_cache_hooks(self, cache: Optional[dict] = None):
        """model_int.py:1575-1618: forward hooks on key/value projections that
        concatenate new keys/values to the cache along the time axis."""
        cache = {**cache} if cache is not None else {}
        hooks = []

        def save_to_cache(module, _, output):
            if module not in cache or output.shape[1] > self.dims.n_text_ctx:
                cache[module] = output
            else:
                cache[module] = torch.cat([cache[module], output], dim=1).detach()
            return cache[module]

        def install_hooks(layer: nn.Module):
            if isinstance(layer, MultiHeadAttention_int):
                hooks.append(layer.key.register_forward_hook(save_to_cache))
                hooks.append(layer.value.register_forward_hook(save_to_cache))

        self.decoder.apply(install_hooks)
        return cache, hooks


# ---------------------------------------------------------------------------
# backend switches (model_int.py:1626-1856)
# ---------------------------------------------------------------------------

def _switch(model: nn.Module, cls, label: str, backend: str, logger: Optional[Logger]):
    check_backend(backend)
    log = logger.debug if logger is not None else (lambda *_: None)
    for name, layer in model.named_modules():
        if isinstance(layer, cls):
            if layer.backend == backend:
                log(f"{label} backend for {name} is already set to {backend}.")
            else:
                log(f"{label} backend for {name} set to {backend}.")
                layer.backend = backend


def set_residual_backend(model, backend, logger=None):
    _switch(model, ResidualAttentionBlock_int, "Residual", backend, logger)


def set_layernorm_backend(model, backend, logger=None):
    _switch(model, LayerNorm_int, "LayerNorm", backend, logger)


def set_gelu_backend(model, backend, logger=None):
    _switch(model, GELU_int, "GeLU", backend, logger)


def set_attention_backend(model, backend, logger=None):
    _switch(model, MultiHeadAttention_int, "Attention", backend, logger)


def set_conv1d_backend(model, backend, logger=None):
    _switch(model, Conv1d_int, "Conv1d", backend, logger)


def set_encoder_backend(model, backend, logger=None):
    _switch(model, AudioEncoder_int, "Encoder", backend, logger)


def set_decoder_backend(model, backend, logger=None):
    _switch(model, TextDecoder_int, "Decoder", backend, logger)


def set_all_backends(model, backend: str = "hip", logger=None):
    from .linear import set_linear8_backend, set_linear32_backend

    for fn in (set_residual_backend, set_layernorm_backend, set_gelu_backend,
               set_attention_backend, set_conv1d_backend, set_encoder_backend,
               set_decoder_backend, set_linear8_backend, set_linear32_backend):
        fn(model, backend, logger)


assert BACKENDS == ("hip",)
