"""Tensor-level ops over the gfx950 kernels: the MI355X counterpart of the
reference's ``i_whisper.kernels._C`` module (i_whisper/kernels/csrc/pybind.cpp:45-415).

Each ``<op>_hip`` takes and returns torch tensors on the GPU and keeps the
reference binding's contract: same argument order and meaning, scalar
parameters as one-element tensors, outputs allocated and returned, and
``RuntimeError`` for wrong dtype / shape / contiguity (the reference's
TORCH_CHECKs in csrc/<op>/<op>_torch.cpp). Work is queued on the current
torch stream; nothing runs on the CPU.
"""
from __future__ import annotations

from typing import Optional

import torch

from . import _lib

Tensor = torch.Tensor


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _check(t: Tensor, dtype: torch.dtype, name: str) -> None:
    if not isinstance(t, torch.Tensor):
        raise RuntimeError(f"{name} must be a tensor")
    if t.device.type != "cuda":
        raise RuntimeError(f"{name} must be a GPU tensor, got device {t.device}")
    if t.dtype != dtype:
        raise RuntimeError(f"{name} must be {str(dtype).replace('torch.', '')}, got {t.dtype}")
    if not t.is_contiguous():
        raise RuntimeError(f"{name} must be contiguous")


def _ptr(t: Optional[Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _check_scalar(t: Tensor, dtype: torch.dtype, name: str) -> None:
    """Scalar parameters may live on the host or the GPU (read once per call)."""
    if not isinstance(t, torch.Tensor):
        raise RuntimeError(f"{name} must be a tensor")
    if t.dtype != dtype:
        raise RuntimeError(f"{name} must be {str(dtype).replace('torch.', '')}, got {t.dtype}")


def _host_scalar(t: Tensor, name: str) -> int:
    if t.numel() != 1:
        raise RuntimeError(f"{name} must be a scalar tensor")
    return int(t.reshape(-1)[0].item())


# ---------------------------------------------------------------------------
# GEMM family
# ---------------------------------------------------------------------------

def _linear_checks(x, weight, bias, weight_zero, multiplier, shift):
    """linear8/linear8_torch.cpp:22-108 (shared by linear32_torch.cpp)."""
    _check(x, torch.int8, "x")
    _check(weight, torch.int8, "weight")
    _check(multiplier, torch.uint32, "multiplier")
    _check(shift, torch.int8, "shift")
    if x.dim() < 1:
        raise RuntimeError("x must have at least 1 dimension")
    if weight.dim() != 2:
        raise RuntimeError(f"weight must have 2 dimensions, got {weight.dim()}")
    if multiplier.dim() != 1:
        raise RuntimeError(f"multiplier should be a 1D tensor, got {multiplier.dim()}")
    if shift.dim() != 1:
        raise RuntimeError(f"shift should be a 1D tensor, got {shift.dim()}")
    K = x.size(-1)
    if K <= 0:
        raise RuntimeError("x.size(-1) must be greater than 0")
    N = weight.size(0)
    if weight.size(1) != K:
        raise RuntimeError(f"weight.size(1) must equal x.size(-1), expected {K}, got {weight.size(1)}")
    if N != multiplier.numel():
        raise RuntimeError(f"weight.size(0) must equal multiplier's number of elements, expected {N}, "
                           f"got {multiplier.numel()}")
    if multiplier.numel() != shift.numel():
        raise RuntimeError("multiplier's number of elements must equal shift's number of elements")
    if bias is not None:
        _check(bias, torch.int32, "bias")
        if bias.dim() != 1:
            raise RuntimeError(f"bias must be a 1D tensor, got {bias.dim()}")
        if bias.size(0) != N:
            raise RuntimeError(f"bias.size(0) must equal weight.size(0), got {bias.size(0)} expected {N}")
    if weight_zero is not None:
        _check(weight_zero, torch.int8, "weight_zero")
        if weight_zero.dim() != 1:
            raise RuntimeError(f"weight_zero must be a 1D tensor, got {weight_zero.dim()}")
        if weight_zero.size(0) != N:
            raise RuntimeError(f"weight_zero.size(0) must equal weight.size(0), got {weight_zero.size(0)} "
                               f"expected {N}")
    return x.numel() // K, K, N


def linear8_hip(x, weight, bias, weight_zero, multiplier, shift) -> Tensor:
    """Counterpart of _C.linear8_simd (linear8/linear8_torch.cpp:14-152)."""
    M, K, N = _linear_checks(x, weight, bias, weight_zero, multiplier, shift)
    out = torch.empty((*x.shape[:-1], N), dtype=torch.int8, device=x.device)
    _lib.call("iw_linear8", x.data_ptr(), weight.data_ptr(), _ptr(bias), _ptr(weight_zero),
              multiplier.data_ptr(), shift.data_ptr(), out.data_ptr(), M, K, N,
              bias is not None, weight_zero is not None, _stream())
    return out


def linear32_hip(x, weight, bias, weight_zero, multiplier, shift) -> Tensor:
    """Counterpart of _C.linear32_simd (linear32/linear32_torch.cpp:10-150)."""
    M, K, N = _linear_checks(x, weight, bias, weight_zero, multiplier, shift)
    out = torch.empty((*x.shape[:-1], N), dtype=torch.int32, device=x.device)
    _lib.call("iw_linear32", x.data_ptr(), weight.data_ptr(), _ptr(bias), _ptr(weight_zero),
              multiplier.data_ptr(), shift.data_ptr(), out.data_ptr(), M, K, N,
              bias is not None, weight_zero is not None, _stream())
    return out


def _gelu_param_checks(channels, lut, luti_multiplier, luti_shift, luto_multiplier, luto_shift):
    """gelu/gelu_torch.cpp:18-112."""
    _check(lut, torch.uint8, "lut")
    _check(luti_multiplier, torch.uint8, "luti_multiplier")
    _check(luti_shift, torch.int8, "luti_shift")
    _check(luto_multiplier, torch.uint8, "luto_multiplier")
    _check(luto_shift, torch.int8, "luto_shift")
    if lut.dim() != 1 or lut.numel() != 16:
        raise RuntimeError("lut must contain exactly 16 entries")
    for t, n in ((luti_multiplier, "luti_multiplier"), (luti_shift, "luti_shift"),
                 (luto_multiplier, "luto_multiplier"), (luto_shift, "luto_shift")):
        if t.dim() != 1:
            raise RuntimeError(f"{n} must be 1D")
    if luti_multiplier.numel() != luti_shift.numel():
        raise RuntimeError("luti multiplier/shift size mismatch")
    if luto_multiplier.numel() != luto_shift.numel():
        raise RuntimeError("luto multiplier/shift size mismatch")
    if luti_multiplier.numel() not in (1, channels):
        raise RuntimeError("luti parameters must be scalar or match input.size(-1)")
    if luto_multiplier.numel() not in (1, channels):
        raise RuntimeError("luto parameters must be scalar or match input.size(-1)")
    return luti_multiplier.numel(), luto_multiplier.numel()


def linear8_gelu_hip(x, weight, bias, weight_zero, multiplier, shift, lut, luti_multiplier,
                     luti_shift, luto_multiplier, luto_shift) -> Tensor:
    """Linear8 followed by GELU_int in one kernel (model_int.py:1103-1107)."""
    M, K, N = _linear_checks(x, weight, bias, weight_zero, multiplier, shift)
    ci, co = _gelu_param_checks(N, lut, luti_multiplier, luti_shift, luto_multiplier, luto_shift)
    out = torch.empty((*x.shape[:-1], N), dtype=torch.int8, device=x.device)
    _lib.call("iw_linear8_gelu", x.data_ptr(), weight.data_ptr(), _ptr(bias), _ptr(weight_zero),
              multiplier.data_ptr(), shift.data_ptr(), lut.data_ptr(), luti_multiplier.data_ptr(),
              luti_shift.data_ptr(), luto_multiplier.data_ptr(), luto_shift.data_ptr(), ci, co,
              out.data_ptr(), M, K, N, bias is not None, weight_zero is not None, _stream())
    return out


def linear32_residual15_hip(x, weight, bias, weight_zero, multiplier, shift, residual,
                            residual_multiplier, out: Optional[Tensor] = None) -> Tensor:
    """Linear32 then residual15 with ``residual`` in one kernel (model_int.py:1126-1169).

    ``out`` may be ``residual`` itself (in-place update of the residual stream).
    """
    M, K, N = _linear_checks(x, weight, bias, weight_zero, multiplier, shift)
    _check(residual, torch.int16, "residual")
    if residual.shape != (*x.shape[:-1], N):
        raise RuntimeError("branch and residual must have the same shape")
    m = _host_scalar(residual_multiplier, "multiplier")
    if out is None:
        out = torch.empty_like(residual)
    _lib.call("iw_linear32_residual15", x.data_ptr(), weight.data_ptr(), _ptr(bias),
              _ptr(weight_zero), multiplier.data_ptr(), shift.data_ptr(), residual.data_ptr(), m,
              out.data_ptr(), M, K, N, bias is not None, weight_zero is not None, _stream())
    return out


def classifier_hip(input, weight, multiplier, shift) -> Tensor:
    """Counterpart of _C.classifier_simd (classifier/classifier_torch.cpp:145-212)."""
    _check(input, torch.int8, "input")
    _check(weight, torch.int8, "weight")
    if input.dim() != 3:
        raise RuntimeError("input must be [B,T,K]")
    if weight.dim() != 2:
        raise RuntimeError("weight must be [N,K]")
    B, T, K = input.shape
    N = weight.size(0)
    if weight.size(1) != K:
        raise RuntimeError("weight hidden size must match input")
    if K <= 0:
        raise RuntimeError("hidden size must be positive")
    if N <= 0:
        raise RuntimeError("vocabulary size must be positive")
    _check_scalar(multiplier, torch.uint32, "multiplier")
    _check_scalar(shift, torch.int8, "shift")
    if multiplier.numel() != 1:
        raise RuntimeError("multiplier must contain exactly one element")
    if shift.numel() != 1:
        raise RuntimeError("shift must contain exactly one element")
    out = torch.empty((B, T, N), dtype=torch.int8, device=input.device)
    _lib.call("iw_classifier", input.data_ptr(), weight.data_ptr(), _host_scalar(multiplier, "multiplier"),
              _host_scalar(shift, "shift"), out.data_ptr(), B * T, K, N, _stream())
    return out


def conv1d_hip(input, weight, bias, multiplier, shift, stride: int, padding: int) -> Tensor:
    """Counterpart of _C.conv1d_simd (conv1d/conv1d_torch.cpp:243-340); weight [Cout, Cin*K]."""
    _check(input, torch.int8, "input")
    _check(weight, torch.int8, "weight")
    if input.dim() != 3:
        raise RuntimeError("input must be [B,Cin,Tin]")
    if weight.dim() != 2:
        raise RuntimeError("weight must be [Cout, Cin*K]")
    B, Cin, Tin = input.shape
    Cout = weight.size(0)
    if weight.size(1) % Cin != 0 or weight.size(1) == 0:
        raise RuntimeError("weight.size(1) must be a positive multiple of Cin")
    ks = weight.size(1) // Cin
    if stride <= 0:
        raise RuntimeError("stride must be positive")
    if padding < 0:
        raise RuntimeError("padding must be non-negative")
    if Tin + 2 * padding < ks:
        raise RuntimeError("input too short for the kernel")
    if bias is not None:
        _check(bias, torch.int32, "bias")
        if bias.numel() != Cout:
            raise RuntimeError("bias must have Cout elements")
    _check_scalar(multiplier, torch.uint32, "multiplier")
    _check_scalar(shift, torch.int8, "shift")
    if multiplier.numel() != 1:
        raise RuntimeError("multiplier must contain exactly one element")
    if shift.numel() != 1:
        raise RuntimeError("shift must contain exactly one element")
    tout = (Tin + 2 * padding - ks) // stride + 1
    out = torch.empty((B, Cout, tout), dtype=torch.int8, device=input.device)
    _lib.call("iw_conv1d", input.data_ptr(), weight.data_ptr(), _ptr(bias),
              _host_scalar(multiplier, "multiplier"), _host_scalar(shift, "shift"), out.data_ptr(),
              B, Cin, Tin, Cout, ks, stride, padding, bias is not None, _stream())
    return out


# ---------------------------------------------------------------------------
# Row / element ops
# ---------------------------------------------------------------------------

LN_WIDTHS = (384, 512, 768, 1024, 1280)
LN_RSQRT_OFFSET = 13  # layernorm/layernorm_torch.cpp:266


def layernorm32_hip(input, weight, bias, ln_multiplier, ln_shift, out_multiplier, out_shift) -> Tensor:
    """Counterpart of _C.layernorm32_simd (layernorm/layernorm_torch.cpp:200-305)."""
    _check(input, torch.int16, "input")
    _check(weight, torch.int8, "weight")
    _check_scalar(ln_multiplier, torch.uint8, "ln_multiplier")
    _check_scalar(ln_shift, torch.int8, "ln_shift")
    _check_scalar(out_multiplier, torch.uint32, "out_multiplier")
    _check_scalar(out_shift, torch.int8, "out_shift")
    if input.dim() < 1:
        raise RuntimeError("input must have at least one dimension")
    if weight.dim() != 1:
        raise RuntimeError("weight must be a 1D tensor")
    H = input.size(-1)
    if H not in LN_WIDTHS:
        raise RuntimeError(f"unsupported LayerNorm hidden size: {H}")
    if weight.numel() != H:
        raise RuntimeError(f"weight.numel() must equal input.size(-1), got {weight.numel()} expected {H}")
    if bias is not None:
        _check(bias, torch.int32, "bias")
        if bias.dim() != 1:
            raise RuntimeError("bias must be a 1D tensor")
        if bias.numel() != H:
            raise RuntimeError(f"bias.numel() must equal input.size(-1), got {bias.numel()} expected {H}")
    out = torch.empty_like(input, dtype=torch.int8)
    _lib.call("iw_layernorm32", input.data_ptr(), weight.data_ptr(), _ptr(bias),
              _host_scalar(ln_multiplier, "ln_multiplier"), _host_scalar(ln_shift, "ln_shift"),
              _host_scalar(out_multiplier, "out_multiplier"), _host_scalar(out_shift, "out_shift"),
              LN_RSQRT_OFFSET, out.data_ptr(), input.numel() // H, H, bias is not None, _stream())
    return out


def layernorm32_rsqrt_hip(variance, offset: int = LN_RSQRT_OFFSET) -> Tensor:
    """Counterpart of _C.layernorm32_rsqrt_scalar (pybind.cpp:195-199)."""
    _check(variance, torch.int32, "variance")
    if not 0 <= offset <= 29:
        raise RuntimeError("rsqrt_offset must be in [0,29]")
    out = torch.empty_like(variance)
    _lib.call("iw_layernorm32_rsqrt", variance.data_ptr(), out.data_ptr(), variance.numel(), offset,
              _stream())
    return out


def gelu_hip(input, lut, luti_multiplier, luti_shift, luto_multiplier, luto_shift) -> Tensor:
    """Counterpart of _C.gelu_simd (gelu/gelu_torch.cpp:9-153)."""
    _check(input, torch.int8, "input")
    if input.dim() < 1:
        raise RuntimeError("input must have at least one dimension")
    C = input.size(-1)
    ci, co = _gelu_param_checks(C, lut, luti_multiplier, luti_shift, luto_multiplier, luto_shift)
    out = torch.empty_like(input)
    if input.numel() == 0:
        return out
    _lib.call("iw_gelu", input.data_ptr(), lut.data_ptr(), luti_multiplier.data_ptr(),
              luti_shift.data_ptr(), luto_multiplier.data_ptr(), luto_shift.data_ptr(),
              out.data_ptr(), input.numel(), C, ci, co, _stream())
    return out


def residual15_hip(branch, residual, multiplier) -> Tensor:
    """Counterpart of _C.residual15_simd (residual15/residual15_torch.cpp:7-70)."""
    _check(branch, torch.int32, "branch")
    _check(residual, torch.int16, "residual")
    _check_scalar(multiplier, torch.uint16, "multiplier")
    if multiplier.numel() != 1:
        raise RuntimeError("multiplier must be a scalar tensor")
    if residual.shape != branch.shape:
        raise RuntimeError("branch and residual must have the same shape")
    out = torch.empty_like(residual)
    _lib.call("iw_residual15", branch.data_ptr(), residual.data_ptr(),
              _host_scalar(multiplier, "multiplier"), out.data_ptr(), branch.numel(), _stream())
    return out


def add_requant15_hip(input, addend, multiplier, shift) -> Tensor:
    """Counterpart of _C.add_requant15_simd (add_requant15/add_requant15_torch.cpp:8-77)."""
    _check(input, torch.int8, "input")
    _check(addend, torch.int8, "addend")
    _check(multiplier, torch.uint16, "multiplier")
    _check(shift, torch.int8, "shift")
    if input.dim() != 3:
        raise RuntimeError("input must be [B,T,C]")
    if addend.dim() != 2:
        raise RuntimeError("addend must be [T,C]")
    B, T, C = input.shape
    if addend.shape != (T, C):
        raise RuntimeError("addend must match input [T,C]")
    if multiplier.dim() != 1:
        raise RuntimeError("multiplier must be 1D")
    if shift.dim() != 1:
        raise RuntimeError("shift must be 1D")
    if multiplier.numel() not in (1, C):
        raise RuntimeError("multiplier must contain 1 or C elements")
    if shift.numel() not in (1, C):
        raise RuntimeError("shift must contain 1 or C elements")
    out = torch.empty((B, T, C), dtype=torch.int16, device=input.device)
    _lib.call("iw_add_requant15", input.data_ptr(), addend.data_ptr(), multiplier.data_ptr(),
              shift.data_ptr(), out.data_ptr(), B, T, C, multiplier.numel(), shift.numel(), _stream())
    return out


# ---------------------------------------------------------------------------
# Attention ops
# ---------------------------------------------------------------------------

def _mask_check(mask, tq, tk, msg="mask must be [Tq,Tk]"):
    if mask is None:
        return None
    _check(mask, torch.bool, "mask")
    if mask.dim() != 2 or mask.size(0) != tq or mask.size(1) != tk:
        raise RuntimeError(msg)
    return mask.data_ptr()


def qk_requant_rowmax_hip(q, k, mask, multiplier, shift):
    """Counterpart of _C.qk_requant_rowmax_simd (attention/attention_torch.cpp:117-229)."""
    _check(q, torch.int8, "q")
    _check(k, torch.int8, "k")
    _check_scalar(multiplier, torch.uint8, "multiplier")
    _check_scalar(shift, torch.int8, "shift")
    if q.dim() != 4:
        raise RuntimeError("q must be [B,H,Tq,D]")
    if k.dim() != 4:
        raise RuntimeError("k must be [B,H,Tk,D]")
    if q.size(0) != k.size(0):
        raise RuntimeError("batch mismatch")
    if q.size(1) != k.size(1):
        raise RuntimeError("head count mismatch")
    if q.size(3) != k.size(3):
        raise RuntimeError("head dimension mismatch")
    if multiplier.numel() != 1:
        raise RuntimeError("multiplier must be a scalar tensor")
    if shift.numel() != 1:
        raise RuntimeError("shift must be a scalar tensor")
    B, H, Tq, D = q.shape
    Tk = k.size(2)
    if mask is not None:
        _check(mask, torch.bool, "mask")
        if mask.dim() != 2:
            raise RuntimeError("mask must be [Tq,Tk]")
        if mask.size(0) != Tq:
            raise RuntimeError("mask.size(0) must equal Tq")
        if mask.size(1) != Tk:
            raise RuntimeError("mask.size(1) must equal Tk")
    qk = torch.empty((B, H, Tq, Tk), dtype=torch.int16, device=q.device)
    rmax = torch.empty((B, H, Tq, 1), dtype=torch.int16, device=q.device)
    _lib.call("iw_qk_requant_rowmax", q.data_ptr(), k.data_ptr(), _ptr(mask), qk.data_ptr(),
              rmax.data_ptr(), B, H, Tq, Tk, D, _host_scalar(multiplier, "multiplier"),
              _host_scalar(shift, "shift"), mask is not None, _stream())
    return qk, rmax


def shift_exp_hip(input, row_max_plus1, mask, frac_bits):
    """Counterpart of _C.shift_exp_simd (attention/attention_torch.cpp:266-369)."""
    _check(input, torch.int16, "input")
    _check(row_max_plus1, torch.int16, "row_max_plus1")
    if frac_bits.dtype != torch.int32:
        raise RuntimeError(f"frac_bits must be int32, got {frac_bits.dtype}")
    if input.dim() != 4:
        raise RuntimeError("input must be [B,H,Tq,Tk]")
    if row_max_plus1.dim() != 4:
        raise RuntimeError("row_max_plus1 must be [B,H,Tq,1]")
    B, H, Tq, Tk = input.shape
    if tuple(row_max_plus1.shape) != (B, H, Tq, 1):
        raise RuntimeError("row_max_plus1.size(0) must equal input.size(0)")
    if frac_bits.numel() != 1:
        raise RuntimeError("frac_bits must be a scalar")
    f = _host_scalar(frac_bits, "frac_bits")
    if not 0 < f < 14:
        raise RuntimeError("frac_bits must be in [1, 14)")
    mp = _mask_check(mask, Tq, Tk)
    p = torch.empty((B, H, Tq, Tk), dtype=torch.uint8, device=input.device)
    rs = torch.empty((B, H, Tq, 1), dtype=torch.int32, device=input.device)
    _lib.call("iw_shift_exp", input.data_ptr(), row_max_plus1.data_ptr(), mp, p.data_ptr(),
              rs.data_ptr(), B, H, Tq, Tk, f, mask is not None, _stream())
    return p, rs


def pv_norm_requant_hip(p, v, row_sum, av_multiplier, av_shift, rsqrt_offset: int) -> Tensor:
    """Counterpart of _C.pv_norm_requant_simd (attention/attention_torch.cpp:523-669).

    A negative row sum raises ValueError, as the reference kernel throws
    std::invalid_argument (attention_scalar.cpp:724-728).
    """
    _check(p, torch.uint8, "p")
    _check(v, torch.int8, "v")
    _check(row_sum, torch.int32, "row_sum")
    _check_scalar(av_multiplier, torch.uint8, "av_multiplier")
    _check_scalar(av_shift, torch.int8, "av_shift")
    if p.dim() != 4:
        raise RuntimeError("p must be [B,H,Tq,Tk]")
    if v.dim() != 4:
        raise RuntimeError("v must be [B,H,D,Tk]")
    if row_sum.dim() != 4:
        raise RuntimeError("row_sum must be [B,H,Tq,1]")
    if p.size(0) != v.size(0) or p.size(0) != row_sum.size(0):
        raise RuntimeError("batch mismatch")
    if p.size(1) != v.size(1) or p.size(1) != row_sum.size(1):
        raise RuntimeError("head count mismatch")
    if p.size(2) != row_sum.size(2):
        raise RuntimeError("query length mismatch")
    if row_sum.size(3) != 1:
        raise RuntimeError("row_sum must have last dimension 1")
    if p.size(3) != v.size(3):
        raise RuntimeError("key length mismatch")
    if av_multiplier.numel() != 1:
        raise RuntimeError("av_multiplier must be scalar")
    if av_shift.numel() != 1:
        raise RuntimeError("av_shift must be scalar")
    if not 0 <= rsqrt_offset <= 29:
        raise RuntimeError("rsqrt_offset must be in [0,29]")
    if row_sum.numel() and bool((row_sum < 0).any()):
        raise ValueError("row_sum must be non-negative")
    B, H, Tq, Tk = p.shape
    D = v.size(2)
    out = torch.empty((B, Tq, H * D), dtype=torch.int8, device=p.device)
    _lib.call("iw_pv_norm_requant", p.data_ptr(), v.data_ptr(), row_sum.data_ptr(),
              _host_scalar(av_multiplier, "av_multiplier"), _host_scalar(av_shift, "av_shift"),
              rsqrt_offset, out.data_ptr(), B, H, Tq, Tk, D, _stream())
    return out


def shift_exp_table_hip(frac_bits: int, device="cuda") -> Tensor:
    """Shift-exp table for the fused attention (one entry per -x_sub)."""
    if not 0 < frac_bits < 14:
        raise RuntimeError("frac_bits must be in [1, 14)")
    t = torch.empty(32768, dtype=torch.uint8, device=device)
    _lib.call("iw_shift_exp_table", t.data_ptr(), frac_bits, _stream())
    return t


def attention_hip(q, k, vt, out, *, batch, heads, q_length, k_length, head_dim, q_strides,
                  k_strides, v_strides, o_strides, mask, qk_multiplier, qk_shift, frac_bits,
                  av_multiplier, av_shift, rsqrt_offset, table=None, decode=False) -> Tensor:
    """Fused qk_requant_rowmax -> shift_exp -> pv_norm_requant (model_int.py:774-1040).

    Strides are in elements: q_strides = (sb, st), k_strides = (sb, sh, st),
    v_strides = (sb, sh, sd) of V transposed per head, o_strides = (sb, st).
    """
    _lib.call("iw_attention", q.data_ptr(), q_strides[0], q_strides[1], k.data_ptr(),
              k_strides[0], k_strides[1], k_strides[2], vt.data_ptr(), v_strides[0], v_strides[1],
              v_strides[2], out.data_ptr(), o_strides[0], o_strides[1], _ptr(mask), batch, heads,
              q_length, k_length, head_dim, qk_multiplier, qk_shift, frac_bits, av_multiplier,
              av_shift, rsqrt_offset, _ptr(table), decode, _stream())
    return out


def argmax_rows_hip(x: Tensor) -> Tensor:
    """First index of the maximum of each row of an int8 [rows, cols] tensor."""
    _check(x, torch.int8, "x")
    rows, cols = x.reshape(-1, x.size(-1)).shape
    out = torch.empty(rows, dtype=torch.int64, device=x.device)
    _lib.call("iw_argmax_rows", x.data_ptr(), rows, cols, cols, out.data_ptr(), _stream())
    return out.reshape(x.shape[:-1])
