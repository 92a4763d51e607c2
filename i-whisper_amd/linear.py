"""Linear8 / Linear32 layers: the MI355X counterpart of i_whisper/modules/linear.py.

Parameter names, shapes and dtypes match the reference (linear.py:12-43) so
integer checkpoints load strictly: ``weight`` int8 [out, in], ``bias`` int32
[out] (optional), buffer ``wgt_zeros`` int8 [out] (asymmetric weights),
``req_multiplier`` uint32 [out], ``req_shiftmount`` int8 [out].

``backend`` selects the implementation as in the reference; this package
implements ``"hip"`` (the gfx950 kernels) and nothing else, so there is no
silent fallback.
"""
from __future__ import annotations

from logging import Logger
from typing import Optional

import torch
from torch import nn

from . import _lib

BACKENDS = ("hip",)


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def check_backend(backend: str) -> None:
    if backend not in BACKENDS:
        raise NotImplementedError(
            f"Backend {backend} is not implemented; this package runs the 'hip' (gfx950) backend")


class LinearBase(nn.Linear):
    """linear.py:12-43 of the reference."""

    def __init__(self, in_features: int, out_features: int, bias: bool = True, asym: bool = True,
                 backend: str = "hip"):
        # float parameters of nn.Linear are replaced below: build them on "meta"
        super().__init__(in_features, out_features, bias, device="meta")
        check_backend(backend)
        self.backend = backend
        self.asym = asym
        self.act_range = 127
        if self.asym:
            self.register_buffer("wgt_zeros", torch.zeros(out_features, dtype=torch.int8))
        else:
            self.wgt_zeros = None
        self.req_multiplier = nn.Parameter(torch.ones(out_features, dtype=torch.uint32),
                                           requires_grad=False)
        self.req_shiftmount = nn.Parameter(torch.zeros(out_features, dtype=torch.int8),
                                           requires_grad=False)
        self.weight = nn.Parameter(torch.ones((out_features, in_features), dtype=torch.int8),
                                   requires_grad=False)
        if self.bias is not None:
            self.bias = nn.Parameter(torch.ones(out_features, dtype=torch.int32), requires_grad=False)

    # raw-pointer argument list shared by the GEMM entry points
    def _gemm_args(self, x: torch.Tensor):
        if x.dtype != torch.int8:
            raise AssertionError("Input activation must be int8 in integer inference mode!")
        if x.device.type != "cuda":
            raise RuntimeError("x must be a GPU tensor")
        x = x.contiguous()
        K = self.in_features
        if x.size(-1) != K:
            raise RuntimeError(f"weight.size(1) must equal x.size(-1), expected {x.size(-1)}, got {K}")
        M = x.numel() // K
        b = self.bias
        z = self.wgt_zeros if self.asym else None
        return x, M, (self.weight.data_ptr(), None if b is None else b.data_ptr(),
                      None if z is None else z.data_ptr(), self.req_multiplier.data_ptr(),
                      self.req_shiftmount.data_ptr())

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        raise NotImplementedError("Use Linear8 or Linear32")


class Linear8(LinearBase):
    """Linear with int8 requantised output (linear.py:47-110; kernel linear8_scalar.cpp:30-85)."""

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        check_backend(self.backend)
        x, M, (w, b, z, m, s) = self._gemm_args(x)
        out = torch.empty((*x.shape[:-1], self.out_features), dtype=torch.int8, device=x.device)
        _lib.call("iw_linear8", x.data_ptr(), w, b, z, m, s, out.data_ptr(), M, self.in_features,
                  self.out_features, b is not None, z is not None, _stream())
        return out

    @staticmethod
    def copy_param(quant_linear):
        new = Linear8(quant_linear.in_features, quant_linear.out_features,
                      bias=quant_linear.bias is not None, asym=quant_linear.asym)
        new.load_state_dict(quant_linear.state_dict())
        return new


class Linear32(LinearBase):
    """Linear with int32 output, mulh then left shift (linear.py:115-199; linear32_scalar.cpp:96-129)."""

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        check_backend(self.backend)
        x, M, (w, b, z, m, s) = self._gemm_args(x)
        out = torch.empty((*x.shape[:-1], self.out_features), dtype=torch.int32, device=x.device)
        _lib.call("iw_linear32", x.data_ptr(), w, b, z, m, s, out.data_ptr(), M, self.in_features,
                  self.out_features, b is not None, z is not None, _stream())
        return out

    def forward_residual15(self, x: torch.Tensor, residual: torch.Tensor, res_multiplier: int,
                           out: Optional[torch.Tensor] = None) -> torch.Tensor:
        """residual15(self(x), residual, res_multiplier) in one kernel; ``out`` may be ``residual``."""
        check_backend(self.backend)
        x, M, (w, b, z, m, s) = self._gemm_args(x)
        if residual.dtype != torch.int16 or not residual.is_contiguous():
            raise RuntimeError("residual must be a contiguous int16 tensor")
        if residual.numel() != M * self.out_features:
            raise RuntimeError("branch and residual must have the same shape")
        if out is None:
            out = torch.empty_like(residual)
        _lib.call("iw_linear32_residual15", x.data_ptr(), w, b, z, m, s, residual.data_ptr(),
                  int(res_multiplier), out.data_ptr(), M, self.in_features, self.out_features,
                  b is not None, z is not None, _stream())
        return out

    @staticmethod
    def copy_param(quant_linear):
        new = Linear32(quant_linear.in_features, quant_linear.out_features,
                       bias=quant_linear.bias is not None, asym=quant_linear.asym)
        new.load_state_dict(quant_linear.state_dict())
        return new


def _set_backend(model: nn.Module, cls, label: str, backend: str, logger: Optional[Logger]):
    check_backend(backend)
    log = logger.debug if logger is not None else (lambda *_: None)
    for name, layer in model.named_modules():
        if isinstance(layer, cls):
            if layer.backend == backend:
                log(f"{label} backend for {name} is already set to {backend}.")
            else:
                log(f"{label} backend for {name} from {layer.backend} to {backend}.")
                layer.backend = backend


def set_linear8_backend(model: nn.Module, backend: str, logger: Optional[Logger] = None):
    """linear.py:202-227 of the reference."""
    _set_backend(model, Linear8, "linear8", backend, logger)


def set_linear32_backend(model: nn.Module, backend: str, logger: Optional[Logger] = None):
    """linear.py:229-254 of the reference."""
    _set_backend(model, Linear32, "linear32", backend, logger)
