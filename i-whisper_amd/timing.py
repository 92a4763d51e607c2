"""Word-timestamp helpers on the GPU: ``median_filter`` and ``dtw`` with the
reference's signatures and results (i_whisper/timing.py:19-55 and :108-150),
backed by the HIP kernels ``iw_median_filter`` and ``iw_dtw`` instead of the
Triton ones (triton_ops.py:13-109)."""
from __future__ import annotations

import numpy as np
import torch

from . import _lib


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def median_filter(x: torch.Tensor, filter_width: int) -> torch.Tensor:
    """Median of width ``filter_width`` (odd, at most 31) along the last
    dimension with reflect padding; returns ``x`` itself when the last
    dimension is not longer than ``filter_width // 2`` (timing.py:19-55)."""
    pad_width = filter_width // 2
    if x.shape[-1] <= pad_width:
        return x
    if not (filter_width > 0 and filter_width % 2 == 1):
        raise AssertionError("`filter_width` should be an odd number")
    if not x.is_cuda or x.dtype != torch.float32:
        raise TypeError("median_filter takes a float32 CUDA tensor")
    xc = x.contiguous()
    n = xc.shape[-1]
    rows = xc.numel() // n
    y = torch.empty_like(xc)
    _lib.call("iw_median_filter", xc.data_ptr(), rows, n, n, filter_width, y.data_ptr(), n, _stream())
    return y


def backtrace(trace: np.ndarray) -> np.ndarray:
    """The alignment path from the trace matrix (timing.py:58-80): a [2, L]
    array of (row, column) indices from (0, 0) to (rows-1, cols-1)."""
    trace = np.array(trace, copy=True)
    i, j = trace.shape[0] - 1, trace.shape[1] - 1
    trace[0, :] = 2
    trace[:, 0] = 1
    result = []
    while i > 0 or j > 0:
        result.append((i - 1, j - 1))
        t = trace[i, j]
        if t == 0:
            i -= 1
            j -= 1
        elif t == 1:
            i -= 1
        elif t == 2:
            j -= 1
        else:
            raise ValueError("Unexpected trace[i, j]")
    return np.array(result)[::-1, :].T


def dtw_trace(x: torch.Tensor) -> torch.Tensor:
    """The int8 trace matrix [M+1, N+1] of x [M, N] (M < 1024), on the device."""
    if not x.is_cuda or x.dtype != torch.float32 or x.dim() != 2:
        raise TypeError("dtw takes a 2-D float32 CUDA tensor")
    M, N = x.shape
    if M >= 1024:
        raise AssertionError(f"M should be smaller than 1024 (got {M})")
    xc = x.contiguous()
    trace = torch.empty((M + 1, N + 1), dtype=torch.int8, device=x.device)
    _lib.call("iw_dtw", xc.data_ptr(), M, N, N, trace.data_ptr(), N + 1, _stream())
    return trace


def dtw(x: torch.Tensor) -> np.ndarray:
    """Dynamic-time-warping path of the cost matrix x [M, N] (timing.py:108-150
    on a CUDA tensor): the recurrence on the GPU, the backtrace on the host."""
    return backtrace(dtw_trace(x).cpu().numpy())

