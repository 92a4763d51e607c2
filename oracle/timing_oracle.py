"""CPU restatement of the word-timestamp kernels (TEST INFRASTRUCTURE ONLY:
the tests compare iw_dtw / iw_median_filter against it; nothing in the product
imports it).

  dtw_trace      the cost recurrence of triton_ops.py:13-40 (dtw_kernel) on
                 the natural (unskewed) layout, float32, with its tie order:
                 the kernel stores 2, then 1, then 0 under "<=" masks, so the
                 first of 0, 1, 2 holding the minimum wins
  dtw_trace_cpu  the numba CPU variant, timing.py:83-105 (strict "<" tests,
                 ties go to 2): equal to dtw_trace wherever no tie occurs
  backtrace      timing.py:58-80
  median_filter  timing.py:19-55: reflect padding, sort of each window, the
                 middle element
"""
from __future__ import annotations

import numpy as np


def dtw_trace(x: np.ndarray):
    x = np.asarray(x, dtype=np.float32)
    M, N = x.shape
    cost = np.full((M + 1, N + 1), np.inf, dtype=np.float32)
    cost[0, 0] = 0
    trace = np.zeros((M + 1, N + 1), dtype=np.int8)
    trace[0, :] = 2
    trace[:, 0] = 1
    for i in range(1, M + 1):
        for j in range(1, N + 1):
            c0, c1, c2 = cost[i - 1, j - 1], cost[i - 1, j], cost[i, j - 1]
            if c0 <= c1 and c0 <= c2:
                c, t = c0, 0
            elif c1 <= c0 and c1 <= c2:
                c, t = c1, 1
            else:
                c, t = c2, 2
            cost[i, j] = np.float32(x[i - 1, j - 1] + c)
            trace[i, j] = t
    return cost, trace


def dtw_trace_cpu(x: np.ndarray):
    x = np.asarray(x, dtype=np.float32)
    M, N = x.shape
    cost = np.full((M + 1, N + 1), np.inf, dtype=np.float32)
    cost[0, 0] = 0
    trace = -np.ones((M + 1, N + 1), dtype=np.int8)
    for j in range(1, N + 1):
        for i in range(1, M + 1):
            c0, c1, c2 = cost[i - 1, j - 1], cost[i - 1, j], cost[i, j - 1]
            if c0 < c1 and c0 < c2:
                c, t = c0, 0
            elif c1 < c0 and c1 < c2:
                c, t = c1, 1
            else:
                c, t = c2, 2
            cost[i, j] = np.float32(x[i - 1, j - 1] + c)
            trace[i, j] = t
    trace[0, :] = 2
    trace[:, 0] = 1
    return cost, trace


def backtrace(trace: np.ndarray) -> np.ndarray:
    trace = np.array(trace, copy=True)
    i, j = trace.shape[0] - 1, trace.shape[1] - 1
    trace[0, :] = 2
    trace[:, 0] = 1
    out = []
    while i > 0 or j > 0:
        out.append((i - 1, j - 1))
        t = trace[i, j]
        if t == 0:
            i, j = i - 1, j - 1
        elif t == 1:
            i -= 1
        else:
            j -= 1
    return np.array(out)[::-1, :].T


def median_filter(x: np.ndarray, width: int) -> np.ndarray:
    x = np.asarray(x, dtype=np.float32)
    p = width // 2
    if x.shape[-1] <= p:
        return x
    xp = np.pad(x, [(0, 0)] * (x.ndim - 1) + [(p, p)], mode="reflect")
    win = np.lib.stride_tricks.sliding_window_view(xp, width, axis=-1)
    return np.sort(win, axis=-1)[..., p]
