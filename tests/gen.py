"""Seeded input generators shared by the oracle and GPU parity tests."""
from __future__ import annotations

import numpy as np


def rng(seed: int) -> np.random.Generator:
    return np.random.default_rng(seed)


def i8(r, shape, lo=-128, hi=127):
    return r.integers(lo, hi + 1, size=shape, dtype=np.int64).astype(np.int8)


def linear_case(seed, M, K, N, *, has_bias=True, asym=True, shift_lo=0, shift_hi=31,
                full_mult=True):
    r = rng(seed)
    x = i8(r, (M, K))
    w = i8(r, (N, K))
    bias = r.integers(-2**31, 2**31, size=N, dtype=np.int64).astype(np.int32) if has_bias else None
    wz = i8(r, N) if asym else None
    if full_mult:
        mult = r.integers(0, 2**32, size=N, dtype=np.uint64).astype(np.uint32)
    else:
        mult = r.integers(2**20, 2**31, size=N, dtype=np.uint64).astype(np.uint32)
    shift = r.integers(shift_lo, shift_hi + 1, size=N).astype(np.int8)
    return x, w, bias, wz, mult, shift


def realistic_linear_case(seed, M, K, N, *, has_bias=True, asym=True):
    """Parameters in the ranges calibration produces (outputs not all saturated)."""
    r = rng(seed)
    x = i8(r, (M, K), -127, 127)
    w = i8(r, (N, K), -127, 127)
    bias = r.integers(-2**15, 2**15, size=N).astype(np.int32) if has_bias else None
    wz = i8(r, N, -8, 8) if asym else None
    mult = r.integers(2**30, 2**31, size=N, dtype=np.uint64).astype(np.uint32)
    shift = r.integers(6, 12, size=N).astype(np.int8)
    return x, w, bias, wz, mult, shift


def gelu_params(r, channels, luti_pc=True, luto_pc=True):
    lut = np.sort(r.integers(0, 256, size=16)).astype(np.uint8)
    ci = channels if luti_pc else 1
    co = channels if luto_pc else 1
    luti_m = r.integers(1, 256, size=ci).astype(np.uint8)
    luti_s = r.integers(0, 14, size=ci).astype(np.int8)
    luto_m = r.integers(1, 256, size=co).astype(np.uint8)
    luto_s = r.integers(6, 16, size=co).astype(np.int8)
    return lut, luti_m, luti_s, luto_m, luto_s


def ln_case(seed, rows, hidden, spread=4000):
    r = rng(seed)
    x = np.clip(r.normal(0, spread, size=(rows, hidden)), -16383, 16383).astype(np.int16)
    gamma = i8(r, hidden, -127, 127)
    beta = r.integers(-2**12, 2**12, size=hidden).astype(np.int32)
    ln_m = int(r.integers(64, 256))
    ln_s = int(r.integers(8, 14))
    out_m = int(r.integers(2**30, 2**32))
    out_s = int(r.integers(2, 8))
    return x, gamma, beta, ln_m, ln_s, out_m, out_s


def attn_case(seed, B, H, Tq, Tk, D, *, spread=127):
    r = rng(seed)
    q = i8(r, (B, H, Tq, D), -spread, spread)
    k = i8(r, (B, H, Tk, D), -spread, spread)
    v = i8(r, (B, H, D, Tk), -127, 127)
    qk_m = int(r.integers(1, 256))
    qk_s = int(r.integers(6, 14))
    f = int(r.integers(5, 12))
    av_m = int(r.integers(64, 256))
    av_s = int(r.integers(4, 10))
    return q, k, v, qk_m, qk_s, f, av_m, av_s


def causal_mask(tq, tk):
    """The decoder's triu(1) mask sliced as model_int.py:786-799 does."""
    off = tk - tq
    full = np.triu(np.ones((tk, tk), dtype=bool), 1)
    return np.ascontiguousarray(full[off:off + tq, :tk])


# V caches of the decode entry points: element (b, h, t, d) at
# b*v_sb + h*v_sh + d*v_sd + (t//4)*v_sq + t%4.
V_LAYOUTS = ("vt", "quads", "quads_pad")


def v_cache_layout(B, H, D, tcap, layout):
    """Array shape and (v_sb, v_sh, v_sd, v_sq) of a V cache of tcap positions:
    'vt' transposed rows [B, H, D, round_up(tcap, 16)]; 'quads' key quads
    [B, H, round_up(tcap, 16) / 4, 4 D]; 'quads_pad' the same with 16 unused
    bytes after each quad."""
    tc16 = (tcap + 15) // 16 * 16
    if layout == "vt":
        return (B, H, D, tc16), (H * D * tc16, D * tc16, tc16, 4)
    qs = 4 * D + (16 if layout == "quads_pad" else 0)
    nq = tc16 // 4
    return (B, H, nq, qs), (H * nq * qs, nq * qs, 4, qs)


def v_cache_put(cache, layout, t0, vt):
    """Write vt [B, H, D, n] (V transposed) at positions t0 .. t0 + n - 1."""
    if layout == "vt":
        cache[..., t0:t0 + vt.shape[-1]] = vt
        return
    D = vt.shape[2]
    for i in range(vt.shape[-1]):
        t = t0 + i
        cache[:, :, t // 4, 4 * np.arange(D) + t % 4] = vt[..., i]
