"""numpy front end of the CPU oracle (TEST INFRASTRUCTURE ONLY).

Three libraries expose the same operations:
  * ``Oracle("oracle")`` - this repository's C restatement, oracle/iw_oracle.c
    (built by ``make -C oracle``), used on every machine;
  * ``Oracle("simd")``   - the SIMD-shaped restatement, oracle/iw_cpu_simd.c
    (dot-product tiles split over threads, as the reference's CPU backend
    runs), bit-identical to the first; timed as bench.py's CPU baseline;
  * ``Oracle("ref")``    - the reference's own scalar kernels compiled from the
    reference tree behind oracle/ref_shim.cpp into oracle/_ref/ (``make -C
    oracle ref``); present only where that build was made.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use this
module. Every function takes and returns numpy arrays with the dtypes and
layouts of the reference's torch bindings.
"""
from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIBS = {
    "oracle": HERE / "build" / "libiw_oracle.so",
    "simd": HERE / "build" / "libiw_cpu_simd.so",
    "ref": HERE / "_ref" / "libiwref.so",
}


def build(ref: bool = False) -> None:
    """Compile the oracle (and, if asked and the reference tree exists, oracle/_ref)."""
    subprocess.run(["make", "-s", "-C", str(HERE), "all"], check=True)
    if ref:
        subprocess.run(["make", "-s", "-C", str(HERE), "ref"], check=True)


def available(kind: str) -> bool:
    return LIBS[kind].exists()


def _p(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


class Oracle:
    """Dispatches each op to ``iwo_*`` (kind "oracle") or ``ref_*`` (kind "ref")."""

    def __init__(self, kind: str = "oracle", threads: int = 1):
        self.kind = kind
        self.threads = threads
        path = LIBS[kind]
        if not path.exists():
            raise RuntimeError(f"{path} is not built")
        self.lib = C.CDLL(str(path))
        self.pre = {"oracle": "iwo_", "simd": "iws_"}.get(kind, "ref_")
        if kind in ("oracle", "simd"):
            for fn, res in (("iwo_mulh", C.c_int32), ("iwo_rshift", C.c_int32),
                            ("iwo_requant", C.c_int32), ("iwo_fisr", C.c_int32),
                            ("iwo_shift_exp_one", C.c_uint8)):
                getattr(self.lib, fn).restype = res
            self.lib.iwo_mulh.argtypes = [C.c_int32, C.c_uint32]
            self.lib.iwo_rshift.argtypes = [C.c_int32, C.c_uint32]
            self.lib.iwo_requant.argtypes = [C.c_int32, C.c_uint32, C.c_uint32]
            self.lib.iwo_fisr.argtypes = [C.c_int32, C.c_uint32]
            self.lib.iwo_shift_exp_one.argtypes = [C.c_int16, C.c_int32]

    def _fn(self, name):
        return getattr(self.lib, self.pre + name)

    def _thr(self):
        return (C.c_int(self.threads),) if self.kind in ("oracle", "simd") else ()

    # ---- fixed point (oracle only) ----
    def mulh(self, x: int, m: int) -> int:
        return self.lib.iwo_mulh(x, m)

    def rshift(self, x: int, s: int) -> int:
        return self.lib.iwo_rshift(x, s)

    def requant(self, x: int, m: int, s: int) -> int:
        return self.lib.iwo_requant(x, m, s)

    def fisr(self, x: int, off: int) -> int:
        return self.lib.iwo_fisr(x, off)

    def shift_exp_one(self, x_sub: int, frac_bits: int) -> int:
        return self.lib.iwo_shift_exp_one(x_sub, frac_bits)

    # ---- GEMM family ----
    def linear8(self, x, w, bias, wz, mult, shift):
        x = _c(x, np.int8)
        w = _c(w, np.int8)
        K = x.shape[-1]
        N = w.shape[0]
        M = x.size // K
        out = np.empty((*x.shape[:-1], N), np.int8)
        b = None if bias is None else _c(bias, np.int32)
        z = None if wz is None else _c(wz, np.int8)
        self._fn("linear8")(_p(x), _p(w), _p(b), _p(z), _p(_c(mult, np.uint32)),
                            _p(_c(shift, np.int8)), _p(out), C.c_int64(M), C.c_int64(K),
                            C.c_int64(N), C.c_int(b is not None), C.c_int(z is not None),
                            *self._thr())
        return out

    def linear32(self, x, w, bias, wz, mult, shift):
        x = _c(x, np.int8)
        w = _c(w, np.int8)
        K = x.shape[-1]
        N = w.shape[0]
        M = x.size // K
        out = np.empty((*x.shape[:-1], N), np.int32)
        b = None if bias is None else _c(bias, np.int32)
        z = None if wz is None else _c(wz, np.int8)
        self._fn("linear32")(_p(x), _p(w), _p(b), _p(z), _p(_c(mult, np.uint32)),
                             _p(_c(shift, np.int8)), _p(out), C.c_int64(M), C.c_int64(K),
                             C.c_int64(N), C.c_int(b is not None), C.c_int(z is not None),
                             *self._thr())
        return out

    def linear_accum(self, x, w, bias, wz):
        x = _c(x, np.int8)
        w = _c(w, np.int8)
        K = x.shape[-1]
        N = w.shape[0]
        M = x.size // K
        out = np.empty((*x.shape[:-1], N), np.int32)
        b = None if bias is None else _c(bias, np.int32)
        z = None if wz is None else _c(wz, np.int8)
        name = "linear_accum" if self.kind == "oracle" else "linear8_accum"
        self._fn(name)(_p(x), _p(w), _p(b), _p(z), _p(out), C.c_int64(M), C.c_int64(K),
                       C.c_int64(N), C.c_int(b is not None), C.c_int(z is not None), *self._thr())
        return out

    def classifier(self, x, w, mult: int, shift: int):
        x = _c(x, np.int8)
        w = _c(w, np.int8)
        K = x.shape[-1]
        N = w.shape[0]
        M = x.size // K
        out = np.empty((*x.shape[:-1], N), np.int8)
        self._fn("classifier")(_p(x), _p(w), C.c_uint32(mult), C.c_int8(shift), _p(out),
                               C.c_int64(M), C.c_int64(K), C.c_int64(N), *self._thr())
        return out

    def conv1d(self, x, w, bias, mult: int, shift: int, stride: int, padding: int):
        x = _c(x, np.int8)
        w = _c(w, np.int8)
        B, Cin, Tin = x.shape
        Cout = w.shape[0]
        ks = w.shape[1] // Cin
        tout = (Tin + 2 * padding - ks) // stride + 1
        out = np.empty((B, Cout, tout), np.int8)
        b = None if bias is None else _c(bias, np.int32)
        self._fn("conv1d")(_p(x), _p(w), _p(b), C.c_uint32(mult), C.c_int8(shift), _p(out),
                           C.c_int64(B), C.c_int64(Cin), C.c_int64(Tin), C.c_int64(Cout),
                           C.c_int64(ks), C.c_int64(stride), C.c_int64(padding),
                           C.c_int(b is not None), *self._thr())
        return out

    # ---- row / element ops ----
    def layernorm32(self, x, gamma, beta, ln_m: int, ln_s: int, out_m: int, out_s: int,
                    rsqrt_offset: int = 13):
        x = _c(x, np.int16)
        H = x.shape[-1]
        out = np.empty(x.shape, np.int8)
        b = None if beta is None else _c(beta, np.int32)
        rc = self._fn("layernorm32")(_p(x), _p(_c(gamma, np.int8)), _p(b), C.c_uint8(ln_m),
                                     C.c_int8(ln_s), C.c_uint32(out_m), C.c_int8(out_s),
                                     C.c_uint32(rsqrt_offset), _p(out), C.c_int64(x.size // H),
                                     C.c_int64(H), C.c_int(b is not None))
        if rc != 0:
            raise ValueError(f"unsupported LayerNorm hidden size: {H}")
        return out

    def rsqrt(self, x, offset: int):
        x = _c(x, np.int32)
        out = np.empty_like(x)
        self._fn("rsqrt")(_p(x), _p(out), C.c_int64(x.size), C.c_uint32(offset))
        return out

    def gelu(self, x, lut, luti_m, luti_s, luto_m, luto_s):
        x = _c(x, np.int8)
        out = np.empty_like(x)
        ch = x.shape[-1]
        luti_m = _c(luti_m, np.uint8)
        luto_m = _c(luto_m, np.uint8)
        self._fn("gelu")(_p(x), _p(_c(lut, np.uint8)), _p(luti_m), _p(_c(luti_s, np.int8)),
                         _p(luto_m), _p(_c(luto_s, np.int8)), _p(out), C.c_int64(x.size),
                         C.c_int64(ch), C.c_int64(luti_m.size), C.c_int64(luto_m.size))
        return out

    def residual15(self, branch, residual, mult: int):
        branch = _c(branch, np.int32)
        residual = _c(residual, np.int16)
        out = np.empty_like(residual)
        self._fn("residual15")(_p(branch), _p(residual), C.c_uint16(mult), _p(out),
                               C.c_int64(branch.size))
        return out

    def add_requant15(self, x, addend, mult, shift):
        x = _c(x, np.int8)
        B, T, Ch = x.shape
        mult = _c(mult, np.uint16)
        shift = _c(shift, np.int8)
        out = np.empty((B, T, Ch), np.int16)
        self._fn("add_requant15")(_p(x), _p(_c(addend, np.int8)), _p(mult), _p(shift), _p(out),
                                  C.c_int64(B), C.c_int64(T), C.c_int64(Ch),
                                  C.c_int64(mult.size), C.c_int64(shift.size))
        return out

    # ---- attention ----
    def qk_requant_rowmax(self, q, k, mask, mult: int, shift: int):
        q = _c(q, np.int8)
        k = _c(k, np.int8)
        B, H, Tq, D = q.shape
        Tk = k.shape[2]
        qk = np.empty((B, H, Tq, Tk), np.int16)
        rm = np.empty((B, H, Tq, 1), np.int16)
        m = None if mask is None else _c(mask, np.bool_)
        self._fn("qk_requant_rowmax")(_p(q), _p(k), _p(m), _p(qk), _p(rm), C.c_int64(B),
                                      C.c_int64(H), C.c_int64(Tq), C.c_int64(Tk), C.c_int64(D),
                                      C.c_uint8(mult), C.c_int32(shift), C.c_int(m is not None),
                                      *self._thr())
        return qk, rm

    def shift_exp(self, qk, rmp1, mask, frac_bits: int):
        qk = _c(qk, np.int16)
        B, H, Tq, Tk = qk.shape
        p = np.empty(qk.shape, np.uint8)
        rs = np.empty((B, H, Tq, 1), np.int32)
        m = None if mask is None else _c(mask, np.bool_)
        self._fn("shift_exp")(_p(qk), _p(_c(rmp1, np.int16)), _p(m), _p(p), _p(rs), C.c_int64(B),
                              C.c_int64(H), C.c_int64(Tq), C.c_int64(Tk), C.c_int32(frac_bits),
                              C.c_int(m is not None), *self._thr())
        return p, rs

    def pv_norm_requant(self, p, v, row_sum, av_m: int, av_s: int, rsqrt_offset: int = 16):
        p = _c(p, np.uint8)
        v = _c(v, np.int8)
        B, H, Tq, Tk = p.shape
        D = v.shape[2]
        out = np.empty((B, Tq, H * D), np.int8)
        rc = self._fn("pv_norm_requant")(_p(p), _p(v), _p(_c(row_sum, np.int32)), C.c_uint8(av_m),
                                         C.c_int8(av_s), C.c_uint32(rsqrt_offset), _p(out),
                                         C.c_int64(B), C.c_int64(H), C.c_int64(Tq), C.c_int64(Tk),
                                         C.c_int64(D), *self._thr())
        if rc != 0:
            raise ValueError("row_sum must be non-negative")
        return out

    def attention(self, q, k, v, mask, qk_m, qk_s, frac_bits, av_m, av_s, rsqrt_offset=16):
        """The reference chain on [B,H,T,D] q/k and [B,H,D,Tk] v (model_int.py:830-1020)."""
        qk, rm = self.qk_requant_rowmax(q, k, mask, qk_m, qk_s)
        p, rs = self.shift_exp(qk, rm, mask, frac_bits)
        return self.pv_norm_requant(p, v, rs, av_m, av_s, rsqrt_offset)
