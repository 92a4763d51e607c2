"""ctypes binding of ``lib/libiwhisper_amd.so`` (C ABI: ``include/iwhisper_amd.h``).

The library is the only compute path of this package: if it is missing, or no
GPU is visible, every op raises instead of falling back to anything else.
"""
from __future__ import annotations

import ctypes as C
import threading
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "lib" / "libiwhisper_amd.so"
ABI_VERSION = 2  # IW_ABI_VERSION of include/iwhisper_amd.h that SIGNATURES describe

_p = C.c_void_p
_i64 = C.c_int64
_i32 = C.c_int32
_u32 = C.c_uint32
_u16 = C.c_uint16
_u8 = C.c_uint8
_i8 = C.c_int8
_b = C.c_bool
_f = C.c_float

# name -> argument types (all return int)
SIGNATURES = {
    "iw_linear8": [_p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _b, _b, _p],
    "iw_linear32": [_p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _b, _b, _p],
    "iw_layernorm32": [_p, _p, _p, _u8, _i8, _u32, _i8, _u32, _p, _i64, _i64, _b, _p],
    "iw_layernorm32_rsqrt": [_p, _p, _i64, _u32, _p],
    "iw_gelu": [_p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _p],
    "iw_residual15": [_p, _p, _u16, _p, _i64, _p],
    "iw_add_requant15": [_p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _p],
    "iw_conv1d": [_p, _p, _p, _u32, _i8, _p, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _b, _p],
    "iw_classifier": [_p, _p, _u32, _i8, _p, _i64, _i64, _i64, _p],
    "iw_qk_requant_rowmax": [_p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _u8, _i32, _b, _p],
    "iw_shift_exp": [_p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i32, _b, _p],
    "iw_pv_norm_requant": [_p, _p, _p, _u8, _i8, _u32, _p, _i64, _i64, _i64, _i64, _i64, _p],
    "iw_linear8_gelu": [_p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _p, _i64, _i64,
                        _i64, _b, _b, _p],
    "iw_linear32_residual15": [_p, _p, _p, _p, _p, _p, _p, _u16, _p, _i64, _i64, _i64, _b, _b, _p],
    "iw_quantize_mel": [_p, _f, _p, _i64, _i64, _i64, _p],
    "iw_conv1d_cl": [_p, _p, _p, _u32, _i8, _p, _p, _p, _p, _p, _i64, _i64, _p, _p, _p, _i64, _i64,
                     _p, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _b, _p],
    "iw_embed_add_requant15": [_p, _p, _p, _i64, _p, _p, _p, _i64, _i64, _i64, _p],
    "iw_shift_exp_table": [_p, _i32, _p],
    "iw_attention": [_p, _i64, _i64, _p, _i64, _i64, _i64, _p, _i64, _i64, _i64, _p, _i64, _i64,
                     _p, _i64, _i64, _i64, _i64, _i64, _u8, _i8, _i32, _u8, _i8, _u32, _p, _b, _p],
    "iw_argmax_rows": [_p, _i64, _i64, _i64, _p, _p],
    "iw_transpose_heads": [_p, _i64, _i64, _p, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _p],
    "iw_copy_rows": [_p, _i64, _i64, _p, _i64, _i64, _i64, _i64, _i64, _i64, _p],
    "iw_gather_heads": [_p, _i64, _i64, _p, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _p],
    "iw_linear8_qkv_cache": [_p, _p, _p, _p, _p, _p, _i64, _i64, _b, _b, _p, _i64, _p, _i64, _i64,
                             _i64, _p, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _p, _p],
    "iw_attention_decode_cache": [_p, _i64, _p, _i64, _i64, _i64, _p, _i64, _i64, _i64, _i64, _p, _i64,
                                  _i64, _i64, _i64, _i64, _p, _i64, _u8, _i8, _i32, _u8, _i8, _u32,
                                  _p],
    "iw_embed_tokens": [_p, _p, _p, _i64, _p, _p, _p, _p, _i64, _i64, _p],
    "iw_greedy_advance": [_p, _i64, _i64, _i64, _p, _p, _i64, _i64, _p, _p, _i32, _p],
    "iw_log_mel": [_p, _i64, _i64, _i64, _p, _p, _p, _p, _p, _p, _i32, _i32, _p, _i64, _p, _p],
    "iw_log_mel_noalloc": [_p, _i64, _i64, _i64, _p, _p, _p, _p, _p, _p, _i32, _i32, _p, _i64, _p],
    "iw_dtw": [_p, _i64, _i64, _i64, _p, _i64, _p],
    "iw_median_filter": [_p, _i64, _i64, _i64, _i32, _p, _i64, _p],
    "iw_greedy_advance_filtered": [_p, _i64, _i64, _i64, _p, _p, _i64, _i64, _p, _p, _i32, _p, _p, _p,
                                   _i32, _i32, _i32, _f, _p, _p, _p],
    "iw_greedy_update": [_p, _i64, _p, _i64, _i64, _i64, _p, _p, _i64, _i64, _p, _p, _i32, _i32, _p, _p, _f,
                         _p, _p, _p],
    "iw_token_prob": [_p, _i64, _i64, _i64, _i64, _f, _p, _p],
    "iw_classifier_argmax_frag": [_p, _p, _u32, _i8, _p, _p, _i64, _i64, _i64, _p],
    "iw_frag_pack": [_p, _i64, _i64, _i64, _p, _p],
    "iw_linear8_frag": [_p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _b, _b, _b, _p],
    "iw_linear8_gelu_frag": [_p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _p, _i64, _i64,
                             _i64, _b, _b, _b, _p, _i64, _i64, _p],
    "iw_linear32_residual15_frag": [_p, _p, _p, _p, _p, _p, _p, _u16, _p, _i64, _i64, _i64, _b, _b, _p],
    "iw_linear8_qkv_cache_frag": [_p, _p, _p, _p, _p, _p, _i64, _i64, _b, _b, _p, _i64, _p, _i64, _i64,
                                  _i64, _p, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _p, _p],
    "iw_layernorm32_frag": [_p, _p, _p, _u8, _i8, _u32, _i8, _u32, _p, _i64, _i64, _b, _p, _i64, _i64,
                            _p],
    "iw_attention_decode_cross_lnq": [_p, _i64, _p, _p, _u8, _i8, _u32, _i8, _u32, _b, _p, _p, _p, _p, _p, _b, _b,
                                      _p, _i64, _i64, _i64, _p, _i64, _i64, _i64, _p, _i64, _i64, _i64, _i64,
                                      _u8, _i8, _i32, _u8, _i8, _u32, _p],
    "iw_attention_decode_cache_frag": [_p, _i64, _p, _i64, _i64, _i64, _p, _i64, _i64, _i64, _i64, _p,
                                       _i64, _i64, _i64, _i64, _p, _i64, _u8, _i8, _i32, _u8, _i8, _u32,
                                       _p, _i64, _i64, _p],
    "iw_classifier_frag": [_p, _p, _u32, _i8, _p, _i64, _i64, _i64, _p],
}

# entry points that return a value rather than a status
VALUE_FUNCS = {"iw_frag_bytes": ([_i64, _i64], C.c_int64),
               "iw_log_mel_scratch_floats": ([_i64, _i64], C.c_int64)}

_lock = threading.Lock()
_lib = None


class IWError(RuntimeError):
    """Raised when a C ABI call returns a non-zero status."""


def load() -> C.CDLL:
    """Load the kernel library once; raise if it has not been built."""
    global _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise IWError(
                    f"{LIB_PATH} is not built; run __graft_entry__.build() or "
                    "python i-whisper_amd/build.py")
            lib = C.CDLL(str(LIB_PATH))
            for name, argtypes in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.argtypes = argtypes
                fn.restype = C.c_int
            for name, (argtypes, restype) in VALUE_FUNCS.items():
                fn = getattr(lib, name)
                fn.argtypes = argtypes
                fn.restype = restype
            lib.iw_last_error.restype = C.c_char_p
            lib.iw_last_error.argtypes = []
            lib.iw_abi_version.restype = C.c_int
            got = lib.iw_abi_version()
            if got != ABI_VERSION:
                raise IWError(f"{LIB_PATH} has C ABI version {got}; these bindings need {ABI_VERSION} "
                              "(rebuild the library)")
            _lib = lib
        return _lib


def call(name: str, *args) -> None:
    """Call ``name`` with ``args``; raise IWError carrying iw_last_error() on failure."""
    lib = load()
    rc = getattr(lib, name)(*args)
    if rc != 0:
        msg = lib.iw_last_error().decode(errors="replace")
        raise IWError(msg)


def value(name: str, *args):
    """Call an entry point of VALUE_FUNCS and return its result."""
    return getattr(load(), name)(*args)


def exported_symbols() -> list[str]:
    return ["iw_abi_version", "iw_last_error", *SIGNATURES.keys(), *VALUE_FUNCS.keys()]
