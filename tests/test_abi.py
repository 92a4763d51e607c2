"""The C ABI boundary without a GPU: the built library loads, exports every
function that include/iwhisper_amd.h declares, the ctypes binding matches the
header's argument counts, and argument validation reports errors through
iw_last_error() before any device work."""
import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "iwhisper_amd.h"


def _declarations():
    """name -> number of parameters, for every function the header declares."""
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    decls = {}
    for m in re.finditer(r"\b(?:int64_t|int|const char\s*\*)\s*(iw_\w+)\s*\(([^)]*)\)\s*;", text):
        params = m.group(2).strip()
        decls[m.group(1)] = 0 if params in ("", "void") else len(params.split(","))
    return decls


@pytest.fixture(scope="module")
def lib(iw):
    path = iw._lib.LIB_PATH
    if not path.exists():
        import __graft_entry__

        __graft_entry__._build_lib()
    return ctypes.CDLL(str(path))


def test_header_declares_the_api():
    decls = _declarations()
    assert len(decls) >= 29
    for name in ("iw_linear8", "iw_attention", "iw_attention_decode_cache", "iw_linear8_qkv_cache",
                 "iw_greedy_advance", "iw_last_error", "iw_abi_version"):
        assert name in decls


def test_library_exports_every_declared_function(lib):
    missing = [name for name in _declarations() if not hasattr(lib, name)]
    assert not missing, f"declared but not exported: {missing}"


def test_binding_matches_header(iw):
    decls = _declarations()
    sigs = dict(iw._lib.SIGNATURES)
    sigs.update({name: argtypes for name, (argtypes, _) in iw._lib.VALUE_FUNCS.items()})
    assert set(sigs) | {"iw_abi_version", "iw_last_error"} == set(decls)
    for name, argtypes in sigs.items():
        assert len(argtypes) == decls[name], name


def test_validation_errors_reach_iw_last_error(iw, lib):
    lib.iw_last_error.restype = ctypes.c_char_p
    fn = lib.iw_layernorm32
    fn.argtypes = iw._lib.SIGNATURES["iw_layernorm32"]
    fn.restype = ctypes.c_int
    # an unsupported width is rejected before any device call
    rc = fn(None, None, None, 1, 1, 1, 1, 13, None, 2, 100, False, None)
    assert rc != 0
    assert b"unsupported LayerNorm hidden size" in lib.iw_last_error()
    lib.iw_abi_version.restype = ctypes.c_int
    assert lib.iw_abi_version() == iw._lib.ABI_VERSION


def test_frag_bytes(iw):
    """Size of a fragment-major image: rows rounded up to 32, columns to 320."""
    v = iw._lib.value
    assert v("iw_frag_bytes", 128, 1280) == 128 * 1280
    assert v("iw_frag_bytes", 5, 384) == 32 * 640
    assert v("iw_frag_bytes", 33, 5120) == 64 * 5120
    assert v("iw_frag_bytes", 51865, 1280) == 51872 * 1280
    assert v("iw_frag_bytes", 1, 5121) == 0 and v("iw_frag_bytes", -1, 4) == 0
