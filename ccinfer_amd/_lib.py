"""ctypes binding of include/ccinfer_attn.h (libccinfer_attn.so, built in-tree).

Loading fails loudly when the library is missing: there is no CPU or PyTorch fallback.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "lib" / "libccinfer_attn.so"

_c_int = ctypes.c_int
_c_size = ctypes.c_size_t
_vp = ctypes.c_void_p

# name -> (restype, argtypes); must match include/ccinfer_attn.h.
SIGNATURES = {
    "ccinfer_write_kv_cache": (_c_int, [_vp, _vp, _vp, _vp, _vp, _c_int, _c_int, _c_int, _c_int, _vp]),
    "ccinfer_qkv_prologue": (
        _c_int,
        [_vp] * 9 + [_c_int] * 6 + [ctypes.c_float, _vp],
    ),
    "ccinfer_build_batch_metadata": (_c_int, [_vp] * 5 + [_c_int] * 6 + [_vp] * 8),
    "ccinfer_decode_workspace_size": (_c_size, [_c_int] * 6),
    "ccinfer_decode_attention": (
        _c_int,
        [_vp, _vp, _vp, _vp, _vp, _vp, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _vp, _c_size, _vp],
    ),
    "ccinfer_decode_shared_workspace_size": (_c_size, [_c_int] * 6),
    "ccinfer_decode_attention_shared_prefix": (
        _c_int,
        [_vp, _vp, _vp, _vp, _vp, _vp, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _vp, _c_size, _vp],
    ),
    "ccinfer_decode_attention_write_kv": (
        _c_int, [_vp] * 8 + [_c_int] * 7 + [_vp, _c_size, _vp]),
    "ccinfer_decode_attention_noalloc": (
        _c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _vp]),
    "ccinfer_write_kv_cache_fp8": (_c_int, [_vp] * 7 + [_c_int] * 4 + [_vp]),
    "ccinfer_decode_attention_fp8": (_c_int, [_vp] * 8 + [_c_int] * 6 + [_vp, _c_size, _vp]),
    "ccinfer_prefill_attention_fp8": (
        _c_int, [_vp] * 9 + [_c_int] * 7 + [_vp, _c_size, _vp]),
    "ccinfer_prefill_workspace_size": (_c_size, [_c_int] * 7),
    "ccinfer_prefill_attention": (
        _c_int,
        [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int,
         _vp, _c_size, _vp],
    ),
    "ccinfer_prefill_attention_overlap": (
        _c_int,
        [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int,
         _vp, _c_size, _vp, _vp, _vp, _vp],
    ),
    "ccinfer_prefill_attention_fp8_overlap": (
        _c_int, [_vp] * 9 + [_c_int] * 7 + [_vp, _c_size, _vp, _vp, _vp, _vp]),
    "ccinfer_error_message": (ctypes.c_char_p, [_c_int]),
    "ccinfer_version": (ctypes.c_char_p, []),
}

_lib = None


def load() -> ctypes.CDLL:
    """Returns the loaded library (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python -m ccinfer_amd.build` "
                "(there is no fallback path)")
        lib = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib
