"""ctypes binding of the C ABI (include/lollm_amd.h).

The shared library is built in-tree by `lollm_amd.build` into
`lollm_amd/_native/liblollm_amd.so`.  There is no fallback: if the library is
missing, every kernel call raises.  Non-zero return codes become RuntimeError with
the library's own message (the reference's "hard-fail, never guess" convention,
README.md:51-54).
"""

from __future__ import annotations

import ctypes
import os
import re

_PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_PKG, "_native", "liblollm_amd.so")
HEADER = os.path.join(os.path.dirname(_PKG), "include", "lollm_amd.h")

_P = ctypes.c_void_p
_I = ctypes.c_int
_F = ctypes.c_float
_U64 = ctypes.c_uint64

# argument types of every entry point, in header order
SIGNATURES = {
    "lollm_strerror": ([_I], ctypes.c_char_p),
    "lollm_abi_version": ([], _I),
    "lollm_gdn_verify": ([_P, _P, _P, _P, _P, _P, _P, _I, _P, _P, _P,
                          _I, _I, _I, _I, _I, _I, _I, _I, _F, _P], _I),
    "lollm_gdn_select_state": ([_P, _P, _P, _I, _I, _I, _I, _I, _P], _I),
    "lollm_attn_workspace_bytes": ([_I, _I, _I, _I, _I, _I, _I], ctypes.c_longlong),
    "lollm_attn_verify": ([_P, _P, _P, _P, _P, _P, _P, ctypes.c_longlong, _I, _I, _I, _I, _I,
                           _I, ctypes.c_longlong, ctypes.c_longlong, _I, _F, _P], _I),
    "lollm_spec_workspace_bytes": ([_I, _I, _I], ctypes.c_longlong),
    "lollm_spec_accept": ([_P, _P, _P, _I, _I, _I, _F, _I, _F, _U64, _U64, _P, _P, _P, _P,
                           ctypes.c_longlong, _P], _I),
    "lollm_spec_accept_rowmax": ([_P, _P, ctypes.c_longlong, _I, _P, _P, _I, _I, _I, _F, _I, _F,
                                  _U64, _U64, _P, _P, _P, _P, ctypes.c_longlong, _P], _I),
    "lollm_spec_accept_noalloc": ([_P, _P, _P, _I, _I, _I, _F, _I, _F, _U64, _U64, _P, _P, _P,
                                   _P], _I),
    "lollm_sample_workspace_bytes": ([_I], ctypes.c_longlong),
    "lollm_sample_rows": ([_P, _I, _I, _F, _I, _F, _U64, _U64, _P, _I, _I, _P, _P,
                           ctypes.c_longlong, _P], _I),
    "lollm_philox_uniform_u24": ([_U64, _U64, _I, _I, _P, _P], _I),
    "lollm_rmsnorm": ([_P, _P, _P, _P, _P, _I, _I, _F, _P], _I),
    "lollm_verify_input": ([_P, _P, _I, _P, _I, _P, _F, _P, _P, _P, _P, _P, _I, _I, _P], _I),
    "lollm_mtp_input": ([_P, ctypes.c_longlong, _P, ctypes.c_longlong, _P, _I, _P, _P, _P, _I, _I,
                         _F, _P], _I),
    "lollm_gemm_argmax_workspace_bytes": ([_I, _I, _I, _I], ctypes.c_longlong),
    "lollm_gemm_argmax": ([_P, ctypes.c_longlong, _P, _I, _I, _I, _P, ctypes.c_longlong, _P,
                           ctypes.c_longlong, _I, _P], _I),
    "lollm_swiglu": ([_P, _P, _I, _I, _P], _I),
    "lollm_attn_small": ([_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _F, _F, _P, _P, _I, _P,
                          _P], _I),
    "lollm_attn_prologue": ([_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _F, _P, _P, _P, _P,
                             _I, _P], _I),
    "lollm_gdn_layer": ([_P, ctypes.c_longlong, _P, _P, _P, _P, _P, _P, _I, _P, _P, _P, _P, _I,
                         _I, _P, _I, _I, _I, _I, _I, _I, _I, _F, _P], _I),
    "lollm_gdn_layer_chunked": ([_P, ctypes.c_longlong, _P, _P, _P, _P, _P, _P, _I, _P, _P, _P,
                                 _P, _I, _I, _P, _I, _I, _I, _I, _I, _I, _I, _F, _P], _I),
    "lollm_gdn_state": ([_P, _P, _P, _P, _I, _I, _I, _I, _I, _P, _P], _I),
    "lollm_gemm_tile_weights": ([_P, _P, _I, _I, _I, _P], _I),
    "lollm_gemm_workspace_bytes": ([_I, _I, _I, _I], ctypes.c_longlong),
    "lollm_gemm": ([_P, ctypes.c_longlong, _P, _P, ctypes.c_longlong, _I, _I, _I, _I, _P,
                    ctypes.c_longlong, _I, _P], _I),
    "lollm_gemm_rowmax_slots": ([_I], _I),
    "lollm_gemm_logits": ([_P, ctypes.c_longlong, _P, _I, _I, _I, _P, ctypes.c_longlong, _P,
                           ctypes.c_longlong, _P, _I, _P, _I, _I, _I, _F, _P, ctypes.c_longlong,
                           _I, _P], _I),
    "lollm_gemm_rmsnorm": ([_P, ctypes.c_longlong, _P, _I, _I, _I, _P, _P, _F, _P, _P, _P, _P,
                            ctypes.c_longlong, _I, _P], _I),
    "lollm_greedy_accept": ([_P, _P, _I, _I, _P, _P, _P], _I),
    "lollm_spec_commit": ([_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _P, _P, _I, _I, _I, _I, _I,
                           _P, _P, _P, _I, _P], _I),
    "lollm_repetition_penalty": ([_P, ctypes.c_longlong, _I, _I, _I, _P, _I, _P, _I, _I, _F, _P],
                                 _I),
    "lollm_seen_mark": ([_P, _I, _I, _P, ctypes.c_longlong, _I, _I, _P], _I),
}

_lib = None


class NativeLibraryMissing(RuntimeError):
    pass


def lib():
    """Load the native library (once).  Raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise NativeLibraryMissing(
                f"{LIB_PATH} is missing: build it with `python -m lollm_amd.build` "
                "(the lollm_amd kernels have no fallback path)")
        L = ctypes.CDLL(LIB_PATH)
        for name, (args, res) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = res
        _lib = L
    return _lib


def check(rc: int, what: str):
    if rc != 0:
        msg = lib().lollm_strerror(rc).decode()
        raise RuntimeError(f"{what} failed: {msg} (code {rc})")


def header_symbols():
    """Entry points declared in include/lollm_amd.h."""
    with open(HEADER) as f:
        text = f.read()
    pat = r"^(?:const\s+)?(?:long\s+long|int|void|char|float)\s*\*?\s*(lollm_\w+)\s*\("
    return sorted(set(re.findall(pat, text, re.M)))
