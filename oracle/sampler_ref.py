"""ctypes binding of the exact C sampler oracle (oracle/sampler_ref.c) -- TEST ONLY.

Inputs are numpy arrays; bf16 logits are passed as their uint16 bit patterns.
"""

from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "liblollm_oracle.so")
_lib = None


def build():
    subprocess.check_call(["make", "-s", "-C", _HERE])


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        P = ctypes.c_void_p
        L.oracle_philox4x32_10.argtypes = [P, P, P]
        L.oracle_uniform_u24.argtypes = [ctypes.c_uint64, ctypes.c_uint64, ctypes.c_uint32,
                                         ctypes.c_uint32]
        L.oracle_uniform_u24.restype = ctypes.c_uint32
        L.oracle_exp2.argtypes = [ctypes.c_float]
        L.oracle_exp2.restype = ctypes.c_float
        L.oracle_weight.argtypes = [ctypes.c_float, ctypes.c_float, ctypes.c_float]
        L.oracle_weight.restype = ctypes.c_uint64
        L.oracle_row_stats.argtypes = [P, ctypes.c_int, ctypes.c_float, ctypes.c_int,
                                       ctypes.c_float, P]
        L.oracle_row_weights.argtypes = [P, ctypes.c_int, ctypes.c_float, ctypes.c_int,
                                         ctypes.c_float, P]
        L.oracle_sample_rows.argtypes = [P, ctypes.c_int, ctypes.c_int, ctypes.c_float,
                                         ctypes.c_int, ctypes.c_float, ctypes.c_uint64,
                                         ctypes.c_uint64, ctypes.c_int, ctypes.c_int, P]
        L.oracle_spec_accept.argtypes = [P, P, P, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                         ctypes.c_float, ctypes.c_int, ctypes.c_float,
                                         ctypes.c_uint64, ctypes.c_uint64, P, P]
        L.oracle_repetition_penalty.argtypes = [P, ctypes.c_int, P, ctypes.c_int, ctypes.c_float]
        _lib = L
    return _lib


def _ptr(a):
    return a.ctypes.data_as(ctypes.c_void_p) if a is not None else None


def _bits(x):
    """bf16 logits as uint16 bits: accepts a torch bf16 tensor or a uint16 array."""
    if hasattr(x, "dtype") and str(x.dtype) == "torch.bfloat16":
        x = x.detach().cpu().contiguous().view(__import__("torch").int16).numpy().view(np.uint16)
    return np.ascontiguousarray(x, dtype=np.uint16)


def inv_temperature(temperature: float) -> float:
    """Host-side rule shared with the product: 1/T as fp32, 0 for greedy (T <= 0)."""
    return float(np.float32(1.0 / temperature)) if temperature > 0 else 0.0


def philox4x32_10(ctr, key):
    c = np.asarray(ctr, dtype=np.uint32)
    k = np.asarray(key, dtype=np.uint32)
    out = np.zeros(4, dtype=np.uint32)
    lib().oracle_philox4x32_10(_ptr(c), _ptr(k), _ptr(out))
    return out


def uniform_u24(seed, offset, row, slot):
    return int(lib().oracle_uniform_u24(seed, offset, row, slot))


def exp2(t: float) -> float:
    return float(lib().oracle_exp2(t))


def weight(x: float, xmax: float, c: float) -> int:
    return int(lib().oracle_weight(x, xmax, c))


def row_stats(x, inv_temp, top_k=0, top_p=1.0):
    xb = _bits(x).reshape(-1)
    out = np.zeros(4, dtype=np.int64)
    lib().oracle_row_stats(_ptr(xb), xb.size, inv_temp, top_k, top_p, _ptr(out))
    return {"argmax": int(out[0]), "kmax": int(out[1]), "cut": int(out[2]),
            "Z": int(out[3].astype(np.uint64))}


def row_weights(x, inv_temp, top_k=0, top_p=1.0):
    xb = _bits(x).reshape(-1)
    w = np.zeros(xb.size, dtype=np.uint64)
    lib().oracle_row_weights(_ptr(xb), xb.size, inv_temp, top_k, top_p, _ptr(w))
    return w


def sample_rows(logits, inv_temp, top_k, top_p, seed, offset, row_base=0, slot=0):
    xb = _bits(logits)
    rows, V = xb.shape
    out = np.zeros(rows, dtype=np.int32)
    lib().oracle_sample_rows(_ptr(xb), rows, V, inv_temp, top_k, top_p, seed, offset,
                             row_base, slot, _ptr(out))
    return out


def spec_accept(target, draft, drafts, inv_temp, top_k, top_p, seed, offset):
    """target (B, k+1, V) bf16; draft (B, k, V) bf16 or None (one-hot q at the
    drafts); drafts (B, k) int.  Returns (n_accepted (B,), next_token (B,))."""
    tb = _bits(target)
    B, T, V = tb.shape
    k = T - 1
    db = _bits(draft) if draft is not None else None
    if db is not None:
        assert db.shape == (B, k, V)
    dr = np.ascontiguousarray(np.asarray(drafts), dtype=np.int32).reshape(B, k)
    na = np.zeros(B, dtype=np.int32)
    nt = np.zeros(B, dtype=np.int32)
    rc = lib().oracle_spec_accept(_ptr(tb), _ptr(db), _ptr(dr), B, k, V, inv_temp, top_k,
                                  top_p, seed, offset, _ptr(na), _ptr(nt))
    if rc:
        raise RuntimeError(f"oracle_spec_accept failed ({rc})")
    return na, nt


def repetition_penalty(row, ids, penalty):
    """generate.py:18-22 on one bf16 row (uint16 bits or a torch bf16 tensor): returns the
    penalised row as uint16 bits.  ids: the context token ids (duplicates allowed)."""
    xb = _bits(row).reshape(-1).copy()
    ids = np.ascontiguousarray(np.asarray(ids, dtype=np.int64).reshape(-1), dtype=np.int32)
    rc = lib().oracle_repetition_penalty(_ptr(xb), xb.size, _ptr(ids), ids.size, penalty)
    if rc:
        raise RuntimeError("oracle_repetition_penalty failed")
    return xb
