"""The C-ABI library builds, loads and exports every entry point the header declares
(no compute calls: this runs without a GPU)."""

import ctypes
import os

import pytest

from lollm_amd import _lib


def test_header_declares_entry_points():
    syms = _lib.header_symbols()
    assert "lollm_gdn_verify" in syms and "lollm_strerror" in syms
    assert set(syms) == set(_lib.SIGNATURES), "ctypes signatures out of sync with header"


def test_library_exports_every_header_symbol():
    if not os.path.exists(_lib.LIB_PATH):
        from lollm_amd.build import build
        build()
    L = ctypes.CDLL(_lib.LIB_PATH)
    for name in _lib.header_symbols():
        assert hasattr(L, name), f"{name} declared in include/lollm_amd.h but not exported"


def test_error_strings_and_version():
    L = _lib.lib()
    assert L.lollm_abi_version() >= 1
    assert L.lollm_strerror(0) == b"ok"
    assert b"invalid" in L.lollm_strerror(1)
    assert b"unsupported" in L.lollm_strerror(2)


def test_bad_arguments_are_rejected_before_any_launch():
    """Null pointers / bad sizes return LOLLM_EINVAL from the host-side checks."""
    L = _lib.lib()
    rc = L.lollm_gdn_verify(None, None, None, None, None, None, None, 1, None, None, None,
                            1, 1, 1, 1, 128, 128, 0, 0, 1.0, None)
    assert rc == 1
    with pytest.raises(RuntimeError, match="invalid argument"):
        _lib.check(rc, "lollm_gdn_verify")
    # the step's other entry points: null buffers are refused before any HIP call
    assert L.lollm_verify_input(None, None, 3, None, 100, None, 1e-6, None, None, None, None,
                                None, 16, 4096, None) == 1
    assert L.lollm_gemm_logits(None, 4096, None, 64, 151936, 4096, None, 151936, None, 5, None,
                               0, None, 0, 0, 4, 1.0, None, 0, 256, None) == 1
    assert L.lollm_spec_accept_rowmax(None, None, 5, 5, None, None, 16, 3, 151936, 1.4, 0,
                                      0.95, 7, 0, None, None, None, None, 0, None) == 1
    assert L.lollm_spec_accept(None, None, None, 16, 3, 151936, 1.4, 0, 0.95, 7, 0, None,
                               None, None, None, 0, None) == 1
    assert L.lollm_attn_prologue(None, None, None, None, None, None, 0, 16, 4, 32, 4, 256, 64,
                                 1e-6, None, None, None, None, 2048, None) == 1
    assert L.lollm_mtp_input(None, 1, None, 4096, None, 100, None, None, None, 16, 4096, 1e-6,
                             None) == 1
    assert L.lollm_rmsnorm(None, None, None, None, None, 64, 4096, 1e-6, None) == 1


def test_missing_library_raises(monkeypatch, tmp_path):
    monkeypatch.setattr(_lib, "LIB_PATH", str(tmp_path / "nope.so"))
    monkeypatch.setattr(_lib, "_lib", None)
    with pytest.raises(_lib.NativeLibraryMissing):
        _lib.lib()
