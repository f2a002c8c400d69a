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


def test_missing_library_raises(monkeypatch, tmp_path):
    monkeypatch.setattr(_lib, "LIB_PATH", str(tmp_path / "nope.so"))
    monkeypatch.setattr(_lib, "_lib", None)
    with pytest.raises(_lib.NativeLibraryMissing):
        _lib.lib()
