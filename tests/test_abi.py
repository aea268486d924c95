"""The C ABI: the built library loads (no GPU needed) and exports every entry
point include/draftkv_hip.h declares, and the ctypes binding covers them all."""

import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "draftkv_hip.h")


def declared() -> set[str]:
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(r"\b(dkv_[a-z0-9_]+)\s*\(", text))


def test_header_declares_the_hot_path():
    names = declared()
    for n in ("dkv_quantize", "dkv_paged_append", "dkv_paged_attention", "dkv_drafter_append",
              "dkv_drafter_truncate", "dkv_drafter_sync", "dkv_drafter_rebuild", "dkv_drafter_attention",
              "dkv_sample", "dkv_accept", "dkv_last_error", "dkv_version"):
        assert n in names


def test_library_exports_every_declared_symbol():
    from draftkv import _lib
    if not os.path.exists(_lib.LIB_PATH):
        pytest.skip("library not built (run draft-kv_amd/build.py)")
    h = ctypes.CDLL(_lib.LIB_PATH)
    missing = [n for n in declared() if not hasattr(h, n)]
    assert not missing, missing
    assert set(_lib.exported_symbols()) == declared()
    assert _lib.lib().dkv_version() == 1


def test_host_validation_errors_without_gpu():
    """Bad arguments are rejected on the host, before any launch."""
    from draftkv import _lib
    if not os.path.exists(_lib.LIB_PATH):
        pytest.skip("library not built")
    L = _lib.lib()
    rc = L.dkv_quantize(None, 4, 64, 4, 64, 0, None, None, None, None, None)
    assert rc == -1 and b"NULL" in L.dkv_last_error()
    rc = L.dkv_quantize(ctypes.c_void_p(16), 4, 64, 5, 64, 0, None, None, None, None, None)
    assert rc == -1 and b"bits" in L.dkv_last_error()
    with pytest.raises(ValueError, match="bits"):
        _lib.check(rc, "dkv_quantize")


def test_noalloc_accept_refuses_oversize_without_gpu():
    """The no-allocation accept checks its request against the static
    scratch on the host, before touching a device."""
    from draftkv import _lib
    if not os.path.exists(_lib.LIB_PATH):
        pytest.skip("library not built")
    L = _lib.lib()
    p = ctypes.c_void_p(16)
    rc = L.dkv_accept_noalloc(p, p, p, 100000, 20, 128256, 0.8, p, None, p, p, p, None)
    assert rc == -4 and b"static scratch" in L.dkv_last_error()
    rc = L.dkv_accept_noalloc(p, p, p, 0, 20, 128256, 0.8, p, None, p, p, p, None)
    assert rc == -1
