"""The C ABI boundary: libmdx.so loads and exports exactly what include/mdx.h declares; the
Python shim binds every declared function. CPU only (no compute calls)."""
import ctypes
import os
import re

import pytest

from conftest import ROOT

HEADER = os.path.join(ROOT, "include", "mdx.h")
LIB = os.path.join(ROOT, "comfy-mono-decode-xpu_amd", "mdx", "libmdx.so")


def declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(mdx_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_entry_points():
    names = declared()
    assert "mdx_w4a8_decode_linear" in names and "mdx_last_error" in names
    assert len(names) >= 6


def test_library_exports_every_declared_symbol():
    if not os.path.exists(LIB):
        pytest.skip("libmdx.so not built")
    lib = ctypes.CDLL(LIB)
    missing = [n for n in declared() if not hasattr(lib, n)]
    assert not missing, missing


def test_shim_binds_every_declared_symbol():
    from mdx import _lib
    assert sorted(_lib.SIGNATURES) == declared()


def test_version_and_error_without_gpu():
    if not os.path.exists(LIB):
        pytest.skip("libmdx.so not built")
    from mdx import _lib
    L = _lib.lib()
    assert L.mdx_version() >= 1
    assert isinstance(L.mdx_last_error(), bytes)
    # a contract violation is reported before any device work: no GPU needed
    rc = L.mdx_rot_quant(None, None, 0, None, None, 1, 100, None)
    assert rc == _lib.MDX_EINVAL
    assert b"null pointer" in L.mdx_last_error()
