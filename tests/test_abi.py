"""The C-ABI library: it loads, exports every symbol include/ancha_hip.h declares, and its
argument checks map to the documented return codes. No kernel is launched (CPU only)."""
import ctypes
import os
import re

import pytest

from ancha_amd import _native

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = [os.path.join(ROOT, "include", "ancha_hip.h")]


def declared(path):
    text = open(path).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(ancha_\w+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    return _native.lib()


def test_library_exports_every_declared_symbol(lib):
    names = [n for h in HEADERS for n in declared(h)]
    assert "ancha_hip_attention" in names and "ancha_hip_gated_attention" in names
    for name in names:
        assert hasattr(lib, name), f"{name} declared but not exported"
        assert name in _native.SIGNATURES, f"{name} has no ctypes signature"


def test_argument_checks_without_a_device(lib):
    buf = ctypes.create_string_buffer(1 << 12)
    p = ctypes.addressof(buf)
    # Column ranges that do not fit the row stride: the reference's assert! -> INVALID.
    rc = lib.ancha_hip_attention(p, p, p, 1, 4, 2, 64, 128, 128, None, p, None)
    assert rc == _native.INVALID and "column ranges" in _native.last_error()
    # Null tensors with work to do -> INVALID.
    assert lib.ancha_hip_attention(None, p, p, 1, 4, 1, 64, 64, 64, None, p, None) == _native.INVALID
    # Packed projection narrower than heads*(3*64+1) -> UNSUPPORTED (the reference's None).
    assert lib.ancha_hip_gated_attention(p, 1, 4, 3 * 64, 1, None, p, None) == _native.UNSUPPORTED
    # Sequences whose rows span more than a 32-bit buffer range -> UNSUPPORTED (checked before
    # any device query; the pointers are never read on the host).
    rc = lib.ancha_hip_attention(p, p, p, 1, 1 << 20, 1, 4096, 4096, 4096, None, p, None)
    assert rc == _native.UNSUPPORTED and "32-bit buffer range" in _native.last_error()
    # Empty problems launch nothing and succeed.
    assert lib.ancha_hip_attention(p, p, p, 0, 4, 1, 64, 64, 64, None, p, None) == _native.OK
    assert lib.ancha_hip_attention(p, p, p, 1, 0, 1, 64, 64, 64, None, p, None) == _native.OK
    # None of these is a device failure.
    assert lib.ancha_hip_check() == 0


def test_python_mirror_maps_return_codes():
    assert _native.check(_native.OK) is True
    assert _native.check(_native.UNSUPPORTED) is False
    with pytest.raises(ValueError):
        _native.check(_native.INVALID)
    with pytest.raises(_native.HipError):
        _native.check(-2)
