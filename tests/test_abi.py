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
    l = _native.lib()
    # These checks hand host buffers to entry points whose argument checks must refuse them
    # before any launch; where a gfx950 device is visible a broken check would launch a kernel
    # on host memory, so they run only where none is.
    if l.ancha_hip_available():
        pytest.skip("host-buffer argument checks run only where no gfx950 device is visible")
    return l


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


def test_model_and_dsp_entry_points_check_arguments(lib):
    """The model, separation and DSP entry points report argument errors with a message and
    the documented code, before touching any device."""
    buf = ctypes.create_string_buffer(1 << 12)
    p = ctypes.addressof(buf) + (-ctypes.addressof(buf)) % 16
    rc = lib.ancha_hip_roformer_forward(None, p, 10, p, 1024, p, None, None)
    assert rc == _native.INVALID and "null model" in _native.last_error()
    rc = lib.ancha_hip_separate(None, p, 10, p, 1024, p, None, None, None)
    assert rc == _native.INVALID and "null model" in _native.last_error()
    rc = lib.ancha_hip_stft(p, 5000, 0, p, None)
    assert rc == _native.INVALID and "hop" in _native.last_error()
    rc = lib.ancha_hip_stft(p, 1000, 441, p, None)
    assert rc == _native.INVALID and "longer than FFT/2" in _native.last_error()
    rc = lib.ancha_hip_istft(p, p, 3, 441, 10_000, 0, p, 1 << 20, p, None)
    assert rc == _native.INVALID and "exceeds frame support" in _native.last_error()
    rc = lib.ancha_hip_block_forward(None, p, 1, 4, p, p, 1024, p, None)
    assert rc == _native.INVALID and "null block" in _native.last_error()
    rc = lib.ancha_hip_axis_pair_forward(None, None, p, 1, 2, 3, p, p, p, 1024, p, None)
    assert rc == _native.INVALID
    assert lib.ancha_hip_check() == 0


def test_attention_grid_guard(lib):
    """A problem count the launch cannot index (a short-sequence grid past HIP's 2^32 threads, or
    more than 2^31 long-sequence passes of 512 queries) is UNSUPPORTED (the caller falls back)
    instead of a launch failure that would poison the sticky state."""
    buf = ctypes.create_string_buffer(1 << 12)
    p = ctypes.addressof(buf)
    for groups, tokens in ((1 << 27, 801), (1 << 25, 60)):
        rc = lib.ancha_hip_attention(p, p, p, groups, tokens, 8, 512, 512, 512, None, p, None)
        assert rc == _native.UNSUPPORTED and "exceeds the grid" in _native.last_error()
    assert lib.ancha_hip_check() == 0


def test_cancelled_maps_to_its_exception():
    with pytest.raises(_native.Cancelled):
        _native.check(_native.CANCELLED)


def test_python_wrappers_reject_host_and_misshaped_tensors():
    """Without a GPU: tensors in host memory, of the wrong dtype or shape raise ValueError
    before anything reaches the C ABI."""
    import torch

    from ancha_amd import _tensors as T
    from ancha_amd import separation as S

    cuda0 = torch.device("cuda:0")
    with pytest.raises(ValueError, match="must be on"):
        T.require(torch.zeros(3), "x", cuda0)
    with pytest.raises(ValueError, match="float32"):
        T.require(torch.zeros(3, dtype=torch.float64), "x", cuda0)
    with pytest.raises(ValueError, match="must be on"):
        S.check_audio(torch.zeros((2, 100)), cuda0)
    with pytest.raises(ValueError, match=r"\[2, samples\]"):
        S.check_audio(torch.zeros((3, 100)), cuda0)
    with pytest.raises(ValueError, match="4100"):
        S.check_spectrum(torch.zeros((5, 4099)), cuda0)
    with pytest.raises(ValueError):
        S.stft(torch.zeros((2, 5000)), 441)
    with pytest.raises(ValueError):
        S.istft(torch.zeros((12, 1025, 2, 2)), torch.zeros((2050, 2, 12)), 441, 4000)
    # fused ops keep the reference's None for tensors off the GPU backend.
    from ancha_amd import fused
    q = torch.zeros((1, 4, 1, 64))
    assert fused.attention(q, q, q) is None
