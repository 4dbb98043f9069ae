"""Loader for the gfx950 kernel library ``ancha_amd/_lib/libancha_hip.so`` (C ABI of
``include/ancha_hip.h``) and its return-code handling.

There is no fallback: if the library is missing, every op raises instead of computing the
result some other way.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "_lib", "libancha_hip.so")
CSRC = os.path.join(HERE, "csrc")

OK, UNSUPPORTED, INVALID, CANCELLED = 0, 1, 2, 3


class HipError(RuntimeError):
    """A HIP runtime failure (sticky, like the reference's device::check)."""


class Cancelled(RuntimeError):
    """The caller's cancellation flag stopped the call ("task cancelled")."""


def build(jobs: int = 8) -> str:
    """Compile the HIP library for gfx950 with hipcc (works without a GPU)."""
    subprocess.run(["make", "-s", f"-j{jobs}", "-C", CSRC], check=True)
    return LIB_PATH


_lib: ctypes.CDLL | None = None
_sz, _p, _int = ctypes.c_size_t, ctypes.c_void_p, ctypes.c_int

# name -> (restype, argtypes); every symbol include/ancha_hip.h declares.
SIGNATURES = {
    "ancha_hip_available": (_int, []),
    "ancha_hip_attention": (_int, [_p, _p, _p, _sz, _sz, _sz, _sz, _sz, _sz, _p, _p, _p]),
    "ancha_hip_gated_attention": (_int, [_p, _sz, _sz, _sz, _sz, _p, _p, _p]),
    "ancha_hip_linear": (_int, [_p, _sz, _sz, _sz, _p, _sz, _p, _int, _p, _sz, _sz, _p, _p, _p]),
    "ancha_hip_linear_supported": (_int, [_sz, _sz]),
    "ancha_hip_norm_linear": (_int, [_p, _sz, _sz, _sz, _p, _sz, _p, _int, _p, _sz, _sz, _p, _p,
                                     _p]),
    "ancha_hip_unit_norm": (_int, [_p, _sz, _sz, _sz, _p, _p, _p]),
    "ancha_hip_block_create": (_int, [_sz, _sz, _sz] + [_p] * 11 + [ctypes.POINTER(_p)]),
    "ancha_hip_block_workspace": (_sz, [_p, _sz]),
    "ancha_hip_block_forward": (_int, [_p, _p, _sz, _sz, _p, _p, _sz, _p, _p]),
    "ancha_hip_block_destroy": (None, [_p]),
    "ancha_hip_swap_axes": (_int, [_p, _sz, _sz, _sz, _sz, _p, _p]),
    "ancha_hip_axis_pair_workspace": (_sz, [_p, _p, _sz]),
    "ancha_hip_axis_pair_forward": (_int, [_p, _p, _p, _sz, _sz, _sz, _p, _p, _p, _sz, _p, _p]),
    "ancha_hip_roformer_create": (_int, [_p, _p, _p, ctypes.POINTER(_p)]),
    "ancha_hip_roformer_workspace": (_sz, [_p, _sz]),
    "ancha_hip_roformer_forward": (_int, [_p, _p, _sz, _p, _sz, _p, _p, _p]),
    "ancha_hip_chunk_plan": (_int, [_sz, _sz, _sz, ctypes.POINTER(_sz), ctypes.POINTER(_sz)]),
    "ancha_hip_separate_workspace": (_sz, [_p, _sz]),
    "ancha_hip_separate": (_int, [_p, _p, _sz, _p, _sz, _p, _p, _p, _p]),
    "ancha_hip_roformer_destroy": (None, [_p]),
    "ancha_hip_stft": (_int, [_p, _sz, _sz, _p, _p]),
    "ancha_hip_istft_workspace": (_sz, [_sz]),
    "ancha_hip_istft": (_int, [_p, _p, _sz, _sz, _sz, _int, _p, _sz, _p, _p]),
    "ancha_hip_istft_noalloc": (_int, [_p, _p, _sz, _sz, _sz, _int, _p, _p]),
    "ancha_hip_check": (_int, []),
    "ancha_hip_last_error": (ctypes.c_char_p, []),
}


def lib() -> ctypes.CDLL:
    """The loaded library; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `make -C {CSRC}` "
                "(or __graft_entry__.build()); there is no non-HIP fallback")
        l = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(l, name, None)
            if fn is None:
                continue
            fn.restype = res
            fn.argtypes = args
        _lib = l
    return _lib


def last_error() -> str:
    return (lib().ancha_hip_last_error() or b"").decode()


def check(rc: int) -> bool:
    """Map a C-ABI return code: True on success, False for UNSUPPORTED (the reference's
    ``None``), raise for contract violations and HIP failures."""
    if rc == OK:
        return True
    if rc == UNSUPPORTED:
        return False
    if rc == INVALID:
        raise ValueError(last_error())
    if rc == CANCELLED:
        raise Cancelled(last_error())
    raise HipError(f"{last_error()} (code {rc})")
