"""ancha_amd: the MI355X-native (gfx950) fused RoFormer attention path of Ancha.

The compute lives in hand-written HIP kernels behind the C ABI of ``include/ancha_hip.h``
(``ancha_amd/_lib/libancha_hip.so``); :mod:`ancha_amd.fused` mirrors the reference's
``ancha_models::fused`` op boundary on top of it.
"""
from . import fused  # noqa: F401
from ._native import HipError, LIB_PATH, build  # noqa: F401

__all__ = ["fused", "HipError", "LIB_PATH", "build"]
