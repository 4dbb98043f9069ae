"""Host mirror of the RoFormer block of crates/ancha-models/src/roformer.rs on the gfx950 C ABI.

``Transformer`` packs one block's weights at load time (``Transformer::load`` /
``Attention::load``, roformer.rs:205-244 and :381-409) and runs ``forward_kernels``
(:464-520): packed q|k|v|gate GEMM with the row norm fused and RoPE in its epilogue, gated
attention, output GEMM (+x), feed-forward GEMMs (norm, bias, GELU; bias, +x), optional output
norm. All arithmetic runs in libancha_hip.so; torch provides device memory and the stream.
"""
from __future__ import annotations

import ctypes
from typing import Optional

import numpy as np
import torch

from . import _native
from ._tensors import require
from .workload import axis_rope_packed

WEIGHT_NAMES = ("attn_gamma", "to_qkv", "to_gates", "to_gates_bias", "to_out", "ff_gamma",
                "ff_in", "ff_in_bias", "ff_out", "ff_out_bias", "output_gamma")


def axis_rope(freqs, tokens: int, device) -> torch.Tensor:
    """AxisRope::new (roformer.rs:282-302): the packed [4, tokens, 64] table of one axis, on
    ``device``. Built per forward and axis, like the reference."""
    return torch.from_numpy(axis_rope_packed(np.asarray(freqs, np.float32), tokens)).to(device)


class Transformer:
    """One block; ``weights`` maps the names of WEIGHT_NAMES (PyTorch nn.Linear layouts,
    float32; ``output_gamma`` optional) plus ``heads``."""

    def __init__(self, weights: dict, device: Optional[torch.device] = None):
        self.device = torch.device(device or "cuda")
        host = {}
        for name in WEIGHT_NAMES:
            w = weights.get(name)
            host[name] = None if w is None else np.ascontiguousarray(w, dtype=np.float32)
        self.heads = int(weights["heads"])
        self.hidden, self.dim = host["ff_in"].shape
        ptr = lambda a: None if a is None else a.ctypes.data
        handle = ctypes.c_void_p()
        with torch.cuda.device(self.device):
            rc = _native.lib().ancha_hip_block_create(
                self.dim, self.heads, self.hidden, *(ptr(host[n]) for n in WEIGHT_NAMES),
                ctypes.byref(handle))
        if not _native.check(rc):
            raise ValueError("block shapes are outside what the kernels cover "
                             "(linear_supported fails for a projection)")
        self._handle = handle
        self._workspace: Optional[torch.Tensor] = None

    def workspace_bytes(self, rows: int) -> int:
        return int(_native.lib().ancha_hip_block_workspace(self._handle, rows))

    def forward(self, x: torch.Tensor, rope: torch.Tensor) -> torch.Tensor:
        """x [groups, tokens, dim] float32 on the block's device; rope the [4, tokens, 64]
        table of this axis. Returns a new [groups, tokens, dim] tensor."""
        if x.dim() != 3:
            raise ValueError("x must be [groups, tokens, dim]")
        groups, tokens, dim = x.shape
        require(x, "x", self.device, (groups, tokens, self.dim))
        require(rope, "rope", self.device, (4, tokens, 64))
        x = x.contiguous()
        rope = rope.contiguous()
        need = self.workspace_bytes(groups * tokens)
        if self._workspace is None or self._workspace.numel() < need:
            self._workspace = torch.empty(need, dtype=torch.uint8, device=self.device)
        out = torch.empty_like(x)
        rc = _native.lib().ancha_hip_block_forward(
            self._handle, x.data_ptr(), groups, tokens, rope.data_ptr(),
            self._workspace.data_ptr(), self._workspace.numel(), out.data_ptr(),
            torch.cuda.current_stream(self.device).cuda_stream)
        if not _native.check(rc):
            raise ValueError("block forward rejected the shapes")
        return out

    __call__ = forward

    def close(self) -> None:
        if self._handle:
            _native.lib().ancha_hip_block_destroy(self._handle)
            self._handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def swap_axes(x: torch.Tensor) -> torch.Tensor:
    """Dense ``x.swap_dims(1, 2)`` of a [batch, a, b, dim] float32 tensor on the GPU
    (network.rs:336-338)."""
    if x.dim() != 4 or x.dtype != torch.float32 or not x.is_cuda:
        raise ValueError("swap_axes takes a float32 CUDA [batch, a, b, dim] tensor")
    x = x.contiguous()
    batch, a, b, dim = x.shape
    out = torch.empty((batch, b, a, dim), device=x.device, dtype=torch.float32)
    _native.check(_native.lib().ancha_hip_swap_axes(x.data_ptr(), batch, a, b, dim,
                                                    out.data_ptr(),
                                                    torch.cuda.current_stream().cuda_stream))
    return out


class AxisPair:
    """One time pass + band pass of the RoFormer axis loop (network.rs:333-339) over
    x [batch, bands, frames, dim]: the time block on groups = batch*bands (sequence = frames),
    an axis swap, the band block on groups = batch*frames (sequence = bands), a swap back."""

    def __init__(self, time: Transformer, band: Transformer):
        if time.dim != band.dim:
            raise ValueError("time and band blocks must share dim")
        self.time, self.band = time, band
        self._workspace: Optional[torch.Tensor] = None

    def forward(self, x: torch.Tensor, time_rope: torch.Tensor,
                band_rope: torch.Tensor) -> torch.Tensor:
        if x.dim() != 4:
            raise ValueError("x must be [batch, bands, frames, dim]")
        batch, bands, frames, dim = x.shape
        require(x, "x", self.time.device, (batch, bands, frames, self.time.dim))
        require(time_rope, "time_rope", self.time.device, (4, frames, 64))
        require(band_rope, "band_rope", self.time.device, (4, bands, 64))
        x = x.contiguous()
        lib = _native.lib()
        need = int(lib.ancha_hip_axis_pair_workspace(self.time._handle, self.band._handle,
                                                     batch * bands * frames))
        if self._workspace is None or self._workspace.numel() < need:
            self._workspace = torch.empty(need, dtype=torch.uint8, device=x.device)
        out = torch.empty_like(x)
        rc = lib.ancha_hip_axis_pair_forward(
            self.time._handle, self.band._handle, x.data_ptr(), batch, bands, frames,
            time_rope.contiguous().data_ptr(), band_rope.contiguous().data_ptr(),
            self._workspace.data_ptr(), self._workspace.numel(), out.data_ptr(),
            torch.cuda.current_stream().cuda_stream)
        if not _native.check(rc):
            raise ValueError("axis pair rejected the shapes")
        return out

    __call__ = forward
