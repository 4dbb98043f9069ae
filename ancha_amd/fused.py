"""Host mirror of Ancha's op boundary ``ancha_models::fused``
(crates/ancha-models/src/fused/mod.rs) over the gfx950 C ABI.

Same names, argument meanings and error behaviour as the reference: each op returns ``None``
when the shape (or device) is outside what the kernels cover, so callers keep their own
implementation as the fallback; contract violations raise. Tensors are torch tensors on the
GPU, used only as device memory; all arithmetic runs in the HIP kernels.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import torch

from . import _native

ATTENTION_HEAD_DIM = 64


def available() -> bool:
    """fused/mod.rs:250-255: whether the kernels can run on the current device."""
    if not torch.cuda.is_available():
        return False
    return bool(_native.lib().ancha_hip_available())


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _rows(t: torch.Tensor) -> tuple[torch.Tensor, int]:
    """View t [G, T, ...] as [G, T, row] with dense rows and a uniform row stride, as the
    kernels read it (fused/attention.rs:230-237 vector_ready); copies when the layout does not
    allow that view. Returns the view and its row stride in elements."""
    if t.dtype != torch.float32:
        raise ValueError("fused ops take float32 tensors")
    g, tok = t.shape[0], t.shape[1]
    try:
        flat = t.view(g, tok, -1)
    except RuntimeError:
        flat = t.contiguous().view(g, tok, -1)
    if flat.stride(2) != 1 or flat.stride(0) != tok * flat.stride(1):
        flat = flat.contiguous()
    return flat, flat.stride(1)


def _table(rope: Optional[torch.Tensor], tokens: int) -> Optional[torch.Tensor]:
    if rope is None:
        return None
    if tuple(rope.shape) != (4, tokens, ATTENTION_HEAD_DIM) or rope.dtype != torch.float32:
        raise ValueError("rotary table must be float32 [4, tokens, 64]")
    return rope.contiguous()


def attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
              rope: Optional[torch.Tensor] = None) -> Optional[torch.Tensor]:
    """fused/mod.rs:22-41: softmax(q.k^T).v per (group, head) over [groups, tokens, heads, 64]
    tensors with q already scaled; returns [groups, tokens, heads, 64] or None.

    ``rope`` (an extension of the reference signature) is the packed [4, tokens, 64] table of
    AxisRope::packed; when given, q and k are rotated as they are loaded (q unscaled: the
    query table carries 1/sqrt(64))."""
    if q.dim() != 4 or q.shape[3] != ATTENTION_HEAD_DIM or k.shape != q.shape or v.shape != q.shape:
        return None
    if not q.is_cuda or not available():
        return None
    groups, tokens, heads, _ = q.shape
    (qf, ldq), (kf, ldk), (vf, ldv) = (_rows(t) for t in (q, k, v))
    table = _table(rope, tokens)
    out = torch.empty((groups, tokens, heads, ATTENTION_HEAD_DIM), device=q.device,
                      dtype=torch.float32)
    rc = _native.lib().ancha_hip_attention(
        qf.data_ptr(), kf.data_ptr(), vf.data_ptr(), groups, tokens, heads, ldq, ldk, ldv,
        _ptr(table), out.data_ptr(), _stream())
    return out if _native.check(rc) else None


def gated_attention(packed: torch.Tensor, heads: int,
                    rope: Optional[torch.Tensor] = None) -> Optional[torch.Tensor]:
    """fused/mod.rs:47-55: the RoFormer attention core from one packed projection
    [groups, tokens, columns] = q | k | v | per-head gate logits | ...;
    softmax(q.k^T).v * sigmoid(gate) as [groups, tokens, heads, 64], or None."""
    if packed.dim() != 3 or packed.shape[2] < heads * (3 * ATTENTION_HEAD_DIM + 1):
        return None
    if not packed.is_cuda or not available():
        return None
    groups, tokens, columns = packed.shape
    flat, ld = _rows(packed)
    if ld != columns:
        flat, ld = flat.contiguous(), columns
    table = _table(rope, tokens)
    out = torch.empty((groups, tokens, heads, ATTENTION_HEAD_DIM), device=packed.device,
                      dtype=torch.float32)
    rc = _native.lib().ancha_hip_gated_attention(
        flat.data_ptr(), groups, tokens, columns, heads, _ptr(table), out.data_ptr(), _stream())
    return out if _native.check(rc) else None


@dataclass
class Epilogue:
    """fused/mod.rs:58-79: work fused into the output pass of :func:`linear`, applied in
    field order."""
    bias: Optional[torch.Tensor] = None
    gelu: bool = False
    rotary: Optional[tuple[torch.Tensor, int]] = None
    residual: Optional[torch.Tensor] = None

    def empty(self) -> bool:
        return (self.bias is None and not self.gelu and self.rotary is None
                and self.residual is None)
