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
from ._tensors import require, require_optional

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


def _table(rope: Optional[torch.Tensor], tokens: int,
           device: torch.device) -> Optional[torch.Tensor]:
    if rope is None:
        return None
    require(rope, "rotary table", device, (4, tokens, ATTENTION_HEAD_DIM))
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
    for name, t in (("q", q), ("k", k), ("v", v)):
        require(t, name, q.device)
    groups, tokens, heads, _ = q.shape
    (qf, ldq), (kf, ldk), (vf, ldv) = (_rows(t) for t in (q, k, v))
    table = _table(rope, tokens, q.device)
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
    require(packed, "packed", packed.device)
    groups, tokens, columns = packed.shape
    flat, ld = _rows(packed)
    if ld != columns:
        flat, ld = flat.contiguous(), columns
    table = _table(rope, tokens, packed.device)
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


def linear_supported(k: int, m: int) -> bool:
    """fused/mod.rs:83-85: the 128-wide tile covers [n, k].[k, m] without padding."""
    return k > 0 and k % 8 == 0 and m > 0 and m % 128 == 0


def _matrix(t: torch.Tensor, name: str, device: torch.device) -> torch.Tensor:
    require(t, name, device)
    return t if t.stride(1) == 1 else t.contiguous()


def _linear(x: torch.Tensor, weight: torch.Tensor, epilogue: Epilogue,
            norm: bool) -> Optional[torch.Tensor]:
    n, k = x.shape
    rows, m = weight.shape
    if rows != k or k == 0 or k % 8 != 0 or m == 0:
        return None
    if m % 128 != 0 and not epilogue.empty():
        return None
    tokens = width = 0
    table = None
    if epilogue.rotary is not None:
        table, width = epilogue.rotary
        four, tokens, dim = table.shape
        if four != 4 or dim != ATTENTION_HEAD_DIM or n % tokens != 0 or width % 64 != 0 \
                or 2 * width > m:
            return None
        table = table.contiguous()
    residual = epilogue.residual
    if residual is not None:
        if tuple(residual.shape) != (n, m):
            return None
        residual = residual.contiguous()
    if not x.is_cuda or not available():
        return None
    x = _matrix(x, "x", x.device)
    w = _matrix(weight, "weight", x.device).contiguous()
    require_optional(epilogue.bias, "bias", x.device, (m,))
    require_optional(residual, "residual", x.device, (n, m))
    if table is not None:
        require(table, "rotary table", x.device)
    bias = None if epilogue.bias is None else epilogue.bias.contiguous()
    out = torch.empty((n, m), device=x.device, dtype=torch.float32)
    fn = _native.lib().ancha_hip_norm_linear if norm else _native.lib().ancha_hip_linear
    rc = fn(x.data_ptr(), n, k, x.stride(0), w.data_ptr(), m, _ptr(bias), int(epilogue.gelu),
            _ptr(table), tokens, width, _ptr(residual), out.data_ptr(), _stream())
    return out if _native.check(rc) else None


def linear(x: torch.Tensor, weight: torch.Tensor,
           epilogue: Optional[Epilogue] = None) -> Optional[torch.Tensor]:
    """fused/mod.rs:100-176: x [n, k] . weight [k, m] (Burn Linear layout) followed by the
    epilogue (bias -> erf-GELU -> rotary -> residual); [n, m] or None when the shape or the
    epilogue does not fit (k % 8, m % 128 with an epilogue, rotary shape, residual shape)."""
    return _linear(x, weight, epilogue or Epilogue(), norm=False)


def norm_linear(x: torch.Tensor, weight: torch.Tensor,
                epilogue: Optional[Epilogue] = None) -> Optional[torch.Tensor]:
    """``linear(unit_norm(x), weight, epilogue)`` in one kernel (the row norm scales the
    product), the call pattern of Transformer::forward_kernels (roformer.rs:477-485, :497-505)."""
    return _linear(x, weight, epilogue or Epilogue(), norm=True)


def unit_norm(x: torch.Tensor, scale: Optional[torch.Tensor] = None) -> torch.Tensor:
    """roformer.rs:16-24 (and SourceNorm::forward :51-53 with scale = sqrt(dim)*gamma):
    x / max(||x||_2, 1e-12) over the last axis, times ``scale``."""
    if x.dtype != torch.float32 or not x.is_cuda:
        raise ValueError("unit_norm takes a float32 CUDA tensor")
    dim = x.shape[-1]
    require_optional(scale, "scale", x.device, (dim,))
    if not available():
        raise RuntimeError("the gfx950 kernels cannot run on this device")
    flat = x.reshape(-1, dim)
    if flat.stride(1) != 1:
        flat = flat.contiguous()
    out = torch.empty(x.shape, device=x.device, dtype=torch.float32)
    s = None if scale is None else scale.contiguous()
    rc = _native.lib().ancha_hip_unit_norm(flat.data_ptr(), flat.shape[0], dim, flat.stride(0),
                                           _ptr(s), out.data_ptr(), _stream())
    _native.check(rc)
    return out
