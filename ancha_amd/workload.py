"""Seeded synthetic workloads for the fused RoFormer attention path, plus the host-side rotary
table of the reference's AxisRope (crates/ancha-models/src/roformer.rs:282-308).

Inputs are N(0, scale^2) streams: splitmix64 -> 53-bit uniform -> Box-Muller, one seed per
tensor (q=1, k=2, v=3, x=4, weights=100+index, audio=7). Element i of a stream uses splitmix64
outputs 2*(i//2) and 2*(i//2)+1 (cosine branch for even i, sine for odd i), so slices can be
generated independently and in chunks.
"""
from __future__ import annotations

import numpy as np

GAMMA = np.uint64(0x9E3779B97F4A7C15)
M1 = np.uint64(0xBF58476D1CE4E5B9)
M2 = np.uint64(0x94D049BB133111EB)

SEED_Q, SEED_K, SEED_V, SEED_X, SEED_AUDIO = 1, 2, 3, 4, 7
SEED_WEIGHTS = 100

# Time-axis op: 2 chunks x 60 bands, 801 STFT frames, 8 heads of 64.
TIME_SHAPE = (120, 801, 8, 64)
# Band-axis op: 2 chunks x 801 frames, 60 bands.
BAND_SHAPE = (1602, 60, 8, 64)


def _splitmix(seed: int, index: np.ndarray) -> np.ndarray:
    with np.errstate(over="ignore"):
        z = np.uint64(seed) + (index + np.uint64(1)) * GAMMA
        z = (z ^ (z >> np.uint64(30))) * M1
        z = (z ^ (z >> np.uint64(27))) * M2
    return z ^ (z >> np.uint64(31))


def normal(shape, seed: int, scale: float = 1.0, first: int = 0,
           chunk: int = 1 << 22) -> np.ndarray:
    """float32 N(0, scale^2) stream elements [first, first + prod(shape))."""
    n = int(np.prod(shape))
    out = np.empty(n, dtype=np.float32)
    two_pi = 2.0 * np.pi
    for c0 in range(0, n, chunk):
        idx = np.arange(first + c0, first + min(n, c0 + chunk), dtype=np.uint64)
        pair = idx >> np.uint64(1)
        z1 = _splitmix(seed, pair * np.uint64(2))
        z2 = _splitmix(seed, pair * np.uint64(2) + np.uint64(1))
        u1 = 1.0 - (z1 >> np.uint64(11)).astype(np.float64) * 2.0 ** -53
        u2 = (z2 >> np.uint64(11)).astype(np.float64) * 2.0 ** -53
        r = np.sqrt(-2.0 * np.log(u1))
        odd = (idx & np.uint64(1)).astype(bool)
        z = np.where(odd, r * np.sin(two_pi * u2), r * np.cos(two_pi * u2))
        out[c0:c0 + idx.size] = (z * scale).astype(np.float32)
    return out.reshape(shape)


def _i64(c: int) -> int:
    return c - (1 << 64) if c >= 1 << 63 else c


def normal_torch(shape, seed: int, scale: float = 1.0, device=None, first: int = 0,
                 chunk: int = 1 << 24):
    """The same stream as :func:`normal`, generated with torch on `device` (wrapping int64
    arithmetic, logical shifts emulated with masks): seconds instead of minutes for the
    full-size operands."""
    import torch

    n = int(np.prod(shape))
    out = torch.empty(n, dtype=torch.float32, device=device)
    gamma, m1, m2 = _i64(int(GAMMA)), _i64(int(M1)), _i64(int(M2))

    def lsr(z, k):
        return (z >> k) & ((1 << (64 - k)) - 1)

    def mix(i):
        z = (i + 1) * gamma + seed
        z = (z ^ lsr(z, 30)) * m1
        z = (z ^ lsr(z, 27)) * m2
        return z ^ lsr(z, 31)

    for c0 in range(0, n, chunk):
        idx = torch.arange(first + c0, first + min(n, c0 + chunk), dtype=torch.int64,
                           device=device)
        pair = idx >> 1
        u1 = 1.0 - lsr(mix(2 * pair), 11).to(torch.float64) * 2.0 ** -53
        u2 = lsr(mix(2 * pair + 1), 11).to(torch.float64) * 2.0 ** -53
        r = torch.sqrt(-2.0 * torch.log(u1))
        ang = (2.0 * np.pi) * u2
        z = torch.where((idx & 1).bool(), r * torch.sin(ang), r * torch.cos(ang))
        out[c0:c0 + idx.numel()] = (z * scale).to(torch.float32)
    return out.reshape(shape)


def rope_freqs(head_dim: int = 64, theta: float = 10000.0) -> np.ndarray:
    """f_i = theta^(-2i/head_dim), i < head_dim/2 (the rotary-embedding-torch default)."""
    i = np.arange(head_dim // 2, dtype=np.float64)
    return (theta ** (-2.0 * i / head_dim)).astype(np.float32)


def axis_rope_packed(freqs: np.ndarray, tokens: int) -> np.ndarray:
    """AxisRope::packed (roformer.rs:282-302): [4, tokens, 2*nf] = query cos, query signed sin
    (both times 1/sqrt(2*nf)), key cos, key signed sin; angle = f32(t) * f32(f)."""
    f = np.asarray(freqs, dtype=np.float32)
    width = 2 * f.size
    scale = np.float32(1.0) / np.sqrt(np.float32(width))
    angle = (np.arange(tokens, dtype=np.float32)[:, None] * f[None, :]).astype(np.float64)
    s = np.sin(angle).astype(np.float32)
    c = np.cos(angle).astype(np.float32)
    cos2 = np.repeat(c, 2, axis=1)
    sin2 = np.stack([-s, s], axis=2).reshape(tokens, width)
    return np.stack([cos2 * scale, sin2 * scale, cos2, sin2]).astype(np.float32)


def attention_inputs(shape, scale: float = 1.0 / 8.0):
    """q, k, v float32 [G, T, H, 64] ~ N(0, scale^2) from seeds 1, 2, 3 (token-major order)."""
    return tuple(normal(shape, seed, scale) for seed in (SEED_Q, SEED_K, SEED_V))
