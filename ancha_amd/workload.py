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


def roformer_tensor_shapes(config: dict) -> dict:
    """Checkpoint tensor names and shapes of a Mel/BS-RoFormer (network.rs:96-177,
    roformer.rs:205-252 and :381-409), in a fixed order."""
    dim, heads, hd = config["dim"], config["heads"], config["head_dim"]
    inner, hidden = heads * hd, dim * config["ff_mult"]
    mh = dim * config["mask_expansion"]
    mel = config["family"] == "mel-band-roformer"
    shapes = {}
    for b, bins in enumerate(config["bands"]):
        w = 4 * len(bins)
        p = f"band_split.to_features.{b}"
        shapes[f"{p}.0.gamma"] = (w,)
        shapes[f"{p}.1.weight"] = (dim, w)
        shapes[f"{p}.1.bias"] = (dim,)
    for i in range(config["depth"]):
        for axis in range(2):
            p = f"layers.{i}.{axis}"
            a, f = f"{p}.layers.0.0", f"{p}.layers.0.1.net"
            shapes[f"{a}.norm.gamma"] = (dim,)
            shapes[f"{a}.to_qkv.weight"] = (3 * inner, dim)
            shapes[f"{a}.to_gates.weight"] = (heads, dim)
            shapes[f"{a}.to_gates.bias"] = (heads,)
            shapes[f"{a}.to_out.0.weight"] = (dim, inner)
            shapes[f"{a}.rotary_embed.freqs"] = (hd // 2,)
            shapes[f"{f}.0.gamma"] = (dim,)
            shapes[f"{f}.1.weight"] = (hidden, dim)
            shapes[f"{f}.1.bias"] = (hidden,)
            shapes[f"{f}.4.weight"] = (dim, hidden)
            shapes[f"{f}.4.bias"] = (dim,)
            if mel:
                shapes[f"{p}.norm.gamma"] = (dim,)
    if not mel:
        shapes["final_norm.gamma"] = (dim,)
    layers = config["mask_depth"] if mel else config["mask_depth"] - 1
    for s in range(len(config["stems"])):
        for b, bins in enumerate(config["bands"]):
            p = f"mask_estimators.{s}.to_freqs.{b}.0"
            fan_in = dim
            for layer in range(layers):
                shapes[f"{p}.{2 * layer}.weight"] = (mh, fan_in)
                shapes[f"{p}.{2 * layer}.bias"] = (mh,)
                fan_in = mh
            shapes[f"{p}.{2 * layers}.weight"] = (8 * len(bins), mh)
            shapes[f"{p}.{2 * layers}.bias"] = (8 * len(bins),)
    return shapes


def roformer_tensors(config: dict, seed: int = SEED_WEIGHTS, scale: float = 0.02,
                     device=None) -> dict:
    """Random-init checkpoint: gammas 1, rotary frequencies theta = 10000, every other tensor
    N(0, scale^2) from one seeded stream, consumed in roformer_tensor_shapes order. With a
    torch `device` the stream is generated there (same values) and copied back."""
    shapes = roformer_tensor_shapes(config)
    random = [(n, s) for n, s in shapes.items() if not n.endswith(("gamma", "freqs"))]
    total = sum(int(np.prod(s)) for _, s in random)
    if device is not None:
        flat = normal_torch((total,), seed, scale, device=device).cpu().numpy()
    else:
        flat = normal((total,), seed, scale)
    out, first = {}, 0
    for name, shape in shapes.items():
        if name.endswith("gamma"):
            out[name] = np.ones(shape, np.float32)
        elif name.endswith("freqs"):
            out[name] = rope_freqs(2 * shape[0])
        else:
            size = int(np.prod(shape))
            out[name] = flat[first:first + size].reshape(shape)
            first += size
    return out


def audio(samples: int, seed: int = SEED_AUDIO, sample_rate: int = 44100) -> np.ndarray:
    """Stereo test audio [2, samples]: pink noise (Paul Kellet's filter on a seeded N(0, 1)
    stream, scaled to ~0.1 RMS) plus three sines at seeded frequencies and amplitudes."""
    from scipy.signal import lfilter

    white = normal((2, samples), seed, 1.0).astype(np.float64)
    out = np.empty((2, samples), np.float64)
    poles = (0.99886, 0.99332, 0.96900, 0.86650, 0.55000, -0.7616)
    gains = (0.0555179, 0.0750759, 0.1538520, 0.3104856, 0.5329522, -0.0168980)
    for c in range(2):
        w = white[c]
        y = w * 0.5362
        for a, g in zip(poles, gains):  # b_k[n] = a b_k[n-1] + g w[n]
            y = y + lfilter([g], [1.0, -a], w)
        y[1:] += 0.115926 * w[:-1]  # b_6: the previous sample's 0.115926 w
        out[c] = y * (0.1 / max(np.std(y), 1e-12))
    params = normal((3, 3), seed + 1, 1.0).astype(np.float64)
    t = np.arange(samples) / sample_rate
    for k in range(3):
        freq = 110.0 * 2.0 ** (abs(params[k, 0]) * 2.0)
        amp = 0.05 + 0.05 * abs(params[k, 1])
        phase = params[k, 2]
        tone = amp * np.sin(2 * np.pi * freq * t + phase)
        out[0] += tone
        out[1] += tone * (0.8 if k % 2 else 1.0)
    return out.astype(np.float32)


def attention_inputs(shape, scale: float = 1.0 / 8.0):
    """q, k, v float32 [G, T, H, 64] ~ N(0, scale^2) from seeds 1, 2, 3 (token-major order)."""
    return tuple(normal(shape, seed, scale) for seed in (SEED_Q, SEED_K, SEED_V))
