"""Inputs of the golden fixtures, regenerated from closed forms (shared by make_golden.py and
the tests). Mirrors the reference's test inputs: `wave` is tests/cuda_contracts.rs:183-189."""
from __future__ import annotations

import numpy as np

from ancha_amd import workload as W

# tests/cuda_contracts.rs:199-204: partial tiles, a single token, a strided layout.
ATTENTION_SHAPES = [(2, 1, 1), (3, 63, 2), (2, 65, 1), (1, 130, 3)]

# tests/cuda_contracts.rs:253-295: the GEMM epilogue case.
LINEAR_GROUPS, LINEAR_TOKENS, LINEAR_K, LINEAR_HEADS = 3, 70, 64, 2
LINEAR_WIDTH = LINEAR_HEADS * 64
LINEAR_GELU_ROWS = np.arange(0, 210, 7)          # 30 of the 210 rows
LINEAR_ROTARY_ROWS = np.arange(70, 140)          # one whole group: every token position

# Single-group slices of the two production shapes (seeds 1/2/3, N(0,1)/8, RoPE on load).
SLICES = {
    "time": ((1, 801, 8, 64), np.r_[np.arange(0, 768, 8), np.arange(768, 801)], [0, 5]),
    "band": ((1, 60, 8, 64), np.arange(60), [0, 7]),
}

# A small RoFormer block (dim 128, 2 heads, FF 512, output norm) on [3, 37, 128].
LAYER_DIM, LAYER_HEADS, LAYER_HIDDEN, LAYER_SHAPE = 128, 2, 512, (3, 37, 128)


def wave(shape, shift):
    n = int(np.prod(shape))
    i = np.arange(n, dtype=np.float32)
    return np.tanh(np.sin(i * np.float32(0.731) + np.float32(shift)) * np.float32(1.7)).astype(
        np.float32).reshape(shape)


def checksum(*arrays):
    """Float64 sums of each input and of its elements weighted by position (order-sensitive)."""
    out = []
    for a in arrays:
        a = np.asarray(a, np.float64).ravel()
        out += [a.sum(), (a * (np.arange(a.size) % 97 + 1)).sum()]
    return np.array(out)


def attention_case(groups, tokens, heads):
    """q (pre-scaled by 1/8), k, v [G, T, H, 64]; gates [G, T, H]; the packed
    q | k | v | gates | 5 zero columns layout of the same values."""
    q = wave((groups, tokens, heads, 64), 0.1) * np.float32(0.4) * np.float32(0.125)
    k = wave((groups, tokens, heads, 64), 1.3)
    v = wave((groups, tokens, heads, 64), 2.9)
    gates = wave((groups, tokens, heads), 4.4) * np.float32(3.0)
    flat = lambda a: a.reshape(groups, tokens, heads * 64)
    packed = np.concatenate([flat(q), flat(k), flat(v), gates,
                             np.zeros((groups, tokens, 5), np.float32)], axis=2)
    return q, k, v, gates, packed


def linear_case():
    rows, m = LINEAR_GROUPS * LINEAR_TOKENS, 3 * LINEAR_WIDTH
    x = wave((rows, LINEAR_K), 0.3)
    w = wave((LINEAR_K, m), 1.1) * np.float32(0.1)
    b = wave((m,), 2.2)
    r = wave((rows, m), 3.3)
    freqs = (np.float32(10000.0) ** (-np.arange(32, dtype=np.float32) / np.float32(32.0))).astype(
        np.float32)
    return x, w, b, r, W.axis_rope_packed(freqs, LINEAR_TOKENS), freqs


def slice_case(shape):
    q, k, v = W.attention_inputs(shape)
    freqs = W.rope_freqs()
    return q, k, v, W.axis_rope_packed(freqs, shape[1]), freqs


def layer_case():
    shapes = {
        "attn_gamma": (LAYER_DIM,), "to_qkv": (3 * LAYER_HEADS * 64, LAYER_DIM),
        "to_gates": (LAYER_HEADS, LAYER_DIM), "to_gates_bias": (LAYER_HEADS,),
        "to_out": (LAYER_DIM, LAYER_HEADS * 64), "ff_gamma": (LAYER_DIM,),
        "ff_in": (LAYER_HIDDEN, LAYER_DIM), "ff_in_bias": (LAYER_HIDDEN,),
        "ff_out": (LAYER_DIM, LAYER_HIDDEN), "ff_out_bias": (LAYER_DIM,),
        "output_gamma": (LAYER_DIM,),
    }
    w = {"heads": LAYER_HEADS, "freqs": W.rope_freqs()}
    for i, (name, shape) in enumerate(sorted(shapes.items())):
        if name.endswith("gamma"):
            w[name] = 1.0 + W.normal(shape, W.SEED_WEIGHTS + i, 0.1)
        else:
            w[name] = W.normal(shape, W.SEED_WEIGHTS + i, 0.02)
    return w, W.normal(LAYER_SHAPE, 4)


# Tiny networks at the reference's kernel_package scale (tests/support/mod.rs:18-55): dim 128,
# 2 heads of 64, FF x4, a 101-frame chunk. Mel: two stems, three overlapping bands (the
# coverage average), mask depth 2 = two tanh hidden layers. BS: one stem, three bands that
# partition the bins, a final norm, mask depth 2 = one hidden layer (every Linear counted).
NETWORKS = ("mel", "bs")
NETWORK_ROWS = np.arange(0, 2050, 11)        # mask rows kept in the fixture
NETWORK_FRAMES = np.arange(0, 101, 5)        # frames kept in the fixture


def network_config(name):
    config = {"family": "mel-band-roformer" if name == "mel" else "bs-roformer", "dim": 128,
              "depth": 2, "heads": 2, "head_dim": 64, "ff_mult": 4, "mask_depth": 2,
              "mask_expansion": 1, "sample_rate": 44100, "n_fft": 2048, "hop": 441,
              "chunk_samples": 44100, "overlap": 2, "zero_dc": True,
              "stems": ["vocals", "instrumental"] if name == "mel" else ["vocals"]}
    if name == "mel":
        config["bands"] = [list(range(0, 400)), list(range(300, 900)), list(range(625, 1025))]
    else:
        config["bands"] = [list(range(0, 300)), list(range(300, 700)), list(range(700, 1025))]
    return config


def network_case(name):
    """(config, checkpoint tensors, packed spectrum [101, 4100]). Weights N(0, 0.05^2) from
    the seeded stream; every gamma 1 + 0.3 wave(...) (not 1, so a dropped gamma shows); the
    rotary frequencies of layer i, axis a use theta = 10000 / (1 + 2i + a) (so a table built
    from the wrong layer's frequencies shows)."""
    config = network_config(name)
    tensors = W.roformer_tensors(config, seed=W.SEED_WEIGHTS + (7 if name == "mel" else 8),
                                 scale=0.05)
    for i, key in enumerate(sorted(k for k in tensors if k.endswith("gamma"))):
        tensors[key] = (np.float32(1.0) + np.float32(0.3) * wave(tensors[key].shape, 0.37 * i))
    for key in tensors:
        if key.endswith("rotary_embed.freqs"):
            i, axis = int(key.split(".")[1]), int(key.split(".")[2])
            tensors[key] = W.rope_freqs(64, 10000.0 / (1 + 2 * i + axis))
    spectrum = wave((101, 4100), 0.7 if name == "mel" else 1.9) * np.float32(2.0)
    return config, tensors, spectrum


def moments(a):
    """Float64 sum, sum of squares and position-weighted sum of a whole output."""
    a = np.asarray(a, np.float64).ravel()
    return np.array([a.sum(), (a * a).sum(), (a * (np.arange(a.size) % 89 + 1)).sum()])


# The two full-size models at their production chunk shapes, random-init N(0, 0.02^2) weights
# (gammas 1, theta 10000), one chunk of seeded audio through the oracle's STFT:
#   mel_karaoke_d6: Mel-Karaoke (60 overlapping bands, dim 384), depth 6, 801 frames;
#   bs_large_d2:    BS-RoFormer-large (62 bands, dim 512, mask MLP x4), depth 2, 1101 frames.
PRODUCTION = {
    "mel_karaoke_d6": ("mel_karaoke", 6, 51, 52),
    "bs_large_d2": ("bs_roformer_large", 2, 53, 54),
}
PRODUCTION_ROW_STEP, PRODUCTION_FRAME_STEP = 41, 16


def production_config(name):
    from ancha_amd import separation as S
    bundled, depth, _, _ = PRODUCTION[name]
    return dict(S.load_config(bundled), depth=depth)


def production_case(name, device=None):
    """(config, checkpoint tensors, packed spectrum [frames, 4100]); with a torch `device`
    the weight stream is generated there (same values)."""
    import oracle.mel as M
    config = production_config(name)
    _, _, seed, audio_seed = PRODUCTION[name]
    tensors = W.roformer_tensors(config, seed=seed, device=device)
    chunk = W.audio(config["chunk_samples"], seed=audio_seed)
    spectrum = M.pack_spectra([M.stft(chunk[c], config["n_fft"], config["hop"])
                               for c in range(2)])
    return config, tensors, spectrum


# Separations at production depth through the whole runtime (chunking, STFT, forward, masked
# iSTFT, overlap-add), stems kept on a sample lattice plus whole-output moments:
#   mel_karaoke_d6_sep: Mel-Karaoke, depth 6, a clip of exactly one 801-frame chunk's step
#                       (88 200 samples: no border, one chunk start);
#   bs_large_d2_sep:    BS-RoFormer-large, depth 2, a clip of one chunk length (485 100 samples:
#                       no border, two chunk starts, batched through one forward).
# name -> (bundled config, depth, weight seed, audio seed, clip samples)
SEPARATIONS = {
    "mel_karaoke_d6_sep": ("mel_karaoke", 6, 81, 82, 88_200),
    "bs_large_d2_sep": ("bs_roformer_large", 2, 83, 84, 485_100),
}
SEPARATION_SAMPLE_STEP = 29


def separation_case(name, device=None):
    """(config, checkpoint tensors, audio [2, samples]); with a torch `device` the weight
    stream is generated there (same values)."""
    from ancha_amd import separation as S
    bundled, depth, seed, audio_seed, samples = SEPARATIONS[name]
    config = dict(S.load_config(bundled), depth=depth)
    tensors = W.roformer_tensors(config, seed=seed, device=device)
    return config, tensors, W.audio(samples, seed=audio_seed)


def separation_index(samples):
    return np.arange(0, samples, SEPARATION_SAMPLE_STEP)


# The reference's bundled deux model (configs/deux.json: Mel-RoFormer with the Mel-Karaoke
# band table, dim 256, 8 heads, 2 stems, 573 300-sample chunks = 1301 frames) at depth 1.
DEUX = {"deux_d1": (1, 87, 88)}


def deux_config(depth):
    from ancha_amd import separation as S
    return dict(S.load_config("mel_karaoke"), dim=256, depth=depth, chunk_samples=573_300,
                overlap=2, stems=["vocals", "instrumental"])


def deux_case(name, device=None):
    """(config, checkpoint tensors, packed spectrum [1301, 4100])."""
    import oracle.mel as M
    depth, seed, audio_seed = DEUX[name]
    config = deux_config(depth)
    tensors = W.roformer_tensors(config, seed=seed, device=device)
    chunk = W.audio(config["chunk_samples"], seed=audio_seed)
    spectrum = M.pack_spectra([M.stft(chunk[c], config["n_fft"], config["hop"])
                               for c in range(2)])
    return config, tensors, spectrum


def production_index(frames):
    return np.arange(0, 2050, PRODUCTION_ROW_STEP), np.arange(0, frames, PRODUCTION_FRAME_STEP)
