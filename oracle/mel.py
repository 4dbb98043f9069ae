"""Oracle for the Mel/BS-RoFormer model around the attention path: STFT, band split, the axis
loop of transformer blocks, mask heads and the chunked separation runtime. TEST
INFRASTRUCTURE ONLY (see the package docstring): the C parts live in mel_oracle.c, the chunk
bookkeeping below is numpy.

Weights are plain dicts (the same layout the GPU host code takes):
  band_split: list over bands of {"gamma": [w], "weight": [dim, w], "bias": [dim]}, w = 4*bins
  layers:     list over depth of (time block, frequency block); a block is the dict of
              oracle.transformer_forward (PyTorch layouts, "heads", "freqs", output_gamma)
  final_norm: [dim] gamma (BS-RoFormer) or None (Mel: per-block output norms instead)
  masks:      list over stems of {"hidden": [(W [bands, out, in], b [bands, out]) per layer],
                                  "out": [(W [2w_b, hidden], b [2w_b]) per band]}
Config: a dict with the fields of crates/ancha-models/src/config.rs:14-32.
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import _check, _p, _sz, lib, transformer_forward, unit_norm

_declared = False


def _l():
    global _declared
    l = lib()
    if not _declared:
        l.anc_reflect_index.argtypes = [ctypes.c_long, _sz]
        l.anc_reflect_index.restype = _sz
        l.anc_stft.argtypes = [_p, _sz, _sz, _sz, _p]
        l.anc_istft.argtypes = [_p, _sz, _sz, _sz, _sz, ctypes.c_int, _p]
        l.anc_band_split.argtypes = [_p, _sz, _sz, _sz, _p, _p, _sz, _p, _p, _p, _sz, _p]
        l.anc_mask_head.argtypes = [_p, _sz, _sz, _p, _p, _sz, _sz, _sz, _sz, _p, _p, _p, _p,
                                    _sz, _p]
        _declared = True
    return l


def weights_from_tensors(config, tensors):
    """The weights dict above from checkpoint tensors by name (the names of
    network.rs:96-177, roformer.rs:205-252 and :381-409)."""
    mel = config["family"] == "mel-band-roformer"
    t = lambda name: np.asarray(tensors[name], np.float32)
    bands = config["bands"]
    band_split = [{"gamma": t(f"band_split.to_features.{b}.0.gamma"),
                   "weight": t(f"band_split.to_features.{b}.1.weight"),
                   "bias": t(f"band_split.to_features.{b}.1.bias")} for b in range(len(bands))]
    layers = []
    for i in range(config["depth"]):
        pair = []
        for axis in range(2):
            p = f"layers.{i}.{axis}"
            a, f = f"{p}.layers.0.0", f"{p}.layers.0.1.net"
            pair.append({"heads": config["heads"], "attn_gamma": t(f"{a}.norm.gamma"),
                         "to_qkv": t(f"{a}.to_qkv.weight"), "to_gates": t(f"{a}.to_gates.weight"),
                         "to_gates_bias": t(f"{a}.to_gates.bias"),
                         "to_out": t(f"{a}.to_out.0.weight"),
                         "freqs": t(f"{a}.rotary_embed.freqs"), "ff_gamma": t(f"{f}.0.gamma"),
                         "ff_in": t(f"{f}.1.weight"), "ff_in_bias": t(f"{f}.1.bias"),
                         "ff_out": t(f"{f}.4.weight"), "ff_out_bias": t(f"{f}.4.bias"),
                         "output_gamma": t(f"{p}.norm.gamma") if mel else None})
        layers.append(tuple(pair))
    hidden_layers = config["mask_depth"] if mel else config["mask_depth"] - 1
    masks = []
    for s in range(len(config["stems"])):
        key = lambda b, layer: f"mask_estimators.{s}.to_freqs.{b}.0.{2 * layer}"
        hidden = [(np.stack([t(key(b, layer) + ".weight") for b in range(len(bands))]),
                   np.stack([t(key(b, layer) + ".bias") for b in range(len(bands))]))
                  for layer in range(hidden_layers)]
        out = [(t(key(b, hidden_layers) + ".weight"), t(key(b, hidden_layers) + ".bias"))
               for b in range(len(bands))]
        masks.append({"hidden": hidden, "out": out})
    return {"band_split": band_split, "layers": layers,
            "final_norm": None if mel else t("final_norm.gamma"), "masks": masks}


def reflect_index(index: int, length: int) -> int:
    """dsp.rs:139-147."""
    return int(_l().anc_reflect_index(index, length))


def stft(signal, n_fft: int = 2048, hop: int = 441) -> np.ndarray:
    """Stft::forward (dsp.rs:46-84): complex64 [frames, n_fft/2 + 1]."""
    x = np.ascontiguousarray(signal, dtype=np.float32)
    frames, bins = x.size // hop + 1, n_fft // 2 + 1
    out = np.empty((frames, bins, 2), np.float32)
    _check(_l().anc_stft(x.ctypes.data, x.size, n_fft, hop, out.ctypes.data))
    return out[..., 0] + 1j * out[..., 1]


def istft(spectrum, length: int, n_fft: int = 2048, hop: int = 441, zero_dc=False):
    """Stft::inverse (dsp.rs:86-134): float32 [length]."""
    s = np.ascontiguousarray(np.stack([spectrum.real, spectrum.imag], -1), dtype=np.float32)
    out = np.empty(length, np.float32)
    _check(_l().anc_istft(s.ctypes.data, s.shape[0], n_fft, hop, length, int(zero_dc),
                          out.ctypes.data))
    return out


def _reflect(index, length: int) -> np.ndarray:
    """reflect_index over an index array (dsp.rs:139-147)."""
    index = np.asarray(index, np.int64)
    if length <= 1:
        return np.zeros_like(index)
    period = 2 * (length - 1)
    i = np.mod(index, period)
    return np.where(i < length, i, period - i)


def _bands(config):
    bands = config["bands"]
    offsets = np.zeros(len(bands) + 1, np.uintp)
    offsets[1:] = np.cumsum([len(b) for b in bands])
    bins = np.ascontiguousarray(np.concatenate([np.asarray(b) for b in bands]), np.uintp)
    return offsets, bins


def band_split(spectrum, config, weights, threads=1):
    """network.rs:316-323: packed spectrum [t, 4*bins] -> x [bands, t, dim]."""
    z = np.ascontiguousarray(spectrum, np.float32)
    t, cols = z.shape
    offsets, bins = _bands(config)
    bs = weights["band_split"]
    dim = bs[0]["weight"].shape[0]
    gamma = np.ascontiguousarray(np.concatenate([b["gamma"] for b in bs]), np.float32)
    weight = np.ascontiguousarray(np.concatenate([b["weight"].ravel() for b in bs]), np.float32)
    bias = np.ascontiguousarray(np.concatenate([b["bias"] for b in bs]), np.float32)
    x = np.empty((len(bs), t, dim), np.float32)
    _check(_l().anc_band_split(z.ctypes.data, t, cols, len(bs), offsets.ctypes.data,
                               bins.ctypes.data, dim, gamma.ctypes.data, weight.ctypes.data,
                               bias.ctypes.data, threads, x.ctypes.data))
    return x


def mask_head(x, config, head, threads=1):
    """network.rs:374-398 for one stem: x [bands, t, dim] -> masks [2*fft_bins, 2, t]."""
    x = np.ascontiguousarray(x, np.float32)
    nb, t, dim = x.shape
    offsets, bins = _bands(config)
    fft_bins = config["n_fft"] // 2 + 1
    hidden = [(np.ascontiguousarray(w, np.float32), np.ascontiguousarray(b, np.float32))
              for w, b in head["hidden"]]
    width = hidden[0][0].shape[1]
    hw = (ctypes.c_void_p * len(hidden))(*[w.ctypes.data for w, _ in hidden])
    hb = (ctypes.c_void_p * len(hidden))(*[b.ctypes.data for _, b in hidden])
    ow = np.ascontiguousarray(np.concatenate([w.ravel() for w, _ in head["out"]]), np.float32)
    ob = np.ascontiguousarray(np.concatenate([b for _, b in head["out"]]), np.float32)
    out = np.empty((2 * fft_bins, 2, t), np.float32)
    _check(_l().anc_mask_head(x.ctypes.data, t, nb, offsets.ctypes.data, bins.ctypes.data,
                              fft_bins, dim, width, len(hidden), ctypes.cast(hw, _p),
                              ctypes.cast(hb, _p), ow.ctypes.data, ob.ctypes.data, threads,
                              out.ctypes.data))
    return out


def model_forward(spectrum, config, weights, threads=1):
    """Roformer::forward (network.rs:303-400): packed spectrum [t, 4*fft_bins] ->
    masks [stems, 2*fft_bins, 2, t]. The time pass runs on groups = bands (sequence t), the
    frequency pass on groups = t (sequence bands) after the dense transpose of :336-338."""
    x = band_split(spectrum, config, weights, threads)
    for time_block, freq_block in weights["layers"]:
        y = transformer_forward(time_block, x, kernels=True, threads=threads)
        y = np.ascontiguousarray(y.transpose(1, 0, 2))
        y = transformer_forward(freq_block, y, kernels=True, threads=threads)
        x = np.ascontiguousarray(y.transpose(1, 0, 2))
    if weights.get("final_norm") is not None:
        g = np.asarray(weights["final_norm"], np.float32) * np.float32(np.sqrt(np.float32(x.shape[2])))
        x = unit_norm(x.reshape(-1, x.shape[2]), scale=g, precision="f32").reshape(x.shape)
    return np.stack([mask_head(x, config, head, threads) for head in weights["masks"]])


def pack_spectra(spectra):
    """runtime.rs:161-172: per-channel complex [t, bins] -> [t, 4*bins] (frame,
    bin*2 + channel, re/im)."""
    s = np.stack(spectra, axis=2)  # [t, bins, channel]
    return np.ascontiguousarray(np.stack([s.real, s.imag], axis=3).reshape(s.shape[0], -1),
                                dtype=np.float32)


def chunk_weight(samples: int, i: np.ndarray, first: bool, last: bool) -> np.ndarray:
    """ChunkPlan::weight (chunk.rs:27-36): linear fades of samples/10 at interior edges."""
    fade = max(samples // 10, 1)
    w = np.ones(i.shape, np.float32)
    if not first:
        m = i < fade
        w[m] = (i[m] + 1).astype(np.float32) / np.float32(fade)
    if not last:
        m = i >= samples - fade
        w[m] = (samples - i[m]).astype(np.float32) / np.float32(fade)
    return w


def chunk_starts(chunk_samples, overlap, n):
    """(starts, border) of the chunk loop for an n-sample clip: ChunkPlan::new and ::starts
    (crates/ancha-audio/src/chunk.rs:9-24) over the clip plus the reflected border of
    src/runtime.rs:103-111 (no border when n <= 2 * border)."""
    if not (chunk_samples > 0 and overlap > 0 and overlap <= chunk_samples):
        raise ValueError("invalid chunk or overlap divisor")
    step = chunk_samples // overlap
    border = chunk_samples - step
    border = border if n > 2 * border else 0
    return list(range(0, n + 2 * border, step)), border


def separate(audio, config, weights, threads=1, chunks=None):
    """The chunked separation loop of src/runtime.rs:103-238 on stereo audio [2, n]:
    reflect-bordered chunks of chunk_samples every chunk_samples/overlap samples, STFT per
    channel, model masks, complex mask multiply, iSTFT, fade-weighted overlap-add, border crop.
    Returns [stems, 2, n]. `chunks` limits the loop to the first chunks (timing samples)."""
    audio = np.asarray(audio, np.float32)
    n = audio.shape[1]
    cs, n_fft, hop = config["chunk_samples"], config["n_fft"], config["hop"]
    starts, border = chunk_starts(cs, config["overlap"], n)
    length = n + 2 * border
    if chunks is not None:
        starts = starts[:chunks]
    stems = len(weights["masks"])
    acc = OverlapAdd(stems * 2, length, cs)
    bins = n_fft // 2 + 1
    for start in starts:
        remaining = min(length - start, cs)
        i = np.arange(cs)
        local = np.where(i < remaining, i, _reflect(i, remaining))
        chunk = audio[:, _reflect(start + local - border, n)]
        if remaining <= cs // 2:
            chunk[:, remaining:] = 0.0
        spectra = [stft(chunk[c], n_fft, hop) for c in range(2)]
        masks = model_forward(pack_spectra(spectra), config, weights, threads)
        planes = []
        for s in range(stems):
            for c in range(2):
                m = masks[s, c::2][:bins]  # rows 2f + c: [bins, 2, t]
                mask = (m[:, 0, :] + 1j * m[:, 1, :]).T.astype(np.complex64)
                planes.append(istft(spectra[c] * mask, cs, n_fft, hop, config["zero_dc"]))
        acc.add(start, planes)
    # A timing sample (`chunks`) leaves later samples uncovered: divide where covered.
    out = acc.finish(strict=chunks is None).reshape(stems, 2, length)
    return out[..., border:border + n]


class OverlapAdd:
    """Accumulator (chunk.rs:39-89): fade-weighted sums of chunk planes and their weights."""

    def __init__(self, channels: int, length: int, samples: int):
        self.sums = np.zeros((channels, length), np.float32)
        self.weights = np.zeros(length, np.float32)
        self.samples = samples

    def add(self, start: int, planes) -> None:
        length = self.weights.size
        end = min(start + self.samples, length)
        w = chunk_weight(self.samples, np.arange(self.samples), start == 0,
                         start + self.samples >= length)[: end - start]
        self.weights[start:end] += w
        for c, plane in enumerate(planes):
            self.sums[c, start:end] += w * np.asarray(plane, np.float32)[: end - start]

    def finish(self, strict: bool = True) -> np.ndarray:
        covered = self.weights > 0
        if strict and not np.all(covered):
            raise ValueError("uncovered overlap-add sample")
        out = np.zeros_like(self.sums)
        out[:, covered] = self.sums[:, covered] / self.weights[covered]
        return out
