"""The oracle's STFT / band split / mask head / separation runtime against the reference's own
known answers (crates/ancha-audio/tests/audio_contracts.rs) and closed forms the maths fixes.
CPU only."""
import numpy as np
import pytest

import oracle.mel as M
from ancha_amd import workload as W


def signal(n):
    """audio_contracts.rs:10-14."""
    i = np.arange(n, dtype=np.float32)
    return ((np.sin(i * np.float32(0.071)) + np.float32(0.2) * np.cos(i * np.float32(0.31)))
            * np.float32(0.4)).astype(np.float32)


def tiny_config(stems=("vocals", "instrumental"), family="mel-band-roformer", depth=1):
    """The reference's kernel_package shape (tests/support/mod.rs:18-55): dim 128, 2 heads of
    64, FF x4, mask depth 2 (x1), three overlapping Mel bands; a 44100-sample chunk at hop 441
    (101 frames) so the time axis exceeds one 64-key tile."""
    return {"family": family, "dim": 128, "depth": depth, "heads": 2, "head_dim": 64,
            "ff_mult": 4, "mask_depth": 2, "mask_expansion": 1, "sample_rate": 44100,
            "n_fft": 2048, "hop": 441, "chunk_samples": 44100, "overlap": 2, "zero_dc": True,
            "stems": list(stems),
            "bands": [list(range(0, 400)), list(range(300, 900)), list(range(625, 1025))]}


def test_reflect_index_known_answers():
    """audio_contracts.rs:62-67."""
    assert [M.reflect_index(i, 4) for i in range(-4, 8)] == [2, 3, 2, 1, 0, 1, 2, 3, 2, 1, 0, 1]
    assert M.reflect_index(-5, 1) == 0
    assert list(M._reflect(np.arange(-4, 8), 4)) == [2, 3, 2, 1, 0, 1, 2, 3, 2, 1, 0, 1]


def test_stft_analytic_dc():
    """audio_contracts.rs:47-60: a constant 1 under the periodic Hann window."""
    spec = M.stft(np.ones(4096, np.float32), 2048, 512)
    assert spec.shape == (9, 1025)
    assert abs(spec[0, 0].real - 1024.0) < 1e-3
    assert abs(spec[0, 1].real + 512.0) < 1e-3
    assert abs(spec[0, 2]) < 1e-3


@pytest.mark.parametrize("hop", [441, 512])
@pytest.mark.parametrize("n", [1025, 2048, 4103, 88201])
def test_stft_inverse_round_trip(hop, n):
    """audio_contracts.rs:16-45 (max error < 2e-6)."""
    x = signal(n)
    x[0], x[-1] = 0.81, -0.72
    spec = M.stft(x, 2048, hop)
    assert spec.shape[0] == n // hop + 1
    y = M.istft(spec, n, 2048, hop)
    assert np.abs(x - y).max() < 2e-6


def test_stft_matches_direct_dft():
    """One frame against the DFT sum written out (brute force, fp64)."""
    rng = np.random.default_rng(3)
    x = rng.standard_normal(3000).astype(np.float32)
    spec = M.stft(x, 2048, 441)
    t = 3
    idx = np.array([M.reflect_index(t * 441 + i - 1024, x.size) for i in range(2048)])
    w = (0.5 - 0.5 * np.cos(2 * np.pi * np.arange(2048) / 2048)).astype(np.float64)
    frame = x[idx].astype(np.float64) * w
    k = np.arange(1025)[:, None]
    dft = (frame[None, :] * np.exp(-2j * np.pi * k * np.arange(2048)[None, :] / 2048)).sum(1)
    assert np.abs(spec[t] - dft).max() < 1e-3 * np.abs(dft).max()


@pytest.mark.parametrize("n", [1, 31, 64, 65, 128, 303])
@pytest.mark.parametrize("overlap", [1, 2, 4])
def test_overlap_add_identity(n, overlap):
    """audio_contracts.rs:69-100: chunks of 64 every 64/overlap samples, weights divide out."""
    x = signal(n)
    acc = M.OverlapAdd(2, n, 64)
    for start in range(0, n, 64 // overlap):
        chunk = np.array([x[start + i] if start + i < n else 0.0 for i in range(64)], np.float32)
        acc.add(start, [chunk, -chunk])
    out = acc.finish()
    assert np.abs(out[0] - x).max() < 1e-6 and np.abs(out[1] + x).max() < 1e-6


def test_band_split_single_column_closed_form():
    """One nonzero feature per band: unit_norm makes it +-1, so x = sign * sqrt(w) * gamma_c *
    W[:, c] + bias exactly (up to fp32 rounding)."""
    config = tiny_config()
    tensors = W.roformer_tensors(config, seed=11)
    weights = M.weights_from_tensors(config, tensors)
    t = 5
    spec = np.zeros((t, 4 * 1025), np.float32)
    picks = []
    # Bands overlap: bins 17, 500 and 1000 each belong to one band only.
    for b, (bins, f) in enumerate(zip(config["bands"], (17, 500, 1000))):
        q, k = bins.index(f), (b + 1) % 4
        picks.append((4 * q + k, 4 * f + k))
    for b, (c, col) in enumerate(picks):
        spec[:, col] = -2.5 if b % 2 else 3.0
    gam = [(0.5 + b) * np.ones(4 * len(bins), np.float32) for b, bins in enumerate(config["bands"])]
    for b in range(3):
        weights["band_split"][b]["gamma"] = gam[b]
    x = M.band_split(spec, config, weights)
    for b, (c, col) in enumerate(picks):
        bs = weights["band_split"][b]
        width = bs["weight"].shape[1]
        sign = -1.0 if b % 2 else 1.0
        want = sign * np.sqrt(np.float32(width)) * gam[b][c] * bs["weight"][:, c] + bs["bias"]
        np.testing.assert_allclose(x[b], np.broadcast_to(want, x[b].shape), rtol=1e-5,
                                   atol=1e-6)


def test_band_split_scale_invariance():
    """unit_norm makes the features independent of the spectrum's scale."""
    config = tiny_config()
    weights = M.weights_from_tensors(config, W.roformer_tensors(config, seed=12))
    spec = W.normal((7, 4 * 1025), 5, 1.0)
    a = M.band_split(spec, config, weights)
    b = M.band_split(spec * np.float32(37.0), config, weights)
    np.testing.assert_allclose(a, b, rtol=1e-5, atol=1e-5)


def test_mask_head_bias_only_closed_form():
    """Zero weights: every hidden layer is tanh(b), the output value * sigmoid(gate) comes
    from the last biases alone, and overlapping bands are averaged."""
    config = tiny_config(stems=("vocals",))
    weights = M.weights_from_tensors(config, W.roformer_tensors(config, seed=13))
    head = weights["masks"][0]
    head["hidden"] = [(np.zeros_like(w), b) for w, b in head["hidden"]]
    head["out"] = [(np.zeros_like(w), b) for w, b in head["out"]]
    t = 4
    x = W.normal((3, t, 128), 9, 1.0)
    masks = M.mask_head(x, config, head)
    # Expected per band: value_bias * sigmoid(gate_bias) on the band's 4 columns per bin.
    want = np.zeros((2 * 1025, 2), np.float64)
    count = np.zeros(2 * 1025)
    for b, bins in enumerate(config["bands"]):
        bias = head["out"][b][1].astype(np.float64)
        w = 4 * len(bins)
        glu = bias[:w] / (1.0 + np.exp(-bias[w:]))
        for j, f in enumerate(bins):
            for ch in range(2):
                want[2 * f + ch] += glu[4 * j + 2 * ch: 4 * j + 2 * ch + 2]
                count[2 * f + ch] += 1
    want /= count[:, None]
    np.testing.assert_allclose(masks, np.broadcast_to(want[..., None], masks.shape), rtol=1e-5,
                               atol=1e-7)
    assert set(np.unique(count)) == {1.0, 2.0}


def identity_model(config, seed=14):
    """A model whose masks are exactly 1 + 0i: zero mask-head weights, value bias 1 on the
    real columns, gate bias 40 (sigmoid = 1 in fp32)."""
    tensors = W.roformer_tensors(config, seed=seed)
    weights = M.weights_from_tensors(config, tensors)
    for head in weights["masks"]:
        head["hidden"] = [(np.zeros_like(w), b) for w, b in head["hidden"]]
        out = []
        for w, b in head["out"]:
            width = b.size // 2
            bias = np.zeros_like(b)
            bias[0:width:2] = 1.0
            bias[width:] = 40.0
            out.append((np.zeros_like(w), bias))
        head["out"] = out
    return weights


def test_separate_identity_masks_reconstruct_input():
    """Unit masks through the whole runtime: chunking, reflect borders, STFT, iSTFT and the
    fade-weighted overlap-add return the input (zero_dc off)."""
    config = dict(tiny_config(stems=("vocals",)), zero_dc=False)
    weights = identity_model(config)
    audio = W.audio(100_000, seed=21)
    out = M.separate(audio, config, weights, threads=4)
    assert out.shape == (1, 2, 100_000)
    assert np.abs(out[0] - audio).max() < 1e-4
