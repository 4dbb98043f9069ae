"""GPU parity of the Mel-RoFormer model around the attention path: STFT / iSTFT, the network
forward (band split, axis loop, mask heads) and the chunked separation, against the oracle.
Bounds: the DSP is fp32 end to end (relative 1e-5 of the signal scale); the network runs its
GEMMs and attention on fp16 operands, so masks and stems are compared by SNR, with the 50 dB
end-to-end gate of the separated stems."""
import numpy as np
import pytest
import torch

import oracle.mel as M
from ancha_amd import separation as S
from ancha_amd import workload as W

from .test_mel_oracle import identity_model, tiny_config

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


def snr_db(ref, got):
    ref = np.asarray(ref, np.float64)
    err = np.asarray(got, np.float64) - ref
    return 10.0 * np.log10(np.sum(ref * ref) / max(np.sum(err * err), 1e-300))


def report(name, value):
    print(f"{name}: {value}", flush=True)


def packed_spectrum(chunk, hop):
    """Oracle STFT of both channels in the model's packed layout [frames, 4*1025]."""
    return M.pack_spectra([M.stft(chunk[c], 2048, hop) for c in range(2)])


def test_stft_matches_oracle(gpu):
    x = W.audio(5000, seed=41)
    got = S.stft(torch.from_numpy(x).to(gpu), 441).cpu().numpy()
    assert got.shape == (5000 // 441 + 1, 1025, 2, 2)
    for c in range(2):
        want = M.stft(x[c], 2048, 441)
        err = np.abs(got[:, :, c, 0] + 1j * got[:, :, c, 1] - want).max()
        report(f"stft channel {c} max|diff| / max", err / np.abs(want).max())
        assert err < 1e-5 * np.abs(want).max()


@pytest.mark.parametrize("n,hop", [(4103, 441), (88201, 512)])
def test_istft_round_trip_and_masks(gpu, n, hop):
    x = W.audio(n, seed=42)
    xs = torch.from_numpy(x).to(gpu)
    spec = S.stft(xs, hop)
    frames = spec.shape[0]
    ones = torch.zeros((2050, 2, frames), device=gpu)
    ones[:, 0, :] = 1.0
    y = S.istft(spec, ones, hop, n).cpu().numpy()
    err = np.abs(y - x).max()
    report(f"istft(stft) n={n} hop={hop} max|diff|", err)
    assert err < 1e-5
    # Random complex masks against the oracle's masked inverse.
    m = W.normal((2050, 2, frames), 43, 1.0)
    y = S.istft(spec, torch.from_numpy(m).to(gpu), hop, n, zero_dc=True).cpu().numpy()
    sp = spec.cpu().numpy()
    for c in range(2):
        spc = sp[:, :, c, 0] + 1j * sp[:, :, c, 1]
        mc = (m[c::2, 0, :] + 1j * m[c::2, 1, :]).T
        want = M.istft(spc * mc, n, 2048, hop, zero_dc=True)
        err = np.abs(y[c] - want).max()
        report(f"masked istft channel {c} max|diff|", err)
        assert err < 1e-5 * max(np.abs(want).max(), 1.0)


@pytest.mark.parametrize("depth", [1, 3])
def test_forward_matches_oracle_tiny(gpu, depth):
    """Two stems, three overlapping bands, 101 frames (time kernel), 3 bands (band kernel).
    Depth 3 covers the hand-over of each block's output norm to the next block's fp16 operand
    across layer pairs."""
    config = tiny_config(depth=depth)
    tensors = W.roformer_tensors(config, seed=31)
    model = S.Roformer(config, tensors, gpu)
    chunk = W.audio(config["chunk_samples"], seed=44)
    spec = packed_spectrum(chunk, config["hop"])
    got = model(torch.from_numpy(spec).to(gpu)).cpu().numpy()
    want = M.model_forward(spec, config, M.weights_from_tensors(config, tensors), threads=8)
    assert got.shape == want.shape == (2, 2050, 2, 101)
    db = snr_db(want, got)
    report(f"tiny forward depth {depth} masks SNR dB", db)
    assert db > 50.0


def test_separate_identity_model(gpu):
    """Unit masks: the GPU runtime returns its input (chunking, STFT, iSTFT, overlap-add)."""
    config = dict(tiny_config(stems=("vocals",)), zero_dc=False)
    tensors = W.roformer_tensors(config, seed=14)
    # identity_model's mask-head edits, written back as checkpoint tensors.
    ident = identity_model(config)
    for b, (w, bias) in enumerate(ident["masks"][0]["out"]):
        tensors[f"mask_estimators.0.to_freqs.{b}.0.4.weight"] = w
        tensors[f"mask_estimators.0.to_freqs.{b}.0.4.bias"] = bias
    for layer, (w, bias) in enumerate(ident["masks"][0]["hidden"]):
        for b in range(3):
            tensors[f"mask_estimators.0.to_freqs.{b}.0.{2 * layer}.weight"] = w[b]
    model = S.Roformer(config, tensors, gpu)
    audio = W.audio(100_000, seed=21)
    stems, residual = model.separate(torch.from_numpy(audio).to(gpu))
    err = np.abs(stems[0].cpu().numpy() - audio).max()
    report("identity separation max|diff|", err)
    assert err < 1e-4
    assert np.abs(residual.cpu().numpy()).max() < 1e-4


def test_separate_matches_oracle_tiny(gpu):
    config = tiny_config(stems=("vocals",))
    tensors = W.roformer_tensors(config, seed=33)
    model = S.Roformer(config, tensors, gpu)
    audio = W.audio(150_000, seed=45)
    stems, residual = model.separate(torch.from_numpy(audio).to(gpu))
    want = M.separate(audio, config, M.weights_from_tensors(config, tensors), threads=8)
    db = snr_db(want[0], stems[0].cpu().numpy())
    report("tiny separation stem SNR dB", db)
    assert db > 50.0
    np.testing.assert_allclose(residual.cpu().numpy(), audio - stems[0].cpu().numpy(), atol=1e-6)


def tiny_bs_config(depth=2):
    """BS-RoFormer at the kernel_package scale: three contiguous bands partitioning the bins, one
    stem, a final norm instead of per-block output norms, mask MLP counting every Linear in
    mask_depth (network.rs:138-157)."""
    config = tiny_config(stems=("vocals",), family="bs-roformer", depth=depth)
    config["bands"] = [list(range(0, 300)), list(range(300, 700)), list(range(700, 1025))]
    return config


def test_forward_matches_oracle_tiny_bs(gpu):
    config = tiny_bs_config()
    tensors = W.roformer_tensors(config, seed=36)
    model = S.Roformer(config, tensors, gpu)
    spec = packed_spectrum(W.audio(config["chunk_samples"], seed=48), config["hop"])
    got = model(torch.from_numpy(spec).to(gpu)).cpu().numpy()
    want = M.model_forward(spec, config, M.weights_from_tensors(config, tensors), threads=8)
    assert got.shape == want.shape == (1, 2050, 2, 101)
    db = snr_db(want, got)
    report("tiny BS forward masks SNR dB", db)
    assert db > 50.0


def test_separate_matches_oracle_tiny_bs(gpu):
    config = tiny_bs_config(depth=1)
    tensors = W.roformer_tensors(config, seed=38)
    model = S.Roformer(config, tensors, gpu)
    audio = W.audio(120_000, seed=49)
    stems, _ = model.separate(torch.from_numpy(audio).to(gpu))
    want = M.separate(audio, config, M.weights_from_tensors(config, tensors), threads=8)
    db = snr_db(want[0], stems[0].cpu().numpy())
    report("tiny BS separation stem SNR dB", db)
    assert db > 50.0


def test_bs_roformer_large_shapes_one_layer_pair(gpu):
    """The bundled BS-RoFormer-large shapes (62 bands, dim 512, 8 heads, mask MLP x4) at depth 1,
    on a 101-frame chunk."""
    config = dict(S.load_config("bs_roformer_large"), depth=1, chunk_samples=44100)
    tensors = W.roformer_tensors(config, seed=37, device=gpu)
    model = S.Roformer(config, tensors, gpu)
    spec = packed_spectrum(W.audio(config["chunk_samples"], seed=47), config["hop"])
    got = model(torch.from_numpy(spec).to(gpu)).cpu().numpy()
    want = M.model_forward(spec, config, M.weights_from_tensors(config, tensors), threads=16)
    db = snr_db(want, got)
    report("bs-roformer-large depth-1 forward masks SNR dB", db)
    assert db > 50.0


def test_separate_mel_karaoke_one_layer_pair(gpu):
    """The bundled Mel-Karaoke shapes (60 bands, dim 384, 8 heads, 801-frame chunks) at depth 1
    on one chunk."""
    config = dict(S.load_config("mel_karaoke"), depth=1)
    tensors = W.roformer_tensors(config, seed=35, device=gpu)
    model = S.Roformer(config, tensors, gpu)
    audio = W.audio(80_000, seed=46)
    stems, _ = model.separate(torch.from_numpy(audio).to(gpu))
    want = M.separate(audio, config, M.weights_from_tensors(config, tensors), threads=16)
    db = snr_db(want[0], stems[0].cpu().numpy())
    report("mel-karaoke depth-1 separation stem SNR dB", db)
    assert db > 50.0
