"""GPU parity of the Mel-RoFormer model around the attention path: STFT / iSTFT, the network
forward (band split, axis loop, mask heads) and the chunked separation, against the oracle.
Bounds: the DSP is fp32 end to end (relative 1e-5 of the signal scale); the network runs its
GEMMs and attention on fp16 operands, so masks and stems are compared by SNR, with the 50 dB
end-to-end gate of the separated stems."""
import os

import numpy as np
import pytest
import torch

import oracle.mel as M
from ancha_amd import _native
from ancha_amd import separation as S
from ancha_amd import workload as W
from tests.golden import cases as C

from .test_mel_oracle import identity_model, tiny_config

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")

pytestmark = pytest.mark.gpu


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


def fixture(name):
    return np.load(os.path.join(GOLDEN, name), allow_pickle=False)


@pytest.mark.parametrize("name", C.NETWORKS)
def test_forward_matches_network_golden(gpu, name):
    """Tiny Mel / BS networks with non-zero weights, non-unit gammas and per-layer rotary
    frequencies against the committed torch float64 restatement (tests/golden/network.npz)."""
    config, tensors, spectrum = C.network_case(name)
    f = fixture("network.npz")
    np.testing.assert_allclose(C.checksum(spectrum, *(tensors[k] for k in sorted(tensors))),
                               f[f"checksum_{name}"], rtol=1e-12)
    model = S.Roformer(config, tensors, gpu)
    got = model(torch.from_numpy(spectrum).to(gpu)).cpu().numpy()
    db = snr_db(f[name], got[:, C.NETWORK_ROWS][..., C.NETWORK_FRAMES])
    report(f"network {name} vs golden SNR dB", db)
    assert db > 50.0
    m = C.moments(got)
    want = f[f"moments_{name}"]
    assert abs(m[1] - want[1]) < 1e-3 * want[1]


@pytest.mark.parametrize("name", sorted(C.PRODUCTION))
def test_forward_production_shapes_match_oracle(gpu, name):
    """Mel-Karaoke at depth 6 on one 801-frame chunk and BS-RoFormer-large at depth 2 on one
    1101-frame chunk against the oracle's masks (tests/golden/production_networks.npz, a
    row/frame lattice of them plus whole-output moments)."""
    config, tensors, spectrum = C.production_case(name, device=gpu)
    f = fixture("production_networks.npz")
    np.testing.assert_allclose(C.checksum(spectrum, *(tensors[k] for k in sorted(tensors))),
                               f[f"checksum_{name}"], rtol=1e-12)
    model = S.Roformer(config, tensors, gpu)
    got = model(torch.from_numpy(spectrum).to(gpu)).cpu().numpy()
    rows, frames = C.production_index(spectrum.shape[0])
    db = snr_db(f[name], got[:, rows][..., frames])
    report(f"{name} forward vs oracle SNR dB", db)
    assert db > 50.0
    m, want = C.moments(got), f[f"moments_{name}"]
    report(f"{name} sum of squares rel. diff", abs(m[1] - want[1]) / want[1])
    assert abs(m[1] - want[1]) < 1e-3 * want[1]
    model.close()


@pytest.mark.parametrize("name", sorted(C.SEPARATIONS))
def test_production_separation_matches_oracle(gpu, name):
    """The separated stems at production depth against the oracle's separation loop
    (runtime.rs:103-238 restated in oracle.mel.separate, tests/golden/production_separations.npz):
    Mel-Karaoke at depth 6 on a one-chunk clip, BS-RoFormer-large at depth 2 on a two-chunk clip
    batched through one forward. The end-to-end gate is 50 dB (scripts/verify_parity.py:93 of the
    reference), measured on a sample lattice plus the whole output's sum of squares."""
    config, tensors, audio = C.separation_case(name, device=gpu)
    f = fixture("production_separations.npz")
    np.testing.assert_allclose(C.checksum(audio, *(tensors[k] for k in sorted(tensors))),
                               f[f"checksum_{name}"], rtol=1e-12)
    model = S.Roformer(config, tensors, gpu)
    stems, residual = model.separate(torch.from_numpy(audio).to(gpu))
    got = stems.cpu().numpy()
    db = snr_db(f[name], got[..., C.separation_index(audio.shape[1])])
    report(f"{name} stems vs oracle SNR dB", db)
    assert db > 50.0
    m, want = C.moments(got), f[f"moments_{name}"]
    report(f"{name} sum of squares rel. diff", abs(m[1] - want[1]) / want[1])
    assert abs(m[1] - want[1]) < 1e-3 * want[1]
    if residual is not None:
        np.testing.assert_allclose(residual.cpu().numpy(), audio - got[0], atol=1e-6)
    model.close()


@pytest.mark.parametrize("name", sorted(C.DEUX))
def test_forward_deux_shape_matches_oracle(gpu, name):
    """The reference's deux model shape (dim 256, 8 heads, 2 stems, Mel-Karaoke bands, 1301
    frames) at depth 1 against the oracle's masks (tests/golden/deux_network.npz): the dim-256
    fused QKV and tail, the 1301-frame time pass (three query blocks per sequence), the
    dim-256 band split and the x4 mask heads."""
    config, tensors, spectrum = C.deux_case(name, device=gpu)
    f = fixture("deux_network.npz")
    np.testing.assert_allclose(C.checksum(spectrum, *(tensors[k] for k in sorted(tensors))),
                               f[f"checksum_{name}"], rtol=1e-12)
    model = S.Roformer(config, tensors, gpu)
    got = model(torch.from_numpy(spectrum).to(gpu)).cpu().numpy()
    assert got.shape == (2, 2050, 2, 1301)
    rows, frames = C.production_index(spectrum.shape[0])
    db = snr_db(f[name], got[:, rows][..., frames])
    report(f"{name} forward vs oracle SNR dB", db)
    assert db > 50.0
    m, want = C.moments(got), f[f"moments_{name}"]
    assert abs(m[1] - want[1]) < 1e-3 * want[1]
    model.close()


def composed_separation(model, audio, config):
    """The chunk loop of runtime.rs:103-238 written out on the host from the library's single
    pieces (GPU STFT, one-chunk forward, masked iSTFT) and the oracle's overlap-add: the
    reference against which the fused ancha_hip_separate (two chunks per forward, GPU
    overlap-add) is checked."""
    n = audio.shape[1]
    cs, hop = config["chunk_samples"], config["hop"]
    step = cs // config["overlap"]
    border = cs - step if n > 2 * (cs - step) else 0
    length = n + 2 * border
    stems = len(config["stems"])
    acc = M.OverlapAdd(stems * 2, length, cs)
    for start in range(0, length, step):
        remaining = min(length - start, cs)
        i = np.arange(cs)
        local = np.where(i < remaining, i, M._reflect(i, remaining))
        chunk = audio[:, M._reflect(start + local - border, n)]
        if remaining <= cs // 2:
            chunk[:, remaining:] = 0.0
        spec = S.stft(torch.from_numpy(np.ascontiguousarray(chunk)).to(model.device), hop)
        masks = model(spec.reshape(spec.shape[0], -1))
        planes = []
        for s in range(stems):
            y = S.istft(spec, masks[s], hop, cs, config["zero_dc"]).cpu().numpy()
            planes += [y[0], y[1]]
        acc.add(start, planes)
    return acc.finish().reshape(stems, 2, length)[..., border:border + n]


def check_separation(model, config, audio, gpu, label):
    """Properties of a full-size separation plus equality with the composed chunk loop."""
    x = torch.from_numpy(audio).to(gpu)
    stems, residual = model.separate(x)
    again, _ = model.separate(x)
    torch.cuda.synchronize()
    assert torch.isfinite(stems).all()
    assert torch.equal(stems, again), "separation must be deterministic"
    got = stems.cpu().numpy()
    assert np.abs(got).max() > 1e-4, "stems must not be silent"
    if residual is not None:
        np.testing.assert_allclose(residual.cpu().numpy(), audio - got[0], atol=1e-6)
    want = composed_separation(model, audio, config)
    db = snr_db(want, got)
    report(f"{label}: fused separation vs composed chunk loop SNR dB", db)
    assert db > 60.0


def test_mel_karaoke_depth6_30s_separation(gpu):
    """BASELINE's Mel-RoFormer workload: Mel-Karaoke at depth 6 on a 30 s clip (21 overlapping
    801-frame chunks, run two at a time through the model)."""
    config = S.load_config("mel_karaoke")
    tensors = W.roformer_tensors(config, seed=55, device=gpu)
    model = S.Roformer(config, tensors, gpu)
    check_separation(model, config, W.audio(30 * 44100, seed=56), gpu, "mel-karaoke 30 s")
    model.close()


def test_bs_large_two_chunks_batched(gpu):
    """BS-RoFormer-large at depth 2: a clip of exactly two 1101-frame chunks goes through the
    model as one batch of two."""
    config = dict(S.load_config("bs_roformer_large"), depth=2)
    tensors = W.roformer_tensors(config, seed=57, device=gpu)
    model = S.Roformer(config, tensors, gpu)
    check_separation(model, config, W.audio(config["chunk_samples"], seed=58), gpu,
                     "bs-large depth 2, two chunks")
    model.close()


def test_bs_large_depth12_separation(gpu):
    """BS-RoFormer-large as configured (depth 12) on a 60 s clip."""
    config = S.load_config("bs_roformer_large")
    tensors = W.roformer_tensors(config, seed=59, device=gpu)
    model = S.Roformer(config, tensors, gpu)
    check_separation(model, config, W.audio(60 * 44100, seed=60), gpu, "bs-large depth 12, 60 s")
    model.close()


def test_forward_other_frame_count(gpu):
    """A frame count other than the chunk's: rotary and tile tables built in the workspace."""
    config = tiny_config(depth=2)
    tensors = W.roformer_tensors(config, seed=61)
    model = S.Roformer(config, tensors, gpu)
    weights = M.weights_from_tensors(config, tensors)
    for samples in (66_150, 20_000):
        spec = packed_spectrum(W.audio(samples, seed=62), config["hop"])
        got = model(torch.from_numpy(spec).to(gpu)).cpu().numpy()
        want = M.model_forward(spec, config, weights, threads=8)
        db = snr_db(want, got)
        report(f"tiny forward at {spec.shape[0]} frames masks SNR dB", db)
        assert db > 50.0


def test_separate_reports_non_finite_input(gpu):
    config = tiny_config(stems=("vocals",))
    model = S.Roformer(config, W.roformer_tensors(config, seed=63), gpu)
    audio = W.audio(60_000, seed=64)
    audio[1, 12_345] = np.nan
    with pytest.raises(ValueError, match="non-finite STFT input"):
        model.separate(torch.from_numpy(audio).to(gpu))
    audio[1, 12_345] = 0.0
    stems, _ = model.separate(torch.from_numpy(audio).to(gpu))
    assert torch.isfinite(stems).all()
    assert _native.lib().ancha_hip_check() == 0


def test_separate_reports_non_finite_model_output(gpu):
    config = tiny_config(stems=("vocals",))
    tensors = W.roformer_tensors(config, seed=65)
    tensors["mask_estimators.0.to_freqs.1.0.4.bias"][7] = np.inf
    model = S.Roformer(config, tensors, gpu)
    with pytest.raises(ValueError, match="non-finite model output"):
        model.separate(torch.from_numpy(W.audio(60_000, seed=66)).to(gpu))


def test_separate_reports_non_finite_istft_output(gpu):
    """Finite masks that overflow the masked spectrum: Stft::inverse's "non-finite iSTFT output"
    (dsp.rs:132-133), reported before the overlap-add (chunk.rs:57-60)."""
    config = tiny_config(stems=("vocals",))
    tensors = W.roformer_tensors(config, seed=65)
    # A value column of band 1's GLU: masks of ~1e38 stay finite, mask * spectrum does not.
    tensors["mask_estimators.0.to_freqs.1.0.4.bias"][7] = np.float32(3e38)
    model = S.Roformer(config, tensors, gpu)
    spec = torch.from_numpy(packed_spectrum(W.audio(44_100, seed=66), config["hop"])).to(gpu)
    assert torch.isfinite(model(spec)).all()
    with pytest.raises(ValueError, match="non-finite iSTFT output"):
        model.separate(torch.from_numpy(W.audio(60_000, seed=66)).to(gpu))
    assert _native.lib().ancha_hip_check() == 0


def test_cancel_from_another_thread_during_separation(gpu):
    """The CancelFlag set by another thread while ancha_hip_separate runs: the call returns
    "task cancelled" at its next check (between chunk pairs, layer pairs and mask heads), after
    the work it enqueued has finished; the model stays usable and an uncancelled run of the
    same clip is unchanged."""
    import threading

    config = tiny_config(stems=("vocals",), depth=2)
    model = S.Roformer(config, W.roformer_tensors(config, seed=71), gpu)
    audio = torch.from_numpy(W.audio(40 * 44_100, seed=72)).to(gpu)
    reference, _ = model.separate(audio)
    torch.cuda.synchronize()
    cancelled = 0
    for delay in (0.0, 0.001, 0.004):
        flag = S.CancelFlag()
        timer = threading.Timer(delay, flag.set)
        timer.start()
        try:
            stems, _ = model.separate(audio, cancelled=flag)
            # The loop finished before it saw the flag: the result is the whole separation.
            assert torch.equal(stems, reference)
        except _native.Cancelled as e:
            assert "task cancelled" in str(e)
            cancelled += 1
        timer.join()
        torch.cuda.synchronize()
    report("separations cancelled mid-run", cancelled)
    assert cancelled >= 1
    assert _native.lib().ancha_hip_check() == 0
    stems, _ = model.separate(audio)
    assert torch.equal(stems, reference)
    model.close()


def test_cancelled_separation_and_forward(gpu):
    config = tiny_config(stems=("vocals",))
    model = S.Roformer(config, W.roformer_tensors(config, seed=67), gpu)
    flag = S.CancelFlag()
    audio = torch.from_numpy(W.audio(60_000, seed=68)).to(gpu)
    model.separate(audio, cancelled=flag)
    flag.set()
    with pytest.raises(_native.Cancelled, match="task cancelled"):
        model.separate(audio, cancelled=flag)
    spec = torch.from_numpy(packed_spectrum(W.audio(44_100, seed=69), config["hop"])).to(gpu)
    with pytest.raises(_native.Cancelled):
        model(spec, cancelled=flag)
    torch.cuda.synchronize()
    assert _native.lib().ancha_hip_check() == 0


def test_wrappers_reject_host_and_misshaped_tensors(gpu):
    config = tiny_config(stems=("vocals",))
    model = S.Roformer(config, W.roformer_tensors(config, seed=70), gpu)
    with pytest.raises(ValueError):
        model.separate(torch.zeros((2, 50_000)))                       # host memory
    with pytest.raises(ValueError):
        model.separate(torch.zeros((2, 50_000), dtype=torch.float64, device=gpu))
    with pytest.raises(ValueError):
        model(torch.zeros((101, 4100), device=gpu, dtype=torch.float16))
    spec = S.stft(torch.zeros((2, 5000), device=gpu), 441)
    with pytest.raises(ValueError):
        S.istft(spec, torch.zeros((2050, 2, spec.shape[0] - 1), device=gpu), 441, 4000)
    with pytest.raises(ValueError):
        S.istft(spec, torch.zeros((2050, 2, spec.shape[0])), 441, 4000)
