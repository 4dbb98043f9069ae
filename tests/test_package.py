"""Model packages (manifest.json + model.safetensors): manifest / config validation, checked
tensor loading, and a GPU load-and-run of a kernel-sized package against the oracle."""
import json
import os

import numpy as np
import pytest

from ancha_amd import package as P
from ancha_amd import workload as W


def leap_bands():
    """ModelConfig::leap_xe's band widths (config.rs:123-136)."""
    counts = [2] * 24 + [4] * 36 + [12] * 16 + [24] * 8 + [48] * 4 + [128, 129]
    bands, o = [], 0
    for n in counts:
        bands.append(list(range(o, o + n)))
        o += n
    return bands


def tiny_package_config(family="mel-band-roformer", kernel=False):
    """tests/support/mod.rs:12-55 (tiny_package / kernel_package)."""
    c = {"family": family, "dim": 4, "depth": 1, "heads": 1, "head_dim": 4, "ff_mult": 1,
         "mask_depth": 2, "mask_expansion": 1, "sample_rate": 44100, "n_fft": 2048, "hop": 512,
         "chunk_samples": 4096, "overlap": 2, "zero_dc": True, "stems": ["vocals"],
         "bands": [list(range(0, 300)), list(range(300, 700)), list(range(700, 1000)),
                   list(range(1000, 1025))]}
    if family == "mel-band-roformer":
        c["stems"] = ["vocals", "instrumental"]
        c["bands"] = [list(range(0, 400)), list(range(300, 900)), list(range(625, 1025))]
    if kernel:
        c.update(dim=128, heads=2, head_dim=64, ff_mult=4)
    return c


def synthetic_values(name, shape):
    """The deterministic tensor formula of tests/support/mod.rs:62-75."""
    n = int(np.prod(shape))
    i = np.arange(n)
    if name.endswith("gamma"):
        v = 0.75 + (i % 3) * 0.25
    elif name.endswith("freqs"):
        v = np.where(i == 0, 1.0, 0.01)
    else:
        v = ((i % 17) - 8) * 0.001
    return v.astype(np.float32).reshape(shape)


def write_package(directory, config, tensors=None):
    from safetensors.numpy import save_file

    os.makedirs(directory, exist_ok=True)
    if tensors is None:
        tensors = {n: synthetic_values(n, s) for n, s in W.roformer_tensor_shapes(config).items()}
    path = os.path.join(directory, "model.safetensors")
    save_file(tensors, path)
    manifest = {"schema_version": 1, "model_id": "synthetic-ci-fixture",
                "weights_sha256": P.sha256_file(path), "checkpoint_sha256": "0" * 64,
                "source_url": "original synthetic tensors", "forward_revision": "synthetic",
                "weight_license": "MIT", "config": config}
    with open(os.path.join(directory, "manifest.json"), "w") as f:
        json.dump(manifest, f)
    return tensors


@pytest.mark.parametrize("family", ["mel-band-roformer", "bs-roformer"])
def test_tiny_package_round_trip(tmp_path, family):
    config = tiny_package_config(family)
    tensors = write_package(str(tmp_path), config)
    m = P.read_manifest(str(tmp_path))
    got = P.load_tensors(str(tmp_path), m)
    assert set(got) == set(tensors)
    for name, a in tensors.items():
        np.testing.assert_array_equal(got[name], a)
    # BS counts all Linears in mask_depth, Mel only hidden ones (network.rs:138-144).
    last = 4 if family == "mel-band-roformer" else 2
    assert f"mask_estimators.0.to_freqs.0.0.{last}.weight" in got
    assert ("final_norm.gamma" in got) == (family == "bs-roformer")


def test_package_rejections(tmp_path):
    config = tiny_package_config()
    tensors = write_package(str(tmp_path), config)
    m = P.read_manifest(str(tmp_path))
    # Tampered weights: checksum mismatch.
    with open(os.path.join(str(tmp_path), "model.safetensors"), "r+b") as f:
        f.seek(-4, os.SEEK_END)
        f.write(b"\x00\x00\x80\x7f")
    with pytest.raises(P.PackageError, match="checksum mismatch"):
        P.load_tensors(str(tmp_path), m)
    # Extra tensor, wrong shape, wrong dtype, non-finite value, missing tensor.
    cases = [
        (dict(tensors, extra=np.zeros(3, np.float32)), "unrecognized checkpoint tensors"),
        (dict(tensors, **{"layers.0.0.layers.0.0.to_gates.bias": np.zeros(2, np.float32)}),
         "expected"),
        (dict(tensors, **{"band_split.to_features.0.1.bias":
                          tensors["band_split.to_features.0.1.bias"].astype(np.float64)}),
         "requires F32"),
        (dict(tensors, **{"layers.0.1.norm.gamma": np.full(4, np.inf, np.float32)}),
         "non-finite"),
        ({k: v for k, v in tensors.items() if k != "layers.0.0.layers.0.1.net.4.bias"},
         "missing tensor"),
    ]
    for i, (bad, msg) in enumerate(cases):
        d = str(tmp_path / f"case{i}")
        write_package(d, config, bad)
        with pytest.raises(P.PackageError, match=msg):
            P.load_tensors(d, P.read_manifest(d))


@pytest.mark.parametrize("edit,msg", [
    (lambda c: c.update(n_fft=1024), "FFT 2048"),
    (lambda c: c.update(head_dim=3), "attention dimensions"),
    (lambda c: c.update(stems=["vocals", "vocals"]), "duplicate stems"),
    (lambda c: c.update(stems=["lead_vocals", "vocals"]), "lead vocals"),
    (lambda c: c["bands"].__setitem__(0, list(range(1, 400))), "uncovered"),
    (lambda c: c["bands"].__setitem__(1, [301, 300]), "strictly ordered"),
    (lambda c: c.update(extra=1), "config fields"),
])
def test_config_validation(edit, msg):
    """ModelConfig::validate (config.rs:36-121) rejections."""
    c = tiny_package_config()
    c["bands"] = [list(b) for b in c["bands"]]
    edit(c)
    with pytest.raises(P.PackageError, match=msg):
        P.validate_config(c)


def test_bundled_configs_validate():
    from ancha_amd import separation as S

    P.validate_config(S.load_config("mel_karaoke"))
    c = tiny_package_config("bs-roformer")
    c["bands"] = leap_bands()
    P.validate_config(c)
    c["bands"][3] = c["bands"][3][:-1]
    with pytest.raises(P.PackageError):
        P.validate_config(c)


@pytest.mark.gpu
def test_kernel_package_loads_and_matches_oracle(tmp_path, gpu):
    """kernel_package (tests/support/mod.rs:17-25) written, loaded and run on the GPU."""
    import torch

    import oracle.mel as M

    config = tiny_package_config(kernel=True)
    tensors = write_package(str(tmp_path), config)
    model, manifest = P.load_model(str(tmp_path), torch.device("cuda:0"))
    settings = model.settings()
    assert (settings["attention_kernel"], settings["gemm_kernel"]) == ("fused", "custom")
    chunk = W.audio(config["chunk_samples"], seed=51)
    spec = M.pack_spectra([M.stft(chunk[c], 2048, config["hop"]) for c in range(2)])
    got = model(torch.from_numpy(spec).cuda()).cpu().numpy()
    want = M.model_forward(spec, config, M.weights_from_tensors(config, tensors), threads=8)
    err = np.sum((got - want) ** 2.0)
    db = 10 * np.log10(np.sum(want.astype(np.float64) ** 2) / max(err, 1e-300))
    print(f"kernel_package masks SNR dB {db:.1f}", flush=True)
    assert db > 50.0
