"""bench.py's contract on the CPU: the one-GPU guard and the algorithmic work each metric is
priced with (the reference's attention FLOP formula, examples/fused_attention.rs:67, and the
per-layer / per-chunk totals derived from the reference's shapes)."""
import json
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr
    assert r.stdout == ""


def test_attention_flops():
    # 4 * G * H * T^2 * d at [120, 801, 8, 64]: 157.68 GFLOP.
    G, T, H, D = 120, 801, 8, 64
    assert 4.0 * G * H * T * T * D == pytest.approx(157.68e9, rel=1e-4)


def test_layer_pair_flops():
    """Time pass on [120, 801, 384] (QKV 113.98, attention 157.68, out 37.80, FF 226.78 GFLOP)
    plus band pass on [1602, 60, 384]: 926.6 GFLOP."""
    c = bench.LAYER
    time_pass = bench.layer_flops(c["batch"] * c["bands"], c["frames"], c["dim"], c["heads"],
                                  c["hidden"])
    band_pass = bench.layer_flops(c["batch"] * c["frames"], c["bands"], c["dim"], c["heads"],
                                  c["hidden"])
    assert time_pass == pytest.approx(536.23e9, rel=1e-3)
    assert time_pass + band_pass == pytest.approx(926.59e9, rel=1e-3)


def test_separation_flops():
    """Mel-Karaoke: 3.107 TFLOP of network work per 801-frame chunk; BS-RoFormer-large: the
    transformer alone is ~12 x 1.02 TFLOP per 1101-frame chunk."""
    from ancha_amd import separation as S

    mel = S.load_config("mel_karaoke")
    assert bench.mel_flops(mel) == pytest.approx(3.107e12, rel=2e-3)
    bs = S.load_config("bs_roformer_large")
    frames, nb = bs["chunk_samples"] // bs["hop"] + 1, len(bs["bands"])
    assert frames == 1101 and nb == 62
    hidden = bs["dim"] * bs["ff_mult"]
    pair = (bench.layer_flops(nb, frames, bs["dim"], bs["heads"], hidden)
            + bench.layer_flops(frames, nb, bs["dim"], bs["heads"], hidden))
    assert bs["depth"] * pair == pytest.approx(12 * 1.02e12, rel=0.03)
    assert bench.mel_flops(bs) > bs["depth"] * pair


def test_bundled_configs_are_the_benchmarked_shapes():
    from ancha_amd import package as P
    from ancha_amd import separation as S

    for name in ("mel_karaoke", "bs_roformer_large"):
        P.validate_config(S.load_config(name))
    with open(os.path.join(ROOT, "ancha_amd", "configs", "bs_roformer_large.json")) as f:
        bs = json.load(f)
    counts = [len(b) for b in bs["bands"]]
    # The reference's 62-band layout (config.rs:181-192).
    assert counts == [2] * 24 + [4] * 12 + [12] * 8 + [24] * 8 + [48] * 8 + [128, 129]
    assert (bs["dim"], bs["depth"], bs["heads"], bs["chunk_samples"]) == (512, 12, 8, 485100)
