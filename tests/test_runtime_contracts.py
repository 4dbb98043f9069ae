"""Runtime contracts of the separation path that hold without a GPU: the chunk plan
(crates/ancha-audio/src/chunk.rs:9-24, src/runtime.rs:103-111) in the oracle and in the C ABI,
and the sticky device-failure state (src/device.rs:11-41) driven from the host.

The reference pins the chunk count with one known answer (tests/runtime_contracts.rs:52: a
5003-sample clip at chunk 4096, overlap 2 makes 5 chunks, reflected borders and a non-aligned
tail) and the stickiness with a host-driven failure (tests/device_guard.rs:3-23): once a device
failure is recorded, every later check reports it. Both run here on the CPU: the chunk plan is
host arithmetic, and the sticky state is checked before any argument or device access, so the
entry points below never reach a kernel launch.
"""
import os
import subprocess
import sys
import textwrap

import numpy as np
import pytest

from ancha_amd import separation
from oracle import mel as M

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_chunk_count_known_answer():
    """runtime_contracts.rs:52: 5003 samples, chunk 4096, overlap 2 -> 5 chunks."""
    starts, border = M.chunk_starts(4096, 2, 5003)
    assert len(starts) == 5 and border == 2048
    assert starts == [0, 2048, 4096, 6144, 8192]
    assert separation.chunk_plan(4096, 2, 5003) == (5, 2048)


@pytest.mark.parametrize("config,samples,chunks,border", [
    ("mel_karaoke", 30 * 44100, 21, 264600),          # the 30 s benchmark clip
    ("mel_karaoke", 88200, 1, 0),                     # one chunk, no border
    ("mel_karaoke", 2 * 264600, 6, 0),                # not longer than two borders: no border
    ("mel_karaoke", 2 * 264600 + 1, 13, 264600),
    ("bs_roformer_large", 5 * 60 * 44100, 57, 242550),  # the 5 min benchmark clip
])
def test_chunk_plan_of_the_bundled_models(config, samples, chunks, border):
    c = separation.load_config(config)
    starts, b = M.chunk_starts(c["chunk_samples"], c["overlap"], samples)
    assert (len(starts), b) == (chunks, border)
    assert separation.chunk_plan(c["chunk_samples"], c["overlap"], samples) == (chunks, border)


def test_chunk_plan_agrees_with_the_oracle_on_random_shapes():
    rng = np.random.default_rng(5)
    for _ in range(400):
        cs = int(rng.integers(1, 5000))
        overlap = int(rng.integers(1, min(cs, 9) + 1))
        n = int(rng.integers(0, 4 * cs + 3))
        starts, border = M.chunk_starts(cs, overlap, n)
        assert separation.chunk_plan(cs, overlap, n) == (len(starts), border), (cs, overlap, n)


@pytest.mark.parametrize("cs,overlap", [(0, 1), (4096, 0), (4, 5)])
def test_chunk_plan_rejects_invalid_divisors(cs, overlap):
    with pytest.raises(ValueError, match="invalid chunk or overlap divisor"):
        M.chunk_starts(cs, overlap, 100)
    with pytest.raises(ValueError, match="invalid chunk or overlap divisor"):
        separation.chunk_plan(cs, overlap, 100)


# Runs in a child process (the sticky state lasts for the process). Every entry point gets
# arguments it would reject by itself (null tensors, null handles), so a broken sticky check
# would return ANCHA_HIP_INVALID, never launch.
_CHILD = textwrap.dedent("""
    import ctypes, sys
    sys.path.insert(0, sys.argv[1])
    from ancha_amd import _native
    lib = _native.lib()
    code = -int(sys.argv[2])
    N = None
    calls = {
        "ancha_hip_attention": lambda: lib.ancha_hip_attention(N, N, N, 1, 4, 1, 64, 64, 64, N, N, N),
        "ancha_hip_gated_attention": lambda: lib.ancha_hip_gated_attention(N, 1, 4, 256, 1, N, N, N),
        "ancha_hip_linear": lambda: lib.ancha_hip_linear(N, 4, 8, 8, N, 128, N, 0, N, 0, 0, N, N, N),
        "ancha_hip_norm_linear": lambda: lib.ancha_hip_norm_linear(N, 4, 8, 8, N, 128, N, 0, N, 0, 0,
                                                                  N, N, N),
        "ancha_hip_unit_norm": lambda: lib.ancha_hip_unit_norm(N, 4, 8, 8, N, N, N),
        "ancha_hip_swap_axes": lambda: lib.ancha_hip_swap_axes(N, 1, 2, 3, 4, N, N),
        "ancha_hip_block_create": lambda: lib.ancha_hip_block_create(384, 8, 1536, *([N] * 11), N),
        "ancha_hip_block_forward": lambda: lib.ancha_hip_block_forward(N, N, 1, 4, N, N, 1024, N, N),
        "ancha_hip_axis_pair_forward": lambda: lib.ancha_hip_axis_pair_forward(N, N, N, 1, 2, 3, N, N,
                                                                              N, 1024, N, N),
        "ancha_hip_roformer_create": lambda: lib.ancha_hip_roformer_create(N, N, N, N),
        "ancha_hip_roformer_forward": lambda: lib.ancha_hip_roformer_forward(N, N, 10, N, 1024, N, N,
                                                                            N),
        "ancha_hip_separate": lambda: lib.ancha_hip_separate(N, N, 10, N, 1024, N, N, N, N),
        "ancha_hip_stft": lambda: lib.ancha_hip_stft(N, 5000, 441, N, N),
        "ancha_hip_istft": lambda: lib.ancha_hip_istft(N, N, 3, 441, 1000, 0, N, 1 << 20, N, N),
        "ancha_hip_istft_noalloc": lambda: lib.ancha_hip_istft_noalloc(N, N, 3, 441, 1000, 0, N, N),
    }
    missing = sorted(n for n in _native.SIGNATURES if n.startswith("ancha_hip_") and n not in calls
                     and not n.endswith(("_workspace", "_destroy", "_supported", "_available",
                                         "_check", "_last_error", "_chunk_plan")))
    assert not missing, missing
    for name, call in calls.items():
        rc = call()
        msg = _native.last_error()
        assert rc == code, (name, rc, msg)
        assert "sticky device failure" in msg and "injected failure" in msg, (name, msg)
    # The check reports the first failure on every call; host-only queries keep working.
    assert lib.ancha_hip_check() == code and lib.ancha_hip_check() == code
    assert lib.ancha_hip_linear_supported(8, 128) == 1
    print("sticky", len(calls))
""")


def test_injected_failure_is_sticky_for_every_entry_point():
    """A HIP failure recorded once (here injected at library load, as the reference's guard test
    records a panic from the host) makes every compute entry point return that same negative
    code, and the last-error text names the first failure."""
    env = dict(os.environ, ANCHA_HIP_INJECT_FAILURE="2")  # hipErrorOutOfMemory
    r = subprocess.run([sys.executable, "-c", _CHILD, ROOT, "2"], env=env, capture_output=True,
                       text=True, timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "sticky 15" in r.stdout


def test_no_failure_without_injection():
    env = {k: v for k, v in os.environ.items() if k != "ANCHA_HIP_INJECT_FAILURE"}
    child = ("import sys; sys.path.insert(0, sys.argv[1]); from ancha_amd import _native; "
             "print(_native.lib().ancha_hip_check())")
    r = subprocess.run([sys.executable, "-c", child, ROOT], env=env, capture_output=True,
                       text=True, timeout=300)
    assert r.returncode == 0 and r.stdout.strip() == "0", r.stdout + r.stderr
