"""The allocation-free iSTFT entry point (static device scratch) against ancha_hip_istft with a
caller workspace, through the C ABI: identical results on two calls in a row, the second with
fewer frames (the scratch keeps the first call's contents), and a clear rejection of a frame
count beyond the scratch."""
import ctypes

import numpy as np
import pytest
import torch

from ancha_amd import _native
from ancha_amd import separation as S
from ancha_amd import workload as W

pytestmark = pytest.mark.gpu


def istft_both(lib, spec, masks, hop, length, zero_dc, gpu):
    frames = spec.shape[0]
    stream = torch.cuda.current_stream().cuda_stream
    ws = torch.empty(int(lib.ancha_hip_istft_workspace(frames)), dtype=torch.uint8, device=gpu)
    want = torch.empty((2, length), device=gpu)
    rc = lib.ancha_hip_istft(spec.data_ptr(), masks.data_ptr(), frames, hop, length, zero_dc,
                             ws.data_ptr(), ws.numel(), want.data_ptr(), stream)
    assert rc == _native.OK, _native.last_error()
    got = torch.full((2, length), float("nan"), device=gpu)
    rc = lib.ancha_hip_istft_noalloc(spec.data_ptr(), masks.data_ptr(), frames, hop, length,
                                     zero_dc, got.data_ptr(), stream)
    assert rc == _native.OK, _native.last_error()
    torch.cuda.synchronize()
    return got, want


def test_noalloc_istft_matches_workspace_istft(gpu):
    lib = _native.lib()
    for n, hop, zero_dc, seed in ((352_800, 441, 1, 71), (50_000, 512, 0, 72)):
        audio = torch.from_numpy(W.audio(n, seed=seed)).to(gpu)
        spec = S.stft(audio, hop)
        frames = spec.shape[0]
        masks = torch.from_numpy(W.normal((2050, 2, frames), seed + 10, 1.0)).to(gpu)
        got, want = istft_both(lib, spec, masks, hop, n, zero_dc, gpu)
        print(f"noalloc istft frames={frames}: max|diff| "
              f"{(got - want).abs().max().item():.3e}", flush=True)
        assert torch.isfinite(got).all()
        assert torch.equal(got, want)


def test_noalloc_istft_rejects_too_many_frames(gpu):
    lib = _native.lib()
    frames, hop = 1537, 441
    length = (frames - 1) * hop
    spec = torch.zeros((frames, 1025, 2, 2), device=gpu)
    masks = torch.zeros((2050, 2, frames), device=gpu)
    out = torch.zeros((2, length), device=gpu)
    rc = lib.ancha_hip_istft_noalloc(spec.data_ptr(), masks.data_ptr(), frames, hop, length, 0,
                                     out.data_ptr(), torch.cuda.current_stream().cuda_stream)
    assert rc == _native.UNSUPPORTED
    assert "1536" in _native.last_error()
    assert lib.ancha_hip_check() == 0
