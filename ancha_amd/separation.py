"""Host mirror of the Mel/BS-RoFormer network (crates/ancha-models/src/network.rs) and of the
separation runtime (src/runtime.rs:103-238, crates/ancha-audio/src/{dsp,chunk}.rs) on the
gfx950 C ABI. All arithmetic runs in libancha_hip.so; torch provides device memory and the
stream.

Weights are the reference checkpoint's tensors by name (the names of network.rs:96-177 and
roformer.rs:205-252, 381-409), served to ``ancha_hip_roformer_create`` through a callback.
"""
from __future__ import annotations

import ctypes
import json
import os
from typing import Optional

import numpy as np
import torch

from . import _native
from ._tensors import require
from .plan import AttentionPlan, backend_plan, require_gpu_kernels, run_settings

# Raised by a forward or separation whose CancelFlag was set (C ABI code 3).
Cancelled = _native.Cancelled

N_FFT = 2048
BINS = N_FFT // 2 + 1
CONFIGS = os.path.join(os.path.dirname(os.path.abspath(__file__)), "configs")


def load_config(name: str = "mel_karaoke") -> dict:
    """A bundled model config (the fields of ModelConfig, config.rs:14-32)."""
    with open(os.path.join(CONFIGS, name + ".json")) as f:
        return json.load(f)


class _Config(ctypes.Structure):
    _fields_ = [("mel", ctypes.c_int)] + [
        (n, ctypes.c_size_t) for n in ("dim", "depth", "heads", "head_dim", "ff_mult",
                                       "mask_depth", "mask_expansion", "n_fft", "hop",
                                       "chunk_samples", "overlap")] + [
        ("zero_dc", ctypes.c_int), ("stems", ctypes.c_size_t), ("bands", ctypes.c_size_t),
        ("band_offsets", ctypes.c_void_p), ("band_bins", ctypes.c_void_p)]


_TensorFn = ctypes.CFUNCTYPE(ctypes.c_void_p, ctypes.c_void_p, ctypes.c_char_p, ctypes.c_size_t)


def _stream(device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


class CancelFlag:
    """The reference's ``cancelled: &AtomicBool`` (runtime.rs:118, network.rs:334,367): an int
    the C ABI reads between chunk pairs, layer pairs and mask heads. ``set()`` may be called
    from another thread while a forward or separation runs."""

    def __init__(self):
        self._flag = ctypes.c_int(0)

    def set(self) -> None:
        self._flag.value = 1

    def is_set(self) -> bool:
        return self._flag.value != 0

    def pointer(self):
        return ctypes.byref(self._flag)


def _flag(cancelled: Optional[CancelFlag]):
    return None if cancelled is None else cancelled.pointer()


def check_spectrum(spectrum: torch.Tensor, device) -> None:
    """The model input: float32 [frames, 4*1025] on ``device``."""
    if spectrum.dim() != 2 or spectrum.shape[1] != 4 * BINS:
        raise ValueError("spectrum must be [frames, 4100]")
    require(spectrum, "spectrum", device)


def check_audio(audio: torch.Tensor, device) -> None:
    """Stereo audio: float32 [2, samples] on ``device``."""
    if audio.dim() != 2 or audio.shape[0] != 2:
        raise ValueError("audio must be [2, samples]")
    require(audio, "audio", device)


class Roformer:
    """``Roformer::load`` + ``forward`` (network.rs:79-400) and the chunked ``separate`` of
    runtime.rs on one device. ``tensors`` maps checkpoint names to float32 arrays; ``plan``
    (default: the GPU backend's, backend.rs:52-67) must select the fused attention and custom
    GEMM kernels."""

    def __init__(self, config: dict, tensors: dict, device: Optional[torch.device] = None,
                 plan: Optional[AttentionPlan] = None):
        self.plan = backend_plan("hip") if plan is None else plan
        require_gpu_kernels(self.plan)
        self.config = dict(config)
        self.device = torch.device(device or "cuda")
        bands = config["bands"]
        offsets = np.zeros(len(bands) + 1, np.uintp)
        offsets[1:] = np.cumsum([len(b) for b in bands])
        bins = np.ascontiguousarray(np.concatenate([np.asarray(b) for b in bands]), np.uintp)
        self.stems = len(config["stems"])
        c = _Config(mel=int(config["family"] == "mel-band-roformer"), dim=config["dim"],
                    depth=config["depth"], heads=config["heads"], head_dim=config["head_dim"],
                    ff_mult=config["ff_mult"], mask_depth=config["mask_depth"],
                    mask_expansion=config["mask_expansion"], n_fft=config["n_fft"],
                    hop=config["hop"], chunk_samples=config["chunk_samples"],
                    overlap=config["overlap"], zero_dc=int(config["zero_dc"]),
                    stems=self.stems, bands=len(bands), band_offsets=offsets.ctypes.data,
                    band_bins=bins.ctypes.data)
        keep = {}

        def get(_ctx, name, numel):
            a = tensors.get(name.decode())
            if a is None:
                return None
            a = np.ascontiguousarray(a, dtype=np.float32)
            if a.size != numel:
                return None
            keep[name] = a
            return a.ctypes.data

        fn = _TensorFn(get)
        handle = ctypes.c_void_p()
        with torch.cuda.device(self.device):
            rc = _native.lib().ancha_hip_roformer_create(ctypes.byref(c), fn, None,
                                                         ctypes.byref(handle))
        keep.clear()
        if rc == _native.INVALID:
            raise ValueError("invalid model config or missing / mis-shaped tensor")
        if not _native.check(rc):
            raise ValueError("model shapes are outside what the kernels cover")
        self._handle = handle
        self._ws: Optional[torch.Tensor] = None

    def settings(self, max_score_mib: int = 512) -> dict:
        """The plan-derived run-report fields of this model (runtime.rs:62-81, :310-330)."""
        return run_settings(self.plan, self.config, max_score_mib)

    def _workspace(self, need: int) -> torch.Tensor:
        if self._ws is None or self._ws.numel() < need:
            self._ws = torch.empty(need, dtype=torch.uint8, device=self.device)
        return self._ws

    def forward(self, spectrum: torch.Tensor,
                cancelled: Optional[CancelFlag] = None) -> torch.Tensor:
        """spectrum [frames, 4*1025] float32 (frame, bin*2 + channel, re/im) ->
        masks [stems, 2*1025, 2, frames]. Raises ``Cancelled`` when ``cancelled`` is set."""
        check_spectrum(spectrum, self.device)
        frames = spectrum.shape[0]
        spectrum = spectrum.contiguous()
        lib = _native.lib()
        ws = self._workspace(int(lib.ancha_hip_roformer_workspace(self._handle, frames)))
        masks = torch.empty((self.stems, 2 * BINS, 2, frames), device=self.device)
        _native.check(lib.ancha_hip_roformer_forward(self._handle, spectrum.data_ptr(), frames,
                                                     ws.data_ptr(), ws.numel(), masks.data_ptr(),
                                                     _flag(cancelled), _stream(self.device)))
        return masks

    __call__ = forward

    def separate(self, audio: torch.Tensor, cancelled: Optional[CancelFlag] = None):
        """Stereo audio [2, samples] float32 on the device -> (stems [stems, 2, samples],
        residual [2, samples] for one-stem models else None). Raises ``ValueError`` with the
        reference runtime's message for non-finite input, model or chunk output, and
        ``Cancelled`` when ``cancelled`` is set."""
        check_audio(audio, self.device)
        audio = audio.contiguous()
        n = audio.shape[1]
        lib = _native.lib()
        ws = self._workspace(int(lib.ancha_hip_separate_workspace(self._handle, n)))
        stems = torch.empty((self.stems, 2, n), device=self.device)
        residual = torch.empty((2, n), device=self.device) if self.stems == 1 else None
        _native.check(lib.ancha_hip_separate(self._handle, audio.data_ptr(), n, ws.data_ptr(),
                                             ws.numel(), stems.data_ptr(),
                                             None if residual is None else residual.data_ptr(),
                                             _flag(cancelled), _stream(self.device)))
        return stems, residual

    def close(self) -> None:
        if getattr(self, "_handle", None):
            _native.lib().ancha_hip_roformer_destroy(self._handle)
            self._handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def chunk_plan(chunk_samples: int, overlap: int, samples: int) -> tuple[int, int]:
    """(chunks, border) of the separation of a `samples`-sample clip: ChunkPlan::new / starts
    (crates/ancha-audio/src/chunk.rs:9-24) with the border rule of src/runtime.rs:103-111.
    Raises ValueError for an invalid chunk or overlap divisor."""
    chunks, border = ctypes.c_size_t(0), ctypes.c_size_t(0)
    _native.check(_native.lib().ancha_hip_chunk_plan(chunk_samples, overlap, samples,
                                                     ctypes.byref(chunks), ctypes.byref(border)))
    return chunks.value, border.value


def stft(signal: torch.Tensor, hop: int) -> torch.Tensor:
    """Stft::forward of both channels of signal [2, samples] -> [frames, 1025, 2, 2]
    (frame, bin, channel, re/im)."""
    check_audio(signal, signal.device)
    signal = signal.contiguous()
    n = signal.shape[1]
    out = torch.empty((n // hop + 1, BINS, 2, 2), device=signal.device)
    _native.check(_native.lib().ancha_hip_stft(signal.data_ptr(), n, hop, out.data_ptr(),
                                               _stream(signal.device)))
    return out


def istft(spectrum: torch.Tensor, masks: torch.Tensor, hop: int, length: int,
          zero_dc: bool = False) -> torch.Tensor:
    """Stft::inverse of spectrum * masks (masks [2*1025, 2, frames]) -> [2, length]."""
    if spectrum.dim() != 4:
        raise ValueError("spectrum must be [frames, 1025, 2, 2]")
    frames = spectrum.shape[0]
    require(spectrum, "spectrum", spectrum.device, (frames, BINS, 2, 2))
    require(masks, "masks", spectrum.device, (2 * BINS, 2, frames))
    spectrum, masks = spectrum.contiguous(), masks.contiguous()
    lib = _native.lib()
    ws = torch.empty(int(lib.ancha_hip_istft_workspace(frames)), dtype=torch.uint8,
                     device=spectrum.device)
    out = torch.empty((2, length), device=spectrum.device)
    _native.check(lib.ancha_hip_istft(spectrum.data_ptr(), masks.data_ptr(), frames, hop, length,
                                      int(zero_dc), ws.data_ptr(), ws.numel(), out.data_ptr(),
                                      _stream(spectrum.device)))
    return out
