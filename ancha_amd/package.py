"""Model packages: `manifest.json` + `model.safetensors` (crates/ancha-models/src/config.rs
Manifest, crates/ancha-models/src/weights.rs), read into the tensor dict that
``separation.Roformer`` takes.

Checks follow the reference: schema 1 metadata (``Manifest::validate_metadata``,
config.rs:203-216), the model config (``ModelConfig::validate``, config.rs:36-121), F32 finite
tensors of the expected shapes (``Weights::take``, weights.rs:73-102), no unrecognized tensors
(``Weights::finish``, :128-141) and the weights' SHA-256 (``verified``, :26-40). The safetensors
file is read with the safetensors library's numpy loader (no pickle, no code execution).
"""
from __future__ import annotations

import hashlib
import json
import os
import re

import numpy as np

from .workload import roformer_tensor_shapes

STEMS = ("vocals", "instrumental", "lead_vocals")
FAMILIES = ("bs-roformer", "mel-band-roformer", "hyperace-v2")
CONFIG_FIELDS = ("family", "dim", "depth", "heads", "head_dim", "ff_mult", "mask_depth",
                 "mask_expansion", "sample_rate", "n_fft", "hop", "chunk_samples", "overlap",
                 "zero_dc", "stems", "bands")


class PackageError(ValueError):
    pass


def _ensure(cond, msg: str) -> None:
    if not cond:
        raise PackageError(msg)


def validate_config(c: dict) -> None:
    """ModelConfig::validate (config.rs:36-121); raises PackageError with the reference's
    messages."""
    _ensure(set(c) == set(CONFIG_FIELDS), "unknown or missing config fields")
    _ensure(c["family"] in FAMILIES, "unknown model family")
    _ensure(0 < c["dim"] <= 4096 and 0 < c["depth"] <= 64, "invalid model dimensions")
    _ensure(0 < c["heads"] <= 64 and c["head_dim"] > 0 and c["head_dim"] % 2 == 0
            and c["head_dim"] <= 256, "invalid attention dimensions")
    _ensure(0 < c["ff_mult"] <= 16 and 0 < c["mask_depth"] <= 8
            and 0 < c["mask_expansion"] <= 16, "invalid MLP dimensions")
    _ensure(c["sample_rate"] == 44100 and c["n_fft"] == 2048 and 1 <= c["hop"] <= 1024,
            "schema 1 requires 44100 Hz, FFT 2048 and hop <= 1024")
    _ensure(c["n_fft"] // 2 < c["chunk_samples"] <= 44100 * 60 and 0 < c["overlap"] <= 16,
            "invalid chunk settings")
    stems = c["stems"]
    _ensure(0 < len(stems) <= 2 and all(s in STEMS for s in stems), "invalid stem labels")
    _ensure(len(stems) == 1 or stems[0] != stems[1], "duplicate stems")
    _ensure("lead_vocals" not in stems
            or (c["family"] == "mel-band-roformer" and len(stems) == 1),
            "lead vocals require a single-head Mel karaoke model")
    bands = c["bands"]
    _ensure(2 <= len(bands) <= 256, "invalid band count")
    bins = c["n_fft"] // 2 + 1
    coverage = np.zeros(bins, np.int64)
    for band in bands:
        _ensure(len(band) > 0 and all(a < b for a, b in zip(band, band[1:])),
                "bands must be nonempty and strictly ordered")
        for f in band:
            _ensure(0 <= f < bins, "band index out of range")
            coverage[f] += 1
    _ensure(np.all(coverage > 0), "bands leave uncovered FFT bins")
    if c["family"] != "mel-band-roformer":
        _ensure(np.all(coverage == 1), "BS bands must partition the frequency axis")
        _ensure([f for b in bands for f in b] == list(range(bins)),
                "BS bands must be contiguous and in frequency order")
    if c["family"] == "hyperace-v2":
        _ensure(c["dim"] == 256 and len(bands) == 62 and len(stems) == 1,
                "HyperACE v2 requires dim=256, 62 bands and one stem")


def read_manifest(package: str) -> dict:
    """read_manifest (weights.rs:42-49) + Manifest::validate."""
    with open(os.path.join(package, "manifest.json"), "rb") as f:
        m = json.loads(f.read())
    _ensure(m.get("schema_version") == 1, "unsupported model package schema")
    _ensure(bool(m.get("model_id")), "model ID is empty")
    for key in ("weights_sha256", "checkpoint_sha256"):
        _ensure(isinstance(m.get(key), str) and re.fullmatch(r"[0-9a-fA-F]{64}", m[key]),
                "invalid SHA256")
    validate_config(m["config"])
    return m


def sha256_file(path: str) -> str:
    h = hashlib.sha256()
    with open(path, "rb") as f:
        for block in iter(lambda: f.read(1 << 20), b""):
            h.update(block)
    return h.hexdigest()


def load_tensors(package: str, manifest: dict) -> dict:
    """The checked checkpoint of a package: every tensor the model reads, F32, finite, of its
    shape; no others; the file's SHA-256 equal to the manifest's."""
    from safetensors.numpy import load_file

    path = os.path.join(package, "model.safetensors")
    _ensure(sha256_file(path) == manifest["weights_sha256"], "model checksum mismatch")
    raw = load_file(path)
    config = manifest["config"]
    _ensure(config["family"] != "hyperace-v2",
            "HyperACE segmentation heads are not part of this build")
    shapes = roformer_tensor_shapes(config)
    out = {}
    for name, shape in shapes.items():
        _ensure(name in raw, f"missing tensor {name}")
        a = raw[name]
        _ensure(tuple(a.shape) == tuple(shape),
                f"{name}: expected {list(shape)}, got {list(a.shape)}")
        _ensure(a.dtype == np.float32, f"{name}: schema 1 requires F32 weights, got {a.dtype}")
        _ensure(bool(np.all(np.isfinite(a))), f"{name}: non-finite weight")
        out[name] = a
    unused = [n for n in raw if n not in shapes][:8]
    _ensure(not unused, f"unrecognized checkpoint tensors: {unused}")
    return out


def load_model(package: str, device=None, plan=None):
    """Roformer::load (network.rs:79-88): manifest, checked tensors, the GPU model run with
    ``plan`` (an ``AttentionPlan``; default the GPU backend's)."""
    from .separation import Roformer

    manifest = read_manifest(package)
    tensors = load_tensors(package, manifest)
    return Roformer(manifest["config"], tensors, device, plan), manifest
