"""Attention plan and backend switches: ``AttentionPlan`` (crates/ancha-models/src/roformer.rs:64-145),
``BackendKind::attention_plan`` (src/backend.rs:49-67) and the run settings that
``runtime::separate`` derives from a plan (src/runtime.rs:62-81, :310-330).

The plan carries the reference's tiling of materialized attention scores (``query_tile``,
``group_tile``, ``score_budget``, ``host_threads``) and its kernel switches. On this library's
GPU path attention is single-pass (``fused_attention``) and the projections run through the
hand-written GEMM (``custom_gemm``): scores are never materialized, so the tiles only enter the
run report, as they do in the reference's fused runs. A plan that asks for the tiled score path
or the backend GEMM is rejected by ``require_gpu_kernels``: this library has no second GPU
implementation to route it to.
"""
from __future__ import annotations

import os
from dataclasses import dataclass, replace
from typing import Optional

SCORE_BUDGET = 512 << 20
BACKENDS = ("cpu", "ndarray", "wgpu", "cuda", "hip")


class PlanError(ValueError):
    pass


def _clamp(v: int, lo: int, hi: int) -> int:
    # Rust's usize::clamp panics on lo > hi; every call here has lo = 1 <= hi.
    return max(lo, min(v, hi))


@dataclass(frozen=True)
class AttentionPlan:
    """roformer.rs:64-84. ``None`` tiles pick the largest tile within ``score_budget``."""
    query_tile: Optional[int] = 128
    group_tile: Optional[int] = 4
    score_budget: int = SCORE_BUDGET
    batched_linear: bool = True
    host_threads: int = 1
    conv_gemm: bool = False
    fused_attention: bool = False
    custom_gemm: bool = False

    def validate(self) -> None:
        """roformer.rs:86-96."""
        if (self.query_tile == 0 or self.group_tile == 0 or self.score_budget <= 0
                or self.host_threads <= 0):
            raise PlanError("attention tiles, score budget and host threads must be positive")

    def tiles(self, groups: int, tokens: int, heads: int) -> tuple[int, int]:
        """Effective ``(group_tile, query_tile)`` for ``groups`` sequences of ``tokens``
        (roformer.rs:97-110): one score row is heads * tokens float32; queries stay whole when
        one group fits the budget."""
        row = heads * tokens * 4
        query = self.query_tile if self.query_tile is not None \
            else max(self.score_budget // row, 1)
        query = _clamp(query, 1, tokens)
        group = self.group_tile if self.group_tile is not None \
            else max(self.score_budget // (row * query), 1)
        group = _clamp(group, 1, groups)
        return group, query

    def score_bytes(self, groups: int, tokens: int, heads: int) -> int:
        """Bytes of one materialized score tile (roformer.rs:111-114)."""
        group, query = self.tiles(groups, tokens, heads)
        return group * heads * query * tokens * 4

    def per_worker(self, groups: int) -> tuple[int, "AttentionPlan"]:
        """Worker count over ``groups`` and each worker's plan; the workers split the score
        budget (roformer.rs:115-124)."""
        parts = _clamp(self.host_threads, 1, max(groups, 1))
        return parts, replace(self, score_budget=max(self.score_budget // parts, 1))

    def worker_tiles(self, groups: int, tokens: int, heads: int) -> tuple[int, int, int]:
        """Per-worker ``(group_tile, query_tile, score bytes)`` (roformer.rs:125-131)."""
        parts, plan = self.per_worker(groups)
        groups = -(-groups // parts)
        group, query = plan.tiles(groups, tokens, heads)
        return group, query, plan.score_bytes(groups, tokens, heads)


def backend_plan(kind: str) -> AttentionPlan:
    """``BackendKind::attention_plan`` (backend.rs:49-67): automatic tiles within 512 MiB of
    scores; all host threads on CPU backends, one on GPUs; on the GPU with hand-written kernels
    (the reference's ``cuda``, this library's ``hip``) folded projections, GEMM convolution,
    the fused attention kernel and the custom GEMM."""
    if kind not in BACKENDS:
        raise PlanError(f"unknown backend {kind!r}")
    gpu = kind in ("wgpu", "cuda", "hip")
    kernels = kind in ("cuda", "hip")
    return AttentionPlan(query_tile=None, group_tile=None, score_budget=SCORE_BUDGET,
                         batched_linear=not kernels,
                         host_threads=1 if gpu else (os.cpu_count() or 1),
                         conv_gemm=kernels, fused_attention=kernels, custom_gemm=kernels)


def require_gpu_kernels(plan: AttentionPlan) -> None:
    """Checks a plan for this library's GPU path: valid, and asking for the single-pass
    attention kernel and the hand-written GEMM, the only GPU kernels built here."""
    plan.validate()
    if not plan.fused_attention:
        raise PlanError("the tiled attention path is not built for the GPU; "
                        "use fused_attention=True")
    if not plan.custom_gemm:
        raise PlanError("the backend GEMM path is not built for the GPU; use custom_gemm=True")


def run_settings(plan: AttentionPlan, config: dict, max_score_mib: int = 512,
                 chunk_samples: Optional[int] = None, overlap: Optional[int] = None,
                 kernels_available: bool = True) -> dict:
    """The plan-derived fields of the run report (runtime.rs:42-81 and :310-330) for a model
    ``config`` (the fields of ModelConfig): tiles of both axis passes, the estimated score
    bytes (zero when attention is fused), the kernel labels and the ``--max-score-mib``
    check. ``kernels_available`` is ``fused::available`` on the run's device."""
    plan.validate()
    c = dict(config)
    profile = "custom-context" if chunk_samples is not None or overlap is not None \
        else "native-context"
    if chunk_samples is not None:
        c["chunk_samples"] = chunk_samples
    if overlap is not None:
        c["overlap"] = overlap
    frames = c["chunk_samples"] // c["hop"] + 1
    bands, heads = len(c["bands"]), c["heads"]
    fused = plan.fused_attention and c["head_dim"] == 64 and kernels_available
    tg, tq, time_bytes = plan.worker_tiles(bands, frames, heads)
    fg, fq, freq_bytes = plan.worker_tiles(frames, bands, heads)
    if fused:
        time_bytes = freq_bytes = 0
    concurrent = max(time_bytes * plan.per_worker(bands)[0],
                     freq_bytes * plan.per_worker(frames)[0])
    if concurrent > max_score_mib * (1 << 20):
        raise PlanError(f"concurrent attention scores need {concurrent / 1048576.0:.1f} MiB, "
                        "above --max-score-mib; reduce tiles or --host-threads")
    return {
        "profile": profile,
        "query_tile": tq, "group_tile": tg,
        "frequency_query_tile": fq, "frequency_group_tile": fg,
        "attention_tiling": "auto" if plan.query_tile is None or plan.group_tile is None
        else "manual",
        "host_threads": plan.host_threads,
        "conv_strategy": ("gemm" if plan.conv_gemm else "backend")
        if c["family"] == "hyperace-v2" else None,
        "attention_kernel": "fused" if fused else "tiled",
        "gemm_kernel": "custom" if plan.custom_gemm and kernels_available else "burn",
        "linear_layout": "batched" if plan.batched_linear else "flattened",
        "estimated_time_attention_score_bytes": time_bytes,
        "estimated_frequency_attention_score_bytes": freq_bytes,
    }
