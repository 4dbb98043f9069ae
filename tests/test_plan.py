"""AttentionPlan and the backend switches (crates/ancha-models/src/roformer.rs:64-145,
src/backend.rs:49-67, src/runtime.rs:62-81): the tiles the reference's own run reports recorded,
the budget invariants of automatic tiling, validation and the fused-path run settings."""
import json
import os

import numpy as np
import pytest

from ancha_amd import separation as S
from ancha_amd.plan import (AttentionPlan, PlanError, backend_plan, require_gpu_kernels,
                            run_settings)

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "plan_vectors.json")


def golden_cases():
    with open(GOLDEN) as f:
        return json.load(f)["cases"]


@pytest.mark.parametrize("case", golden_cases(), ids=lambda c: f"{c['source']}:{c['pass']}")
def test_tiles_match_reference_reports(case):
    """Tiles (and, where reported, score bytes) of docs/reports/*.json; the CPU rows of
    cuda-benchmark.json ran 24 host threads, so they also pin per_worker's budget split."""
    plan = AttentionPlan(**case["plan"])
    group, query, score = plan.worker_tiles(case["groups"], case["tokens"], case["heads"])
    want = case["want"]
    assert (group, query) == (want["group_tile"], want["query_tile"])
    if "score_bytes" in want:
        assert score == want["score_bytes"]
    if "linear_layout" in want:
        kind = case["backend"]
        assert backend_plan(kind).batched_linear == (want["linear_layout"] == "batched")
        if kind != "cpu":
            assert backend_plan(kind).host_threads == case["plan"]["host_threads"] == 1


def test_automatic_tiles_are_the_largest_within_budget():
    """With no explicit tiles one tile holds at most score_budget bytes (when one query row
    fits), and growing either tile by one would exceed it unless that tile is already whole."""
    rng = np.random.default_rng(7)
    for _ in range(3000):
        groups, tokens, heads = (int(v) for v in rng.integers(1, 300, 3))
        budget = int(rng.integers(1, 1 << 24))
        plan = AttentionPlan(query_tile=None, group_tile=None, score_budget=budget)
        group, query = plan.tiles(groups, tokens, heads)
        assert 1 <= group <= groups and 1 <= query <= tokens
        row = heads * tokens * 4
        size = lambda g, q: g * heads * q * tokens * 4
        assert plan.score_bytes(groups, tokens, heads) == size(group, query)
        if row <= budget:
            assert size(group, query) <= budget
            assert query == tokens or size(1, query + 1) > budget
            assert group == groups or size(group + 1, query) > budget
        else:
            assert (group, query) == (1, 1)


def test_explicit_tiles_clamp_to_the_problem():
    plan = AttentionPlan(query_tile=128, group_tile=4)
    assert plan.tiles(60, 801, 8) == (4, 128)
    assert plan.tiles(2, 60, 8) == (2, 60)
    assert AttentionPlan(query_tile=7, group_tile=1).tiles(3, 63, 2) == (1, 7)


def test_workers_split_the_budget():
    plan = AttentionPlan(query_tile=None, group_tile=None, host_threads=24)
    parts, worker = plan.per_worker(60)
    assert parts == 24 and worker.score_budget == (512 << 20) // 24
    assert plan.per_worker(5)[0] == 5
    assert plan.per_worker(0)[0] == 1
    # Concurrent workers stay within the whole budget.
    for groups in (1, 7, 60, 301, 1876):
        parts, worker = plan.per_worker(groups)
        g, q, score = plan.worker_tiles(groups, 801, 8)
        assert parts * score <= plan.score_budget


@pytest.mark.parametrize("field", ["query_tile", "group_tile", "score_budget", "host_threads"])
def test_validate_rejects_zero(field):
    with pytest.raises(PlanError, match="must be positive"):
        AttentionPlan(**{field: 0}).validate()
    AttentionPlan(query_tile=None, group_tile=None).validate()


def test_backend_defaults():
    """backend.rs:52-67 and the Default of roformer.rs:133-145."""
    d = AttentionPlan()
    assert (d.query_tile, d.group_tile, d.score_budget, d.batched_linear, d.host_threads) == \
        (128, 4, 512 << 20, True, 1)
    assert not (d.conv_gemm or d.fused_attention or d.custom_gemm)
    for kind in ("cuda", "hip"):
        p = backend_plan(kind)
        assert (p.query_tile, p.group_tile, p.batched_linear, p.host_threads) == \
            (None, None, False, 1)
        assert p.conv_gemm and p.fused_attention and p.custom_gemm
    w = backend_plan("wgpu")
    assert w.batched_linear and w.host_threads == 1 and not w.fused_attention
    assert backend_plan("cpu").host_threads == (os.cpu_count() or 1)
    with pytest.raises(PlanError):
        backend_plan("metal")


def test_fused_run_settings():
    """tests/cuda_contracts.rs:449-454: a fused run reports the fused kernel, the custom GEMM
    and no materialized scores."""
    config = S.load_config("mel_karaoke")
    s = run_settings(backend_plan("hip"), config, max_score_mib=16)
    assert s["attention_kernel"] == "fused" and s["gemm_kernel"] == "custom"
    assert s["estimated_time_attention_score_bytes"] == 0
    assert s["estimated_frequency_attention_score_bytes"] == 0
    assert s["linear_layout"] == "flattened" and s["attention_tiling"] == "auto"
    assert s["profile"] == "native-context" and s["conv_strategy"] is None
    frames = config["chunk_samples"] // config["hop"] + 1
    assert (s["query_tile"], s["frequency_query_tile"]) == (frames, len(config["bands"]))


def test_tiled_run_settings_and_score_limit():
    """The tiled path's estimates and the --max-score-mib check (runtime.rs:75-81)."""
    config = S.load_config("mel_karaoke")
    plan = AttentionPlan(query_tile=128, group_tile=4)
    s = run_settings(plan, config, kernels_available=False)
    frames = config["chunk_samples"] // config["hop"] + 1
    assert s["attention_kernel"] == "tiled" and s["gemm_kernel"] == "burn"
    assert s["estimated_time_attention_score_bytes"] == 4 * 8 * 128 * frames * 4
    assert s["attention_tiling"] == "manual"
    # A fused plan on a device without the kernels falls back to the tiled estimate.
    s = run_settings(backend_plan("hip"), config, kernels_available=False)
    assert s["attention_kernel"] == "tiled" and s["estimated_time_attention_score_bytes"] > 0
    with pytest.raises(PlanError, match="max-score-mib"):
        run_settings(backend_plan("hip"), config, max_score_mib=1, kernels_available=False)
    s = run_settings(plan, config, chunk_samples=132300, kernels_available=False)
    assert s["profile"] == "custom-context" and s["query_tile"] == 128


def test_gpu_model_requires_the_kernel_plan():
    """A plan asking for the tiled attention or the backend GEMM is rejected before any GPU
    work: this library has no second GPU implementation to run it."""
    require_gpu_kernels(backend_plan("hip"))
    for plan in (AttentionPlan(), backend_plan("wgpu"),
                 AttentionPlan(fused_attention=True, custom_gemm=False),
                 AttentionPlan(fused_attention=True, custom_gemm=True, host_threads=0)):
        with pytest.raises(PlanError):
            S.Roformer(S.load_config("mel_karaoke"), {}, "cpu", plan)
