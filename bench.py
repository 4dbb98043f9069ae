#!/usr/bin/env python3
"""Benchmark of the fused RoFormer attention path on one MI355X.

Default workload (the op the headline metric is quoted on): the time-axis fused attention
over q, k, v float32 [G=120 (2 chunks x 60 bands), T=801 frames, H=8, d=64], N(0,1)/8 entries
from seeds 1/2/3, RoPE (theta=10000) applied on load from the packed [4, 801, 64] table whose
query half carries the 1/8 softmax scale. One step = one call of the op over the whole batch,
inputs resident in HBM.

Prints ONE JSON line: throughput in TFLOP/s (4*G*H*T^2*d per call), the live roofline of the
attention kernel (HIP events over the timed region on the launch stream) and the restated
reference CPU path (the oracle's materialized-tile attention) timed on the host's cores. The
same line carries the path's other configurations, each as its `--workload` measures it with
its own roofline and CPU baseline: "band_attention" (the band-axis op), "layer_pair" (one
RoFormer layer pair), "mel_roformer" (the second half of the headline metric: audio-seconds per
second of the Mel-RoFormer separation of a 30 s clip) and "bs_roformer_large" (BS-RoFormer-large
on a 5 min clip). `--no-extra` / `--no-mel` leave sections out.

`--workload band` measures the band-axis op [1602, 60, 8, 64] instead (HBM-bound roofline),
`--workload layer` one RoFormer layer pair on [2, 60, 801, 384], and `--workload mel` the
Mel-RoFormer separation of a 30 s stereo clip (audio-seconds per second; one step = the whole
clip: 21 chunks of STFT, network, iSTFT and overlap-add).
"""
from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_MFMA_TFLOPS = 2500.0  # MI355X dense fp16/bf16 MFMA
PEAK_HBM_GBS = 8000.0      # MI355X HBM3E


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def profiled_traffic(pattern: str, key: str = "traffic_bytes_per_launch"):
    """HBM bytes per launch (attention ops) or per step (layer pair, separations) from the
    committed counter summary profiles/<pattern> (FETCH_SIZE + WRITE_SIZE, copy-calibrated)."""
    import glob
    for path in sorted(glob.glob(os.path.join(ROOT, "profiles", pattern))):
        for line in open(path):
            if line.startswith(key + ":"):
                return int(line.split(":")[1])
    return None


def cpu_threads() -> int:
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    limit = os.environ.get("OMP_NUM_THREADS")
    if limit and limit.isdigit():
        n = min(n, int(limit))
    return max(1, n)


def cpu_baseline(q, k, v, table, gpu_out, budget_s: float = 12.0) -> dict:
    """The restated reference CPU path (oracle): RoPE tables applied on the host, then the
    Flex-path materialized score tiles (roformer.rs:324-363) with groups split over all host
    threads, on a bounded sample of the same groups. Median of 3 runs."""
    import oracle as O

    threads = cpu_threads()
    G, T, H, D = q.shape
    tq = table

    def rotate(x, c, s):
        sw = np.empty_like(x)
        sw[..., 0::2], sw[..., 1::2] = x[..., 1::2], x[..., 0::2]
        return (x * c[None, :, None, :] + sw * s[None, :, None, :]).astype(np.float32)

    # Probe one group to size the sample.
    g1 = max(1, min(G, threads))
    sample = lambda n: [np.ascontiguousarray(a[:n]) for a in (q, k, v)]
    qs, ks, vs = sample(g1)
    t0 = time.perf_counter()
    O.token_major_attention(rotate(qs, tq[0], tq[1]), rotate(ks, tq[2], tq[3]), vs,
                            threads=threads)
    probe = time.perf_counter() - t0
    groups = int(min(G, max(g1, g1 * budget_s / 3.0 / max(probe, 1e-3))))
    if groups < G and groups >= threads:
        groups = groups // threads * threads
    qs, ks, vs = sample(groups)
    times, out = [], None
    for _ in range(3):
        t0 = time.perf_counter()
        qr, kr = rotate(qs, tq[0], tq[1]), rotate(ks, tq[2], tq[3])
        out = O.token_major_attention(qr, kr, vs, threads=threads)
        times.append(time.perf_counter() - t0)
    t = statistics.median(times)
    flops = 4.0 * groups * H * T * T * D
    err = float(np.abs(out - gpu_out[:groups]).max())
    return {
        "value": round(flops / t / 1e12, 5),
        "unit": "TFLOP/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"{groups} of {G} groups x {H} heads, T={T}: host RoPE + materialized "
                   f"fp32 score tiles, groups over {threads} threads, median of 3 "
                   f"({t:.2f} s)"),
        "max_abs_vs_gpu": err,
    }


def copy_calibration(torch, dev, elements: int, steps: int) -> int:
    """A plain float32 device copy of `elements` values (read once, written once) repeated
    `steps` times; prints the bytes moved and the rate."""
    src = torch.ones(elements, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        dst.copy_(src)
    end.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / steps
    print(json.dumps({"copy_bytes_read": elements * 4, "copy_bytes_written": elements * 4,
                      "ms_per_copy": round(ms, 4),
                      "GB/s": round(2 * elements * 4 / ms / 1e6, 1)}), flush=True)
    return 0


LAYER = dict(batch=2, bands=60, frames=801, dim=384, heads=8, hidden=1536)


def layer_weights(dim, heads, hidden, seed):
    """Random-init block weights ~N(0, 0.02) (projections, gate W and b, FF W and b), gamma = 1,
    no output norm, in PyTorch nn.Linear layout."""
    from ancha_amd import workload as W
    inner = heads * 64
    shapes = {"to_qkv": (3 * inner, dim), "to_gates": (heads, dim), "to_gates_bias": (heads,),
              "to_out": (dim, inner), "ff_in": (hidden, dim), "ff_in_bias": (hidden,),
              "ff_out": (dim, hidden), "ff_out_bias": (dim,)}
    w = {name: W.normal(shape, seed + i, 0.02) for i, (name, shape) in enumerate(shapes.items())}
    w.update(heads=heads, attn_gamma=np.ones(dim, np.float32), ff_gamma=np.ones(dim, np.float32),
             output_gamma=None, freqs=W.rope_freqs())
    return w


def layer_flops(groups, tokens, dim, heads, hidden):
    """Algorithmic FLOPs of one block pass: QKV+gate projection (3*inner+heads columns),
    attention 4*G*H*T^2*64, output projection, feed-forward."""
    n, inner = groups * tokens, heads * 64
    return (2.0 * n * dim * (3 * inner + heads) + 4.0 * groups * heads * tokens ** 2 * 64
            + 2.0 * n * inner * dim + 4.0 * n * dim * hidden)


def run_layer(args, torch, dev) -> int:
    print(json.dumps(layer_result(args.steps, args.warmup, args.no_cpu_baseline, torch, dev)),
          flush=True)
    return 0


def layer_result(steps, warmup, no_cpu_baseline, torch, dev) -> dict:
    """One RoFormer layer pair (time pass then band pass) on x [2, 60, 801, 384]."""
    from ancha_amd import roformer
    from ancha_amd import workload as W
    c = LAYER
    B, NB, T, D = c["batch"], c["bands"], c["frames"], c["dim"]
    wt = layer_weights(D, c["heads"], c["hidden"], 300)
    wb = layer_weights(D, c["heads"], c["hidden"], 400)
    pair = roformer.AxisPair(roformer.Transformer(wt, dev), roformer.Transformer(wb, dev))
    x = W.normal_torch((B, NB, T, D), W.SEED_X, 1.0, device=dev)
    tt = roformer.axis_rope(wt["freqs"], T, dev)
    tb = roformer.axis_rope(wb["freqs"], NB, dev)
    step = lambda: pair(x, tt, tb)
    out = step()
    for _ in range(warmup):
        out = step()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record(stream)
    for _ in range(steps):
        out = step()
    end.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    gpu_ms = start.elapsed_time(end) / steps
    flops_time = layer_flops(B * NB, T, D, c["heads"], c["hidden"])
    flops_band = layer_flops(B * T, NB, D, c["heads"], c["hidden"])
    flops = flops_time + flops_band
    achieved = flops / (gpu_ms * 1e-3) / 1e12
    log(f"layer pair: {gpu_ms:.3f} ms/step, {achieved:.1f} TFLOP/s")
    result = {
        "metric": "RoFormer layer pair TFLOP/s (% MFMA peak)",
        "value": round(flops * steps / wall / 1e12, 3),
        "unit": "TFLOP/s", "n_gpus": 1, "steps": steps, "warmup": warmup,
        "ms_per_step": round(wall * 1e3 / steps, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "fp16",
        "data": "synthetic: x ~ N(0,1), weights ~ N(0,0.02), gamma = 1 (seeded)",
        "config": {"workload": "RoFormer layer pair: time pass on [120, 801, 384] then band "
                               "pass on [1602, 60, 384]", "dim": D, "heads": c["heads"],
                   "head_dim": 64, "ff_hidden": c["hidden"], "io": "fp32",
                   "mfma_operands": "fp16", "accumulate": "fp32",
                   "gflop_per_step": round(flops / 1e9, 2), "parallelism": "single GPU"},
        "roofline": {"bound": "mfma", "achieved": round(achieved, 3), "peak": PEAK_MFMA_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(achieved / PEAK_MFMA_TFLOPS, 4),
                     "traffic": profiled_traffic("layer_pair_*.md", "traffic_bytes_per_step"),
                     "scope": "whole layer pair (all kernels); traffic = HBM bytes per step"},
    }
    if not no_cpu_baseline:
        log("timing the restated reference CPU path (Burn-path block) on sampled groups")
        result["cpu_baseline"] = layer_cpu_baseline(wt, wb, x, out)
    del out, x, pair
    return result


def layer_cpu_baseline(wt, wb, x, gpu_out, budget_s: float = 12.0) -> dict:
    """The oracle's Burn-path block (separate projections, host RoPE tables, materialized score
    tiles, groups over all host threads) on a sample of time-pass groups, timed; the rate
    (TFLOP/s of that pass's algorithmic FLOPs) stands for the layer pair."""
    import oracle as O
    c = LAYER
    threads = cpu_threads()
    xs = x.view(-1, c["frames"], c["dim"])
    groups = max(1, min(threads, xs.shape[0]))
    sample = xs[:groups].cpu().numpy()
    times = []
    for _ in range(3):
        t0 = time.perf_counter()
        O.transformer_forward(wt, sample, kernels=False, threads=threads)
        times.append(time.perf_counter() - t0)
        if sum(times) > budget_s:
            break
    t = statistics.median(times)
    flops = layer_flops(groups, c["frames"], c["dim"], c["heads"], c["hidden"])
    return {"value": round(flops / t / 1e12, 5), "unit": "TFLOP/s", "cores": threads,
            "kind": "port",
            "sample": (f"time-pass block on {groups} of {xs.shape[0]} groups x 801 frames "
                       f"(Burn-path restatement, groups over {threads} threads), median of "
                       f"{len(times)} ({t:.2f} s)")}




def mel_flops(config: dict) -> float:
    """Algorithmic FLOPs of one chunk's network forward: band split, depth x (time block on
    groups = bands, frequency block on groups = frames), mask heads (hidden layers and the
    value|gate projections). The STFT / iSTFT (O(n log n)) are left out."""
    frames = config["chunk_samples"] // config["hop"] + 1
    nb, dim = len(config["bands"]), config["dim"]
    widths = [4 * len(b) for b in config["bands"]]
    hidden = dim * config["ff_mult"]
    mh = dim * config["mask_expansion"]
    layers = config["mask_depth"] if config["family"] == "mel-band-roformer" \
        else config["mask_depth"] - 1
    f = 2.0 * frames * sum(widths) * dim
    f += config["depth"] * (layer_flops(nb, frames, dim, config["heads"], hidden)
                            + layer_flops(frames, nb, dim, config["heads"], hidden))
    head = 2.0 * frames * nb * (dim * mh + (layers - 1) * mh * mh) + 2.0 * frames * sum(
        2 * w for w in widths) * mh
    return f + len(config["stems"]) * head


SEPARATIONS = {
    # workload: (bundled config, clip seconds, metric, config description)
    "mel": ("mel_karaoke", 30, "audio-seconds/sec for Mel-RoFormer fwd",
            "Mel-RoFormer separation (Mel-Karaoke: 60 bands, dim 384, depth 6, 8x64 heads, "
            "chunk 352800 / overlap 4, two chunks per forward) of a 30 s clip"),
    "bs": ("bs_roformer_large", 300, "audio-seconds/sec for BS-RoFormer-large fwd",
           "BS-RoFormer-large separation (62 bands, dim 512, depth 12, 8x64 heads, chunk 485100 "
           "/ overlap 2, two chunks per forward) of a 5 min clip"),
}
SEPARATION_PROFILES = {"mel": "mel_separation_*.md", "bs": "bs_roformer_large_*.md"}


# The reference's own published CPU speed on this model (Flex backend, batched), for context
# beside the restated CPU path: one 3 s clip (301 frames) in 6.21 s total (5.12 s model) on an
# Intel i5-12400 (6 cores / 12 threads), docs/reports/derur-benchmark.json:930-939.
REFERENCE_CPU_MEL = {"value": round(3.0 / 6.21, 4), "unit": "audio-s/s", "cores": 12,
                     "sample": "Mel-Karaoke, one 3 s clip (301 frames): 6.21 s total, 5.12 s "
                               "model, i5-12400 6C/12T (docs/reports/derur-benchmark.json:930-939)"}


def run_separation(args, torch, dev) -> int:
    result = separation_result(args.workload, args.steps, args.warmup, args.no_cpu_baseline,
                               torch, dev)
    print(json.dumps(result), flush=True)
    return 0


def separation_result(workload, steps, warmup, no_cpu_baseline, torch, dev) -> dict:
    """Separation of a stereo clip resident in HBM with a bundled config and random
    N(0, 0.02) weights: Mel-Karaoke on 30 s (`mel`) or BS-RoFormer-large on 5 min (`bs`)."""
    from ancha_amd import separation as S
    from ancha_amd import workload as W
    name, seconds, metric, described = SEPARATIONS[workload]
    config = S.load_config(name)
    sr = config["sample_rate"]
    n = seconds * sr
    log("generating weights (GPU stream) and the clip")
    tensors = W.roformer_tensors(config, device=dev)
    model = S.Roformer(config, tensors, dev)
    audio_np = W.audio(n)
    audio = torch.from_numpy(audio_np).to(dev)
    step = lambda: model.separate(audio)
    out = step()
    for _ in range(warmup):
        out = step()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record(stream)
    for _ in range(steps):
        out = step()
    end.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    gpu_ms = start.elapsed_time(end) / steps
    step_ = config["chunk_samples"] // config["overlap"]
    border = config["chunk_samples"] - step_
    border = border if n > 2 * border else 0
    chunks = len(range(0, n + 2 * border, step_))
    flops = chunks * mel_flops(config)
    achieved = flops / (gpu_ms * 1e-3) / 1e12
    log(f"{workload} separation: {gpu_ms:.1f} ms per {seconds} s clip ({chunks} chunks), "
        f"{seconds / (gpu_ms * 1e-3):.1f} audio-s/s, {achieved:.1f} TFLOP/s")
    result = {
        "metric": metric,
        "value": round(seconds * steps / wall, 3),
        "unit": "audio-s/s", "n_gpus": 1, "steps": steps, "warmup": warmup,
        "ms_per_step": round(wall * 1e3 / steps, 3), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "fp16",
        "data": f"synthetic: seeded pink noise + 3 sines, {seconds} s stereo 44.1 kHz; weights "
                "N(0,0.02), gamma 1, rotary theta 10000 (seeded)",
        "config": {"workload": described,
                   "chunks": chunks, "frames_per_chunk": config["chunk_samples"] //
                   config["hop"] + 1, "gflop_per_clip": round(flops / 1e9, 1),
                   "mfma_operands": "fp16", "accumulate": "fp32", "dsp": "fp32",
                   "parallelism": "single GPU"},
        "roofline": {"bound": "mfma", "achieved": round(achieved, 3), "peak": PEAK_MFMA_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(achieved / PEAK_MFMA_TFLOPS, 4),
                     "traffic": profiled_traffic(SEPARATION_PROFILES[workload],
                                                 "traffic_bytes_per_step"),
                     "scope": "whole separation (all kernels); traffic = HBM bytes per clip"},
    }
    if not no_cpu_baseline:
        import oracle.mel as OM
        threads = cpu_threads()
        weights = OM.weights_from_tensors(config, tensors)
        if workload == "mel":
            log(f"timing the restated reference CPU path on the first chunk ({threads} threads)")
            t0 = time.perf_counter()
            OM.separate(audio_np, config, weights, threads=threads, chunks=1)
            t = time.perf_counter() - t0
            value = seconds / chunks / t
            sample = (f"first of the clip's {chunks} chunks through the full model (STFT, "
                      f"band split, {config['depth']} layer pairs, mask head, iSTFT, "
                      f"overlap-add), credited {seconds}/{chunks} s of audio ({t:.1f} s)")
        else:
            # A whole depth-12 chunk is minutes of CPU work: time the first chunk through a
            # depth-1 model (same band split, first layer pair, mask head, DSP) and scale the
            # chunk's CPU time by the FLOP ratio of the full depth.
            shallow = dict(config, depth=1)
            weights1 = dict(weights, layers=weights["layers"][:1])
            log(f"timing the restated reference CPU path: first chunk at depth 1 "
                f"({threads} threads)")
            t0 = time.perf_counter()
            OM.separate(audio_np, shallow, weights1, threads=threads, chunks=1)
            t = time.perf_counter() - t0
            full = t * mel_flops(config) / mel_flops(shallow)
            value = seconds / chunks / full
            sample = (f"first of the clip's {chunks} chunks through a depth-1 model (band split, "
                      f"1 layer pair, mask head, STFT / iSTFT) in {t:.1f} s, scaled by the FLOP "
                      f"ratio {mel_flops(config) / mel_flops(shallow):.2f} to depth "
                      f"{config['depth']} and credited {seconds}/{chunks} s of audio")
        result["cpu_baseline"] = {"value": round(value, 5), "unit": "audio-s/s",
                                  "cores": threads, "kind": "port", "sample": sample}
        if workload == "mel":
            result["cpu_baseline"]["reference_published"] = REFERENCE_CPU_MEL
    del out
    model.close()
    return result


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None,
                    help="timed steps (default 100; 5 for --workload bs)")
    ap.add_argument("--warmup", type=int, default=None,
                    help="untimed steps (default 10; 1 for --workload bs)")
    ap.add_argument("--workload", choices=["time", "band", "layer", "mel", "bs"], default="time")
    ap.add_argument("--tokens", type=int, default=None,
                    help="sequence length of the time / band op workloads (default 801 / 60); "
                         "for length sweeps, the headline uses the default")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-mel", action="store_true",
                    help="time workload: leave out the Mel-RoFormer 30 s separation section")
    ap.add_argument("--no-extra", action="store_true",
                    help="time workload: leave out the band-op, layer-pair and BS-RoFormer-large "
                         "sections")
    ap.add_argument("--bs-steps", type=int, default=2,
                    help="timed clips of the BS-RoFormer-large section of the time workload")
    ap.add_argument("--mel-steps", type=int, default=5,
                    help="timed clips of the Mel-RoFormer section of the time workload")
    ap.add_argument("--mel-warmup", type=int, default=1)
    ap.add_argument("--copy-calibration", action="store_true",
                    help="time a plain device copy of the workload's I/O size instead; its "
                         "FETCH_SIZE / WRITE_SIZE counters calibrate the HBM traffic figures")
    args = ap.parse_args()
    if args.steps is None:
        args.steps = 5 if args.workload == "bs" else 100
    if args.warmup is None:
        args.warmup = 1 if args.workload == "bs" else 10
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path "
              "(chunk-level data parallelism would need no communication). Run with --gpus 1.",
              file=sys.stderr)
        return 2

    import torch

    from ancha_amd import fused

    if not torch.cuda.is_available() or not fused.available():
        print("bench.py needs an MI355X (gfx950) GPU and the built kernel library",
              file=sys.stderr)
        return 2
    dev = torch.device("cuda:0")
    if args.workload == "layer":
        return run_layer(args, torch, dev)
    if args.workload in SEPARATIONS:
        return run_separation(args, torch, dev)
    if args.tokens is not None and not 1 <= args.tokens <= 8192:
        print("--tokens must be in [1, 8192]", file=sys.stderr)
        return 2
    result = attention_result(args.workload, args.steps, args.warmup, args.no_cpu_baseline,
                              args.tokens, args.copy_calibration, torch, dev)
    if result is None:
        return 0
    if args.workload == "time" and args.tokens is None:
        # The other configurations of the path, each with its own roofline (and CPU baseline),
        # in the same JSON line: the band-axis op, one layer pair, and the second half of the
        # headline metric, the Mel-RoFormer separation of a 30 s clip; BS-RoFormer-large last.
        if not args.no_extra:
            log("band-axis op [1602, 60, 8, 64]")
            result["band_attention"] = attention_result(
                "band", args.steps, args.warmup, args.no_cpu_baseline, None, False, torch, dev)
            log("layer pair [2, 60, 801, 384]")
            result["layer_pair"] = layer_result(args.steps, min(args.warmup, 10),
                                                args.no_cpu_baseline, torch, dev)
        if not args.no_mel:
            log("Mel-RoFormer separation of a 30 s clip")
            result["mel_roformer"] = separation_result("mel", args.mel_steps, args.mel_warmup,
                                                       args.no_cpu_baseline, torch, dev)
        if not args.no_extra:
            log("BS-RoFormer-large separation of a 5 min clip")
            result["bs_roformer_large"] = separation_result(
                "bs", args.bs_steps, 1, args.no_cpu_baseline, torch, dev)
    print(json.dumps(result), flush=True)
    return 0


def attention_result(workload, steps, warmup, no_cpu_baseline, tokens, copy_cal, torch, dev):
    """The fused attention op on q, k, v resident in HBM: the time-axis shape (MFMA roofline)
    or the band-axis shape (HBM roofline), RoPE on load."""
    from ancha_amd import fused
    from ancha_amd import workload as W
    shape = W.TIME_SHAPE if workload == "time" else W.BAND_SHAPE
    if tokens is not None:
        shape = (shape[0], tokens, shape[2], shape[3])
    G, T, H, D = shape
    default_shape = tokens is None
    log(f"generating q, k, v {shape} on the GPU")
    q, k, v = (W.normal_torch(shape, s, 1.0 / 8.0, device=dev) for s in (1, 2, 3))
    if copy_cal:
        copy_calibration(torch, dev, G * T * H * D * 2, steps)
        return None
    table_np = W.axis_rope_packed(W.rope_freqs(), T)
    table = torch.from_numpy(table_np).to(dev)
    torch.cuda.synchronize()

    def step():
        return fused.attention(q, k, v, rope=table)

    out = step()
    assert out is not None, "attention kernel rejected the workload"
    for _ in range(warmup):
        out = step()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record(stream)
    for _ in range(steps):
        out = step()
    end.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    kernel_ms = start.elapsed_time(end) / steps
    flops = 4.0 * G * H * T * T * D
    io_bytes = 4.0 * 4 * G * T * H * D  # q, k, v read + out written, fp32
    value = flops * steps / wall / 1e12
    log(f"{workload}: {kernel_ms * 1e3:.1f} us/launch, {flops / kernel_ms / 1e9:.1f} TFLOP/s, "
        f"{io_bytes / kernel_ms / 1e6:.0f} GB/s")
    if workload == "time":
        achieved = flops / (kernel_ms * 1e-3) / 1e12
        roofline = {"bound": "mfma", "achieved": round(achieved, 3), "peak": PEAK_MFMA_TFLOPS,
                    "unit": "TFLOP/s", "frac": round(achieved / PEAK_MFMA_TFLOPS, 4),
                    "traffic": profiled_traffic("attention_time_*.md") if default_shape else None}
    else:
        achieved = io_bytes / (kernel_ms * 1e-3) / 1e9
        roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_HBM_GBS,
                    "unit": "GB/s", "frac": round(achieved / PEAK_HBM_GBS, 4),
                    "traffic": profiled_traffic("attention_band_*.md") if default_shape else None}
    result = {
        "metric": "fused attn TFLOP/s (% MFMA peak)",
        "value": round(value, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": round(wall * 1e3 / steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic: seeded N(0,1)/8 q, k, v (splitmix64 + Box-Muller)",
        "config": {"workload": f"{workload}-axis fused attention, RoPE on load",
                   "groups": G, "tokens": T, "heads": H, "head_dim": D,
                   "io": "fp32", "mfma_operands": "fp16", "accumulate": "fp32",
                   "parallelism": "single GPU"},
        "roofline": roofline,
    }
    if not no_cpu_baseline:
        log("timing the restated reference CPU path")
        result["cpu_baseline"] = cpu_baseline(q.cpu().numpy(), k.cpu().numpy(),
                                              v.cpu().numpy(), table_np, out.cpu().numpy())
    del q, k, v, out
    return result


if __name__ == "__main__":
    sys.exit(main())
