"""Parity of the gfx950 attention kernels (through the C ABI) with the oracle.

Tolerance: max-abs <= 2e-3 on the attention block, the bound the fused path is held to
(fp16 MFMA operands with fp32 accumulation and an fp32 softmax vs the reference's fp32 CPU
path), and, where outputs are small (N(0,1)/8 inputs give a near-uniform softmax and outputs
of ~4e-3), also max-abs <= 1e-3 * max|expected| (REL): about twice the fp16 rounding of the
operands, so a dropped or mis-masked key block fails it. Cases mirror
tests/cuda_contracts.rs:196-251 of the reference plus the two production shapes (time axis
T=801, band axis S=60) and their edges.
"""
import math

import numpy as np
import pytest
import torch

import oracle as O
from ancha_amd import fused
from ancha_amd import workload as W

pytestmark = pytest.mark.gpu

TOL = 2e-3
REL = 1e-3


def check(name, got, expected):
    """Both bars: max-abs <= TOL and max-abs <= REL * max|expected|."""
    err = float(np.abs(np.asarray(got, np.float64) - expected).max())
    scale = float(np.abs(expected).max())
    print(f"{name}: max|diff| {err:.3e} (max|expected| {scale:.3e}, "
          f"relative {err / max(scale, 1e-30):.2e})", flush=True)
    assert err < TOL
    assert err <= REL * scale, f"{name}: {err:.3e} > {REL} * {scale:.3e}"


def wave(shape, shift):
    n = int(np.prod(shape))
    i = np.arange(n, dtype=np.float32)
    return np.tanh(np.sin(i * np.float32(0.731) + np.float32(shift)) * np.float32(1.7)).astype(
        np.float32).reshape(shape)


def dev(a, gpu):
    return torch.from_numpy(np.ascontiguousarray(a)).to(gpu)


def report(name, err):
    print(f"{name}: max|diff| {err:.3e}", flush=True)


@pytest.mark.parametrize("groups,tokens,heads,strided",
                         [(2, 1, 1, False), (3, 63, 2, False), (2, 65, 1, True),
                          (1, 130, 3, False)])
def test_fused_attention_matches_reference_cases(gpu, groups, tokens, heads, strided):
    width = 128 if strided else 64
    raw = [wave((groups, tokens, heads, width), s)[..., :64] for s in (0.1, 1.3, 2.9)]
    q, k, v = raw[0] * np.float32(0.4), raw[1], raw[2]
    qs = q * np.float32(0.125)
    expected = O.attention_op(qs, k, v)
    if strided:
        full = [dev(wave((groups, tokens, heads, width), s), gpu) for s in (0.1, 1.3, 2.9)]
        tq = full[0][..., :64] * 0.4 * 0.125
        tk, tv = full[1][..., :64], full[2][..., :64]
    else:
        tq, tk, tv = dev(qs, gpu), dev(k, gpu), dev(v, gpu)
    got = fused.attention(tq, tk, tv)
    assert got is not None and tuple(got.shape) == (groups, tokens, heads, 64)
    err = np.abs(got.cpu().numpy() - expected).max()
    report(f"attention {groups}x{tokens}x{heads}", err)
    assert err < TOL

    # The packed RoFormer layout: q | k | v | per-head gates | 5 zero columns (unaligned rows).
    gates = wave((groups, tokens, heads), 4.4) * np.float32(3.0)
    flat = lambda a: a.reshape(groups, tokens, heads * 64)
    packed = np.concatenate([flat(qs), flat(k), flat(v), gates,
                             np.zeros((groups, tokens, 5), np.float32)], axis=2)
    got = fused.gated_attention(dev(packed, gpu), heads)
    gated = expected / (1.0 + np.exp(-gates.astype(np.float64)))[..., None]
    err = np.abs(got.cpu().numpy() - gated).max()
    report(f"gated {groups}x{tokens}x{heads}", err)
    assert err < TOL


def test_unsupported_shapes_return_none(gpu):
    narrow = dev(wave((1, 8, 1, 32), 0.0), gpu)
    assert fused.attention(narrow, narrow, narrow) is None
    packed = dev(np.zeros((1, 8, 3 * 64), np.float32), gpu)
    assert fused.gated_attention(packed, 1) is None


def seeded(shape, gpu):
    q, k, v = (W.normal_torch(shape, s, 1.0 / 8.0, device=gpu) for s in (1, 2, 3))
    return q, k, v


def oracle_slice(q, k, v, table, groups):
    """Oracle (fp64) output for the listed groups."""
    idx = torch.tensor(groups, device=q.device)
    pick = lambda t: t.index_select(0, idx).cpu().numpy()
    return O.attention_op(pick(q), pick(k), pick(v), rope=table)


@pytest.mark.parametrize("tokens", [2, 60, 62, 64, 65, 127, 128, 129, 530, 640, 641, 801, 1101])
def test_rope_on_load_matches_oracle(gpu, tokens):
    """T = 530, 640 and 1101 end in a partial query block of at most four 32-query tiles after
    whole 512-query blocks, 641 in one of five."""
    groups = 3 if tokens > 200 else 5
    q, k, v = seeded((groups, tokens, 8, 64), gpu)
    table = W.axis_rope_packed(W.rope_freqs(), tokens)
    got = fused.attention(q, k, v, rope=dev(table, gpu)).cpu().numpy()
    expected = O.attention_op(q.cpu().numpy(), k.cpu().numpy(), v.cpu().numpy(), rope=table)
    check(f"rope T={tokens}", got, expected)


@pytest.mark.parametrize("tokens,table_offset", [(60, 0), (130, 0), (801, 0), (130, 1), (801, 1),
                                                (1101, 0), (1101, 1)])
def test_gated_rope_on_unaligned_packed_rows(gpu, tokens, table_offset):
    # RoPE on load with rows whose stride is not a multiple of 4 floats (q | k | v | gates |
    # 6 zero columns: 585 per row): the element-wise load path of both attention kernels; with
    # table_offset 1 the rotary table also starts 4 bytes past a 16-byte boundary (its rows are
    # then read element-wise too).
    groups, heads = 2, 3
    q, k, v = (W.normal_torch((groups, tokens, heads, 64), s, 1.0, device=gpu) for s in (5, 6, 7))
    gates = W.normal_torch((groups, tokens, heads), 8, 2.0, device=gpu)
    flat = lambda t: t.reshape(groups, tokens, heads * 64)
    packed = torch.cat([flat(q), flat(k), flat(v), gates,
                        torch.zeros((groups, tokens, 6), device=gpu)], dim=2)
    assert packed.shape[2] % 4 != 0
    table = W.axis_rope_packed(W.rope_freqs(), tokens)
    store = torch.zeros(table.size + table_offset, device=gpu)
    store[table_offset:] = dev(table.ravel(), gpu)
    table_dev = store[table_offset:].view(table.shape)
    assert (table_dev.data_ptr() % 16 == 0) == (table_offset == 0)
    got = fused.gated_attention(packed, heads, rope=table_dev)
    assert got is not None
    expected = O.attention_op(q.cpu().numpy(), k.cpu().numpy(), v.cpu().numpy(), rope=table)
    expected = expected / (1.0 + np.exp(-gates.cpu().numpy().astype(np.float64)))[..., None]
    check(f"gated rope unaligned T={tokens} table offset {table_offset}", got.cpu().numpy(),
          expected)


def test_rope_on_load_equals_prerotated_inputs(gpu):
    # The two boundary modes agree: rotation in the kernel vs q/k rotated (and q scaled) by
    # the caller, as the reference's GEMM epilogue does.
    tokens = 801
    q, k, v = seeded((2, tokens, 8, 64), gpu)
    table = W.axis_rope_packed(W.rope_freqs(), tokens)
    tq = dev(table, gpu)

    def rotate(x, c, s):
        sw = torch.stack([x[..., 1::2], x[..., 0::2]], dim=-1).reshape(x.shape)
        return x * c[None, :, None, :] + sw * s[None, :, None, :]

    qr, kr = rotate(q, tq[0], tq[1]), rotate(k, tq[2], tq[3])
    a = fused.attention(q, k, v, rope=tq)
    b = fused.attention(qr, kr, v)
    err = (a - b).abs().max().item()
    report("rope modes", err)
    assert err < TOL


def test_time_axis_full_size(gpu):
    """The time-axis op at its production size [120, 801, 8, 64], RoPE on load: sampled groups
    against the oracle, every output checked finite and inside the convex hull of v."""
    q, k, v = seeded(W.TIME_SHAPE, gpu)
    table = W.axis_rope_packed(W.rope_freqs(), W.TIME_SHAPE[1])
    out = fused.attention(q, k, v, rope=dev(table, gpu))
    torch.cuda.synchronize()
    assert torch.isfinite(out).all()
    lo, hi = v.amin(dim=1, keepdim=True), v.amax(dim=1, keepdim=True)
    assert (out >= lo - TOL).all() and (out <= hi + TOL).all()
    groups = [0, 61, 119]
    expected = oracle_slice(q, k, v, table, groups)
    check("time full-size", out[groups].cpu().numpy(), expected)
    # Every (group, head) pass, against the fp32 restatement: the persistent walk (here the
    # paired walk of uneven rounds) must cover each pass exactly once.
    ref = torch_attention(q, k, v, dev(table, gpu))
    err = float((out - ref).abs().max())
    print(f"time full-size, all groups vs fp32: max|diff| {err:.3e}", flush=True)
    assert err <= REL * float(ref.abs().max())
    again = fused.attention(q, k, v, rope=dev(table, gpu))
    assert torch.equal(out, again), "kernel must be deterministic"


def torch_attention(q, k, v, table):
    """fp32 torch restatement used only where the oracle would be too slow: every group at the
    production size. q, k, v [G, T, H, 64]; table [4, T, 64] (q cos, q sin, k cos, k sin)."""
    def rotate(x, c, s):
        sw = torch.stack([x[..., 1::2], x[..., 0::2]], dim=-1).reshape(x.shape)
        return x * c[None, :, None, :] + sw * s[None, :, None, :]

    g, t, h, d = q.shape
    per_head = lambda x: x.permute(0, 2, 1, 3).reshape(g * h, t, d).contiguous()
    qr, kr, vh = per_head(rotate(q, table[0], table[1])), per_head(rotate(k, table[2], table[3])), \
        per_head(v)
    p = torch.softmax(torch.matmul(qr, kr.transpose(1, 2).contiguous()), dim=-1)
    return torch.matmul(p, vh).reshape(g, h, t, d).permute(0, 2, 1, 3)


def test_band_axis_full_size(gpu):
    """The band-axis op at its production size [1602, 60, 8, 64]: sampled groups against the
    oracle (including the last two, outside the whole chunks of eight groups of the kernel's
    XCD-grouped problem order) and every group against an fp32 torch restatement."""
    q, k, v = seeded(W.BAND_SHAPE, gpu)
    table = W.axis_rope_packed(W.rope_freqs(), W.BAND_SHAPE[1])
    tq = dev(table, gpu)
    out = fused.attention(q, k, v, rope=tq)
    torch.cuda.synchronize()
    assert torch.isfinite(out).all()
    groups = [0, 1, 7, 8, 800, 1599, 1600, 1601]
    expected = oracle_slice(q, k, v, table, groups)
    check("band full-size", out[groups].cpu().numpy(), expected)
    ref = torch_attention(q, k, v, tq)
    err, scale = (out - ref).abs().max().item(), ref.abs().max().item()
    report("band full-size, every group vs fp32 torch", err)
    assert err < TOL and err <= REL * scale, (err, scale)


@pytest.mark.parametrize("groups,tokens,heads", [(19, 60, 3), (17, 33, 8), (8, 64, 5)])
def test_band_problem_order_covers_every_problem(gpu, groups, tokens, heads):
    """Short-sequence problems are taken in an XCD-grouped order (whole chunks of eight groups,
    then the rest in plain order): every (group, head) must be computed once, for group counts
    that are not a multiple of eight and head counts other than eight."""
    q, k, v = seeded((groups, tokens, heads, 64), gpu)
    table = W.axis_rope_packed(W.rope_freqs(), tokens)
    got = fused.attention(q, k, v, rope=dev(table, gpu)).cpu().numpy()
    expected = O.attention_op(q.cpu().numpy(), k.cpu().numpy(), v.cpu().numpy(), rope=table)
    check(f"band order {groups}x{tokens}x{heads}", got, expected)


@pytest.mark.parametrize("tokens", [60, 801])
def test_gated_attention_production_layout(gpu, tokens):
    """The Mel-RoFormer packed projection: [G, T, 1664] = q | k | v (512 each) | 8 gates | pad,
    RoPE on load."""
    groups, heads = 4, 8
    packed = W.normal_torch((groups, tokens, 1664), 9, 0.5, device=gpu)
    table = W.axis_rope_packed(W.rope_freqs(), tokens)
    got = fused.gated_attention(packed, heads, rope=dev(table, gpu)).cpu().numpy()
    expected = O.gated_attention(packed.cpu().numpy(), heads, rope=table)
    check(f"gated production T={tokens}", got, expected)


def test_runs_on_a_side_stream(gpu):
    q, k, v = seeded((2, 801, 8, 64), gpu)
    ref = fused.attention(q, k, v)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        got = fused.attention(q, k, v)
    torch.cuda.current_stream().wait_stream(s)
    assert torch.equal(ref, got)


def test_kernels_match_golden_fixtures(gpu):
    from tests.golden import cases as C
    import os
    here = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
    slices = np.load(os.path.join(here, "production_slices.npz"), allow_pickle=False)
    for name, (shape, rows, heads) in C.SLICES.items():
        q, k, v, table, _ = C.slice_case(shape)
        got = fused.attention(dev(q, gpu), dev(k, gpu), dev(v, gpu), rope=dev(table, gpu))
        err = np.abs(got.cpu().numpy()[0][np.ix_(rows, heads)] - slices[name]).max()
        report(f"golden {name} slice", err)
        assert err < TOL
    cases = np.load(os.path.join(here, "attention_cases.npz"), allow_pickle=False)
    for shape in C.ATTENTION_SHAPES:
        q, k, v, gates, packed = C.attention_case(*shape)
        got = fused.gated_attention(dev(packed, gpu), shape[2])
        err = np.abs(got.cpu().numpy() - cases["gated_" + "x".join(map(str, shape))]).max()
        report(f"golden gated {shape}", err)
        assert err < TOL


@pytest.mark.parametrize("tokens", [801, 1101, 60])
def test_tail_keys_are_attended_and_padding_is_masked(gpu, tokens):
    """Every real key scores -5 (q . k = -5 for all pairs), so the softmax is uniform over the
    real keys and the output is the mean of v. v is 0 except on the last partial 64-key tile
    (keys 768..800 at T = 801), where it is +-1. Dropping that tile moves the output by
    33/801 ~ 0.04; scoring the zero-filled padding keys past T instead of masking them (score 0
    beats -5 by e^5 per key) shrinks it several-fold. Both fail the bars by orders of
    magnitude."""
    groups, heads = 2, 8
    tail0 = tokens // 64 * 64 if tokens % 64 else tokens - 64
    q = np.zeros((groups, tokens, heads, 64), np.float32)
    k = np.zeros_like(q)
    q[..., 0] = 1.0
    k[..., 0] = -5.0
    v = np.zeros_like(q)
    sign = np.where(np.arange(64) % 2 == 0, 1.0, -1.0).astype(np.float32)
    # 0.5 + h/16: exact in fp16, so the kernel's operand rounding adds no error here.
    v[:, tail0:] = sign * (0.5 + np.arange(heads, dtype=np.float32) / 16)[:, None]
    expected = O.attention_op(q, k, v)
    got = fused.attention(dev(q, gpu), dev(k, gpu), dev(v, gpu)).cpu().numpy()
    want_mean = 0.9375 * (tokens - tail0) / tokens
    assert abs(expected[0, 0, 7, 0] - want_mean) < 1e-6
    check(f"tail keys T={tokens}", got, expected)


@pytest.mark.parametrize("tokens", [96, 128, 130, 801, 1101])
def test_time_attention_is_repeatable(gpu, tokens):
    """Three calls on the same inputs give identical bits, and all of them match the oracle.
    Every query block of a wave is covered (T = 96 ends inside a wave's second 32-query block).
    An MFMA chain whose 16-register destination overlaps its operand registers gives
    products that vary from call to call, in the second query block of each wave."""
    q, k, v = seeded((2, tokens, 4, 64), gpu)
    expected = O.attention_op(q.cpu().numpy(), k.cpu().numpy(), v.cpu().numpy())
    outs = [fused.attention(q, k, v) for _ in range(3)]
    torch.cuda.synchronize()
    for i, out in enumerate(outs):
        check(f"repeat {i} T={tokens}", out.cpu().numpy(), expected)
    assert all(torch.equal(outs[0], o) for o in outs[1:]), "attention must be deterministic"
