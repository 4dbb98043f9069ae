"""Parity of the gfx950 projection GEMM, row norm and RoFormer block (through the C ABI) with
the oracle.

GEMM tolerance: the kernel rounds x and w to fp16 (relative error <= 2^-11 each) and
accumulates in fp32, so |got - exact| <= 2^-10 * sum_k |x_ik| |w_kj| (+ fp32 accumulation,
~1e-6 relative). Tests assert that bound per element, times the Lipschitz constant of the
epilogue that follows (1.13 for erf-GELU, sqrt(2) for a pair rotation, 1 for bias/residual).
Attention-block outputs are held to the path's 2e-3 max-abs bound.
Cases follow tests/cuda_contracts.rs:253-297 of the reference (the GEMM epilogues) and
Transformer::forward_kernels (roformer.rs:464-520) for the block.
"""
import os

import numpy as np
import pytest
import torch

import oracle as O
from ancha_amd import fused, roformer
from ancha_amd import workload as W
from tests.golden import cases as C

pytestmark = pytest.mark.gpu

EPS16 = 2.0 ** -10
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def dev(a, gpu):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(gpu)


def bound(x, w, lipschitz=1.0):
    return lipschitz * (EPS16 * (np.abs(x).astype(np.float64) @ np.abs(w).astype(np.float64))
                        + 1e-5)


def check(name, got, want, tol):
    err = np.abs(got.astype(np.float64) - want)
    ratio = float((err / tol).max())
    print(f"{name}: max|diff| {err.max():.3e}, worst diff/bound {ratio:.3f}", flush=True)
    assert ratio <= 1.0, name


def test_reference_epilogue_cases(gpu):
    x, w, b, r, table, _ = C.linear_case()
    tokens, width = C.LINEAR_TOKENS, C.LINEAR_WIDTH
    X, Wt, B, R = dev(x, gpu), dev(w, gpu), dev(b, gpu), dev(r, gpu)
    ep = fused.Epilogue(bias=B, gelu=True, residual=R)
    got = fused.linear(X, Wt, ep).cpu().numpy()
    want = O.linear(x, w, bias=b, gelu=True, residual=r)
    check("bias+GELU+residual", got, want, bound(x, w, 1.13))
    ep = fused.Epilogue(bias=B, rotary=(dev(table, gpu), width))
    got = fused.linear(X, Wt, ep).cpu().numpy()
    want = O.linear(x, w, bias=b, rope=table, tokens=tokens, width=width)
    check("bias+rotary", got, want, bound(x, w, 1.42))
    # The committed golden rows (independent float64 restatement).
    f = np.load(os.path.join(GOLDEN, "linear_epilogue.npz"), allow_pickle=False)
    check("rotary golden rows", got[C.LINEAR_ROTARY_ROWS], f["rotary_rows"],
          bound(x, w, 1.42)[C.LINEAR_ROTARY_ROWS] + 1e-6)


@pytest.mark.parametrize("n,k,m,ldx", [(1000, 384, 1664, 384), (77, 1536, 384, 1536),
                                       (130, 512, 384, 515), (5, 8, 128, 8)])
def test_shapes_and_strides(gpu, n, k, m, ldx):
    base = W.normal((n, ldx), 11, 1.0)
    x = base[:, :k]
    w = W.normal((k, m), 12, 0.05)
    b = W.normal((m,), 13, 0.1)
    r = W.normal((n, m), 14, 1.0)
    X = dev(base, gpu)[:, :k]
    got = fused.linear(X, dev(w, gpu), fused.Epilogue(bias=dev(b, gpu), residual=dev(r, gpu)))
    check(f"linear {n}x{k}x{m} ldx {ldx}", got.cpu().numpy(),
          O.linear(x, w, bias=b, residual=r), bound(x, w))


def test_bare_product_pads_narrow_m(gpu):
    x = W.normal((300, 64), 21, 1.0)
    w = W.normal((64, 200), 22, 0.1)
    got = fused.linear(dev(x, gpu), dev(w, gpu))
    assert tuple(got.shape) == (300, 200)
    check("bare 300x64x200", got.cpu().numpy(), O.linear(x, w), bound(x, w))
    # Odd m takes the element-wise path.
    w = W.normal((64, 131), 23, 0.1)
    got = fused.linear(dev(x, gpu), dev(w, gpu))
    check("bare 300x64x131", got.cpu().numpy(), O.linear(x, w), bound(x, w))


def test_unsupported_shapes_return_none(gpu):
    x = dev(np.ones((4, 12), np.float32), gpu)
    assert fused.linear(x, dev(np.ones((12, 128), np.float32), gpu)) is None        # k % 8
    x = dev(np.ones((4, 16), np.float32), gpu)
    b = dev(np.ones(200, np.float32), gpu)
    assert fused.linear(x, dev(np.ones((16, 200), np.float32), gpu),
                        fused.Epilogue(bias=b)) is None                            # m % 128
    t = dev(np.ones((4, 3, 64), np.float32), gpu)
    assert fused.linear(x, dev(np.ones((16, 128), np.float32), gpu),
                        fused.Epilogue(rotary=(t, 64))) is None                    # 2w > m


def test_norm_linear_matches_unit_norm_then_linear(gpu):
    n, k, m = 1001, 384, 1536
    x = W.normal((n, k), 31, 2.0)
    x[7] = 0.0                                    # the 1e-12 floor: a zero row stays zero
    w = W.normal((k, m), 32, 0.4)
    b = W.normal((m,), 33, 0.1)
    got = fused.norm_linear(dev(x, gpu), dev(w, gpu),
                            fused.Epilogue(bias=dev(b, gpu), gelu=True)).cpu().numpy()
    xn = O.unit_norm(x)
    want = O.linear(xn, w, bias=b, gelu=True)
    check("norm_linear + bias + GELU", got, want, bound(xn, w, 1.13) + 1e-6)


@pytest.mark.parametrize("rows,dim,scaled", [(96120, 384, False), (1000, 384, True),
                                             (33, 131, True), (4, 8, False)])
def test_unit_norm(gpu, rows, dim, scaled):
    x = W.normal((rows, dim), 41, 3.0)
    x[min(2, rows - 1)] = 0.0
    scale = (1.0 + W.normal((dim,), 42, 0.1)) * np.float32(np.sqrt(dim)) if scaled else None
    got = fused.unit_norm(dev(x, gpu), None if scale is None else dev(scale, gpu))
    want = O.unit_norm(x, scale)
    err = float(np.abs(got.cpu().numpy() - want).max())
    print(f"unit_norm {rows}x{dim}: max|diff| {err:.3e}", flush=True)
    assert err < (2e-6 if scale is None else 5e-5)


def _block_weights(dim, heads, hidden, normalized=True):
    w, _ = C.layer_case() if (dim, heads, hidden) == (C.LAYER_DIM, C.LAYER_HEADS,
                                                      C.LAYER_HIDDEN) else (None, None)
    if w is None:
        shapes = {
            "attn_gamma": (dim,), "to_qkv": (3 * heads * 64, dim), "to_gates": (heads, dim),
            "to_gates_bias": (heads,), "to_out": (dim, heads * 64), "ff_gamma": (dim,),
            "ff_in": (hidden, dim), "ff_in_bias": (hidden,), "ff_out": (dim, hidden),
            "ff_out_bias": (dim,), "output_gamma": (dim,)}
        w = {"heads": heads, "freqs": W.rope_freqs()}
        for i, (name, shape) in enumerate(sorted(shapes.items())):
            w[name] = (1.0 + W.normal(shape, 100 + i, 0.1) if name.endswith("gamma")
                       else W.normal(shape, 100 + i, 0.02))
    if not normalized:
        w = dict(w, output_gamma=None)
    return w


def test_block_matches_golden_layer(gpu):
    w, x = C.layer_case()
    block = roformer.Transformer(w, gpu)
    table = roformer.axis_rope(w["freqs"], x.shape[1], gpu)
    got = block(dev(x, gpu), table).cpu().numpy()
    golden = np.load(os.path.join(GOLDEN, "layer.npz"), allow_pickle=False)["out"]
    err = float(np.abs(got - golden).max())
    ref = float(np.abs(O.transformer_forward(w, x, kernels=True) - golden).max())
    print(f"block vs golden layer: max|diff| {err:.3e} (oracle f32 {ref:.1e})", flush=True)
    assert err < 2e-3
    xd = dev(x, gpu)
    assert torch.equal(block(xd, table), block(xd, table))  # deterministic


@pytest.mark.parametrize("axis", ["time", "band"])
def test_block_attention_core_at_layer_pair_shape(gpu, axis):
    """The dim-384 block of the layer-pair workload ([2, 60, 801, 384]) on a sample of its
    groups: the attention-block output (packed GEMM -> gated attention) within 2e-3 of the
    oracle, and the block output within the GEMM bound's scale."""
    dim, heads, hidden = 384, 8, 1536
    tokens = 801 if axis == "time" else 60
    groups = 3
    w = _block_weights(dim, heads, hidden, normalized=True)
    x = W.normal((groups, tokens, dim), 4, 1.0)
    table_np = W.axis_rope_packed(W.rope_freqs(), tokens)
    table = dev(table_np, gpu)
    block = roformer.Transformer(w, gpu)
    # Attention core through the block's own packed weights and the public ops.
    inner, columns = heads * 64, 1664
    s = np.float32(np.sqrt(np.float32(dim))) * w["attn_gamma"]
    wp = np.zeros((dim, columns), np.float32)
    wp[:, :3 * inner] = (w["to_qkv"] * s[None, :]).T
    wp[:, 3 * inner:3 * inner + heads] = (w["to_gates"] * s[None, :]).T
    bp = np.zeros(columns, np.float32)
    bp[3 * inner:3 * inner + heads] = w["to_gates_bias"]
    rows = groups * tokens
    packed = fused.norm_linear(dev(x.reshape(rows, dim), gpu), dev(wp, gpu),
                               fused.Epilogue(bias=dev(bp, gpu), rotary=(table, inner)))
    attended = fused.gated_attention(packed.view(groups, tokens, columns), heads).cpu().numpy()
    xn = O.unit_norm(x.reshape(rows, dim), precision="f32")
    packed_ref = O.linear(xn, wp, bias=bp, rope=table_np, tokens=tokens, width=inner,
                          precision="f32").reshape(groups, tokens, columns)
    want = O.gated_attention(packed_ref, heads)
    err = float(np.abs(attended - want).max())
    print(f"{axis} attention block [3, {tokens}, 384]: max|diff| {err:.3e}", flush=True)
    assert err < 2e-3
    got = block(dev(x, gpu), table).cpu().numpy()
    want = O.transformer_forward(w, x, kernels=True, threads=8)
    err = float(np.abs(got - want).max())
    print(f"{axis} block output: max|diff| {err:.3e}", flush=True)
    assert err < 2e-3


def _oracle_pair(wt, wb, x):
    batch, bands, frames, dim = x.shape
    y = O.transformer_forward(wt, x.reshape(batch * bands, frames, dim), kernels=True, threads=8)
    y = y.reshape(batch, bands, frames, dim).transpose(0, 2, 1, 3).copy()
    z = O.transformer_forward(wb, y.reshape(batch * frames, bands, dim), kernels=True, threads=8)
    return z.reshape(batch, frames, bands, dim).transpose(0, 2, 1, 3)


def test_swap_axes(gpu):
    x = W.normal((2, 5, 7, 12), 51, 1.0)
    got = roformer.swap_axes(dev(x, gpu)).cpu().numpy()
    assert np.array_equal(got, x.transpose(0, 2, 1, 3))
    x = W.normal((2, 60, 33, 384), 52, 1.0)
    assert np.array_equal(roformer.swap_axes(dev(x, gpu)).cpu().numpy(), x.transpose(0, 2, 1, 3))


def test_axis_pair_small(gpu):
    wt, _ = C.layer_case()
    wb = _block_weights(C.LAYER_DIM, C.LAYER_HEADS, C.LAYER_HIDDEN)
    wb = {k: (v * np.float32(1.1) if isinstance(v, np.ndarray) and k.startswith("to_") else v)
          for k, v in wb.items()}
    x = W.normal((2, 5, 37, C.LAYER_DIM), 53, 1.0)
    pair = roformer.AxisPair(roformer.Transformer(wt, gpu), roformer.Transformer(wb, gpu))
    got = pair(dev(x, gpu), roformer.axis_rope(wt["freqs"], 37, gpu),
               roformer.axis_rope(wb["freqs"], 5, gpu)).cpu().numpy()
    err = float(np.abs(got - _oracle_pair(wt, wb, x)).max())
    print(f"axis pair [2, 5, 37, 128]: max|diff| {err:.3e}", flush=True)
    assert err < 2e-3


def test_axis_pair_layer_pair_shape(gpu):
    """The layer-pair workload [2, 60, 801, 384]: finite, deterministic, and its band pass on
    sampled frames equals the oracle's block applied to the GPU's own time-pass output."""
    dim, heads, hidden, batch, bands, frames = 384, 8, 1536, 2, 60, 801
    wt = _block_weights(dim, heads, hidden, normalized=False)
    wb = {k: (W.normal(v.shape, 200 + i, 0.02) if isinstance(v, np.ndarray) and
              k.startswith(("to_", "ff_in", "ff_out")) else v)
          for i, (k, v) in enumerate(sorted(wt.items()))}
    x = dev(W.normal((batch, bands, frames, dim), 4, 1.0), gpu)
    tt, tb = roformer.axis_rope(W.rope_freqs(), frames, gpu), roformer.axis_rope(
        W.rope_freqs(), bands, gpu)
    time, band = roformer.Transformer(wt, gpu), roformer.Transformer(wb, gpu)
    pair = roformer.AxisPair(time, band)
    out = pair(x, tt, tb)
    assert torch.isfinite(out).all()
    assert torch.equal(out, pair(x, tt, tb))
    y = roformer.swap_axes(time(x.view(batch * bands, frames, dim), tt).view(
        batch, bands, frames, dim))                       # [batch, frames, bands, dim]
    sample = [0, 400, 800 + frames]                       # flattened (batch, frame) groups
    ys = y.view(batch * frames, bands, dim)[sample].cpu().numpy()
    want = O.transformer_forward(wb, ys, kernels=True, threads=8)
    got = out.permute(0, 2, 1, 3).reshape(batch * frames, bands, dim)[sample].cpu().numpy()
    err = float(np.abs(got - want).max())
    print(f"layer pair band pass on sampled frames: max|diff| {err:.3e}", flush=True)
    assert err < 2e-3


@pytest.mark.parametrize("tokens", [1, 2, 17, 63, 64, 65, 127, 128, 129, 200])
def test_block_ragged_sequence_lengths(gpu, tokens):
    """The block (fp16 normalised operands, fp16 packed projection read by the attention kernels)
    at sequence lengths around the band kernel's limit (64) and the time kernel's 64-key tiles,
    with an output norm; 3 sequences each."""
    dim, heads, hidden, groups = C.LAYER_DIM, C.LAYER_HEADS, C.LAYER_HIDDEN, 3
    w = _block_weights(dim, heads, hidden, normalized=True)
    x = W.normal((groups, tokens, dim), 60 + tokens, 1.0)
    block = roformer.Transformer(w, gpu)
    got = block(dev(x, gpu), roformer.axis_rope(w["freqs"], tokens, gpu)).cpu().numpy()
    want = O.transformer_forward(w, x, kernels=True)
    err = float(np.abs(got - want).max())
    print(f"block T={tokens}: max|diff| {err:.3e}", flush=True)
    assert err < 2e-3


@pytest.mark.parametrize("dim,hidden,tokens,normalized", [
    (256, 1024, 1301, True),     # the reference's deux model (configs/deux.json): time pass
    (256, 1024, 60, False),      # its band pass (60 bands), no output norm
    (128, 512, 801, False),      # dim 128 with 8 heads (inner 512 > dim)
    (128, 512, 61, True),
])
def test_block_eight_heads_small_dims(gpu, dim, hidden, tokens, normalized):
    """The fused QKV projection and block tail at dim 256 and dim 128 with 8 heads of 64 (the
    qkv_kernel<16> / <8> and block_tail_kernel<2, 512> / <1, 512> instantiations), against the
    oracle's kernel-path block (roformer.rs:464-520)."""
    heads, groups = 8, 2
    w = _block_weights(dim, heads, hidden, normalized=normalized)
    x = W.normal((groups, tokens, dim), 80 + dim + tokens, 1.0)
    block = roformer.Transformer(w, gpu)
    xd = dev(x, gpu)
    table = roformer.axis_rope(w["freqs"], tokens, gpu)
    got = block(xd, table).cpu().numpy()
    want = O.transformer_forward(w, x, kernels=True, threads=8)
    err = float(np.abs(got - want).max())
    print(f"block dim {dim} x 8 heads, T={tokens}: max|diff| {err:.3e}", flush=True)
    assert err < 2e-3
    assert torch.equal(block(xd, table), block(xd, table))


def test_block_wide_rows(gpu):
    """dim 640 (> 512): the fp16 operand kernel's multi-pass row path."""
    dim, heads, hidden, groups, tokens = 640, 4, 1280, 2, 70
    w = _block_weights(dim, heads, hidden, normalized=True)
    x = W.normal((groups, tokens, dim), 71, 1.0)
    block = roformer.Transformer(w, gpu)
    got = block(dev(x, gpu), roformer.axis_rope(W.rope_freqs(), tokens, gpu)).cpu().numpy()
    want = O.transformer_forward(w, x, kernels=True)
    err = float(np.abs(got - want).max())
    print(f"block dim {dim}: max|diff| {err:.3e}", flush=True)
    assert err < 2e-3


@pytest.mark.parametrize("heads", [3, 1])
@pytest.mark.parametrize("tokens", [60, 130])
def test_block_odd_head_count(gpu, tokens, heads):
    """3 heads (inner 192) and 1 head (inner 64): the attention kernels' one-head items (an odd
    head count cannot be paired) on the block's packed fp16 projection, band (T <= 64) and
    long-sequence lengths. With one head the projection has 7 column blocks: three pairs, and
    an odd block whose row tiles go to waves 0-3, wave 3 holding no pair of its own."""
    dim, hidden, groups = 128, 512, 2
    w = _block_weights(dim, heads, hidden, normalized=True)
    x = W.normal((groups, tokens, dim), 90 + tokens, 1.0)
    block = roformer.Transformer(w, gpu)
    got = block(dev(x, gpu), roformer.axis_rope(W.rope_freqs(), tokens, gpu)).cpu().numpy()
    want = O.transformer_forward(w, x, kernels=True)
    err = float(np.abs(got - want).max())
    print(f"block {heads} heads, T={tokens}: max|diff| {err:.3e}", flush=True)
    assert err < 2e-3
