"""Pins the oracle (the C restatement of the reference CPU path) before it is trusted.

Each check is independent of the oracle's own code: the reference's known-answer tests
(ancha-kernels/tests/contracts.rs, ancha-models/tests/model_contracts.rs), textbook
definitions computed with torch in float64 (a library routine, used here in the container
only), closed forms and invariants of RoPE, and brute force on tiny inputs.
"""
import math

import numpy as np
import pytest
import torch

import oracle as O
from ancha_amd import workload as W


def values(n, shift):
    """contracts.rs:7-11"""
    return np.array([math.sin((i * 17 + shift) * 0.13) for i in range(n)], dtype=np.float32)


def wave(shape, shift):
    """cuda_contracts.rs:183-189: tanh(1.7 * sin(0.731 i + shift))."""
    n = int(np.prod(shape))
    i = np.arange(n, dtype=np.float32)
    return np.tanh(np.sin(i * np.float32(0.731) + np.float32(shift)) * np.float32(1.7)).astype(
        np.float32).reshape(shape)


def torch_attention(q, k, v, scale):
    """softmax(q k^T * scale) v in float64, [..., T, d]."""
    q, k, v = (torch.as_tensor(np.asarray(a, np.float64)) for a in (q, k, v))
    return (torch.softmax(q @ k.transpose(-1, -2) * scale, dim=-1) @ v).numpy()


# ---- ancha-kernels/tests/contracts.rs --------------------------------------------------------

@pytest.mark.parametrize("nq,nk,d,dv", [(1, 1, 1, 1), (19, 23, 7, 5), (33, 37, 64, 64)])
def test_online_softmax_matches_dense_for_rectangles_and_partial_tiles(nq, nk, d, dv):
    q, k, v = values(2 * nq * d, 1), values(2 * nk * d, 2), values(2 * nk * dv, 3)
    for precision in ("f32", "f64"):
        a = O.attention_dense(q, k, v, 2, nq, nk, d, dv, precision)
        for qt, kt in [(1, 1), (8, 7), (64, 128)]:
            b = O.attention_tiled(q, k, v, 2, nq, nk, d, dv, qt, kt, precision)
            assert np.abs(a - b).max() < 2e-5


def test_attention_rejects_empty_nonfinite_and_zero_tiles():
    one = np.ones(1, np.float32)
    with pytest.raises(O.OracleError, match="tiles must be positive"):
        O.attention_tiled(one, one, one, 1, 1, 1, 1, 1, 0, 1)
    with pytest.raises(O.OracleError, match="non-finite input"):
        O.attention_dense(np.array([np.nan], np.float32), one, one, 1, 1, 1, 1, 1)
    with pytest.raises(O.OracleError, match="all dimensions must be positive"):
        O.attention_dense(one, one, one, 0, 1, 1, 1, 1)


def test_norm_zero_and_small_values_keep_source_epsilon_semantics():
    s, y = O.residual_l2norm([0, 0, 1e-14, 0], [0] * 4, [1, 1], 2, 2, 1e-12)
    assert list(s[:2]) == [0, 0] and list(y[:2]) == [0, 0]
    assert abs(y[2] - 0.01 * math.sqrt(2)) < 1e-6


def test_pack_keeps_gate_bias_and_fold_is_columnwise():
    w, b = O.pack_qkv_gate([1, 2, 3, 4, 5, 6], [7, 8], [0.5], 2)
    assert list(b) == [0, 0, 0, 0.5]
    f = O.fold_norm_scale(w, [2, 3])
    assert abs(f[6] - 7 * 2 * math.sqrt(2)) < 1e-5
    assert abs(f[7] - 8 * 3 * math.sqrt(2)) < 1e-5


# ---- ancha-models/tests/model_contracts.rs ---------------------------------------------------

@pytest.mark.parametrize("n", [1, 19, 35])
def test_tiled_attention_matches_independent_scalar_reference(n):
    groups, heads, dim = 3, 2, 8
    vals = lambda s: np.array([math.sin(i * 0.31 + s) for i in range(groups * heads * n * dim)],
                              np.float32)
    q, k, v = vals(1.0), vals(2.0), vals(3.0)
    expected = O.attention_dense(q, k, v, groups * heads, n, n, dim, dim, "f32")
    # heads-major [G, H, n, d] -> the token-major layout the CPU path takes
    tm = lambda a: a.reshape(groups, heads, n, dim).transpose(0, 2, 1, 3).copy()
    for qt in (1, 7, 128):
        out = O.token_major_attention(tm(q) / np.float32(math.sqrt(dim)), tm(k), tm(v),
                                      query_tile=qt, threads=2)
        got = out.transpose(0, 2, 1, 3).reshape(-1)
        assert np.abs(got - expected).max() < 2e-5


def test_source_norm_has_f_normalize_epsilon_semantics():
    x = np.array([[0, 0], [1e-14, 0], [3, 4]], np.float32)
    scale = np.array([1, 2], np.float32) * np.float32(math.sqrt(2))
    y = O.unit_norm(x, scale, "f32").reshape(-1)
    assert list(y[:2]) == [0, 0]
    assert abs(y[2] - 0.01 * math.sqrt(2)) < 1e-6
    assert abs(y[4] - 3 / 5 * math.sqrt(2)) < 1e-6
    assert abs(y[5] - 4 / 5 * 2 * math.sqrt(2)) < 1e-6


# ---- independent pins: library routines, closed forms, brute force ---------------------------

@pytest.mark.parametrize("g,t,d", [(1, 1, 64), (3, 37, 64), (2, 130, 64), (2, 9, 5)])
def test_dense_matches_torch_float64(g, t, d):
    q, k, v = (W.normal((g, t, d), s, 0.7) for s in (11, 12, 13))
    got = O.attention_dense(q, k, v, g, t, t, d, d, "f64").reshape(g, t, d)
    np.testing.assert_allclose(got, torch_attention(q, k, v, 1 / math.sqrt(d)), atol=1e-13)
    got32 = O.attention_dense(q, k, v, g, t, t, d, d, "f32").reshape(g, t, d)
    np.testing.assert_allclose(got32, got, atol=2e-6)


def test_dense_brute_force_two_keys():
    # Two keys: out = v0 + sigmoid(s1 - s0) (v1 - v0), a closed form independent of softmax code.
    q = np.array([0.3, -1.1], np.float32)
    k = np.array([[0.5, 0.2], [-0.4, 0.9]], np.float32)
    v = np.array([[1.0, 2.0], [-3.0, 0.5]], np.float32)
    s = (k.astype(np.float64) @ q) / math.sqrt(2)
    w = 1 / (1 + math.exp(-(s[1] - s[0])))
    expected = v[0] + w * (v[1] - v[0])
    got = O.attention_dense(q, k, v, 1, 1, 2, 2, 2, "f64")
    np.testing.assert_allclose(got, expected, atol=1e-14)


def test_token_major_threads_and_tiles_do_not_change_results():
    # runtime_contracts.rs: the CPU schedule (host threads, tiles) is arithmetic-invariant.
    q, k, v = (W.normal((5, 67, 3, 64), s, 0.2) for s in (1, 2, 3))
    a = O.token_major_attention(q, k, v, query_tile=None, threads=1)
    b = O.token_major_attention(q, k, v, query_tile=5, threads=3)
    assert np.array_equal(a, b)
    ref = torch_attention(q.transpose(0, 2, 1, 3), k.transpose(0, 2, 1, 3),
                          v.transpose(0, 2, 1, 3), 1.0).transpose(0, 2, 1, 3)
    np.testing.assert_allclose(a, ref, atol=2e-6)


def test_attention_op_equals_textbook_with_rotation():
    g, t, h = 2, 23, 3
    q, k, v = (W.normal((g, t, h, 64), s, 0.5) for s in (1, 2, 3))
    table = O.axis_rope_packed(W.rope_freqs(), t)
    got = O.attention_op(q, k, v, rope=table)
    # Independent rotation: complex multiply by e^{i t f} on channel pairs (2i, 2i+1).
    f = W.rope_freqs().astype(np.float64)
    ang = np.arange(t)[:, None] * f[None, :]
    rot = lambda x: ((x[..., 0::2] + 1j * x[..., 1::2]) *
                     np.exp(1j * ang)[None, :, None, :])
    def back(z):
        out = np.empty(z.shape[:-1] + (64,))
        out[..., 0::2], out[..., 1::2] = z.real, z.imag
        return out
    qr, kr = back(rot(q.astype(np.float64))), back(rot(k.astype(np.float64)))
    ref = torch_attention(qr.transpose(0, 2, 1, 3) / 8, kr.transpose(0, 2, 1, 3),
                          v.transpose(0, 2, 1, 3), 1.0).transpose(0, 2, 1, 3)
    np.testing.assert_allclose(got, ref, atol=1e-6)


def test_rope_table_closed_form_and_relative_position():
    f = W.rope_freqs()
    table = O.axis_rope_packed(f, 50)
    t = np.arange(50)[:, None]
    c, s = np.cos(t * f.astype(np.float64)), np.sin(t * f.astype(np.float64))
    np.testing.assert_allclose(table[2][:, 0::2], c, atol=2e-6)
    np.testing.assert_allclose(table[3][:, 1::2], s, atol=2e-6)
    np.testing.assert_allclose(table[3][:, 0::2], -s, atol=2e-6)
    np.testing.assert_allclose(table[0], table[2] / 8, atol=1e-7)
    # RoPE scores depend on the position difference only: rotate the same q, k at (m, n) and
    # (m + 7, n + 7).
    qv, kv = W.normal((64,), 21), W.normal((64,), 22)
    def rotate(x, row_c, row_s):
        y = np.empty(64)
        y[0::2] = x[0::2] * row_c[0::2] + x[1::2] * row_s[0::2]
        y[1::2] = x[1::2] * row_c[1::2] + x[0::2] * row_s[1::2]
        return y
    score = lambda m, n: rotate(qv, table[2][m], table[3][m]) @ rotate(kv, table[2][n], table[3][n])
    assert abs(score(3, 10) - score(10, 17)) < 1e-4
    assert abs(score(3, 10) - score(3, 11)) > 1e-3
    # Rotation preserves each pair's norm.
    r = rotate(qv, table[2][33], table[3][33])
    np.testing.assert_allclose(r[0::2] ** 2 + r[1::2] ** 2, qv[0::2] ** 2 + qv[1::2] ** 2,
                               rtol=1e-5)


def test_rope_tables_match_packed_layout():
    f = W.rope_freqs()
    cos, sin = O.rope_tables(f, 9, 3, 0.125)
    packed = O.axis_rope_packed(f, 9)
    np.testing.assert_array_equal(cos.reshape(9, 3, 64), np.repeat(packed[0][:, None], 3, 1))
    np.testing.assert_array_equal(sin.reshape(9, 3, 64), np.repeat(packed[1][:, None], 3, 1))
    np.testing.assert_allclose(W.axis_rope_packed(f, 801), O.axis_rope_packed(f, 801),
                               atol=1.2e-7, rtol=0)


def test_linear_epilogue_matches_textbook():
    # cuda_contracts.rs:254-298: bias + GELU + residual, and the rotary epilogue equals
    # RopeTables applied to the q / k column ranges.
    groups, tokens, k, heads = 3, 70, 64, 2
    rows, width = groups * tokens, heads * 64
    m = 3 * width
    x = wave((rows, k), 0.3)
    w = wave((k, m), 1.1) * np.float32(0.1)
    b = wave((m,), 2.2)
    r = wave((rows, m), 3.3)
    y = x.astype(np.float64) @ w + b
    gelu = 0.5 * y * (1 + np.vectorize(math.erf)(y / math.sqrt(2)))
    got = O.linear(x, w, bias=b, gelu=True, residual=r)
    np.testing.assert_allclose(got, gelu + r, atol=1e-12)
    got32 = O.linear(x, w, bias=b, gelu=True, residual=r, precision="f32")
    np.testing.assert_allclose(got32, gelu + r, atol=2e-5)

    freqs = np.array([10000.0 ** (-i / 32) for i in range(32)], np.float32)
    table = O.axis_rope_packed(freqs, tokens)
    got = O.linear(x, w, bias=b, rope=table, tokens=tokens, width=width, precision="f32")
    cq, sq = O.rope_tables(freqs, tokens, heads, 0.125)
    ck, sk = O.rope_tables(freqs, tokens, heads, 1.0)
    yy = (x.astype(np.float64) @ w + b).reshape(groups, tokens, m)
    def apply(z, c, s):
        swapped = z.copy()
        swapped[..., 0::2], swapped[..., 1::2] = z[..., 1::2], z[..., 0::2]
        return z * c.reshape(tokens, -1) + swapped * s.reshape(tokens, -1)
    expected = np.concatenate([apply(yy[..., :width], cq, sq), apply(yy[..., width:2 * width], ck, sk),
                               yy[..., 2 * width:]], axis=2).reshape(rows, m)
    np.testing.assert_allclose(got, expected, atol=2e-5)


def test_gated_attention_is_attention_times_sigmoid_gate():
    g, t, h = 3, 63, 2
    q, k, v = (wave((g, t, h, 64), s) for s in (0.1, 1.3, 2.9))
    q = q * np.float32(0.4 * 0.125)
    gates = wave((g, t, h), 4.4) * np.float32(3.0)
    packed = np.concatenate([q.reshape(g, t, -1), k.reshape(g, t, -1), v.reshape(g, t, -1),
                             gates, np.zeros((g, t, 5), np.float32)], axis=2)
    got = O.gated_attention(packed, h)
    ref = torch_attention(q.transpose(0, 2, 1, 3), k.transpose(0, 2, 1, 3),
                          v.transpose(0, 2, 1, 3), 1.0).transpose(0, 2, 1, 3)
    ref = ref / (1 + np.exp(-gates.astype(np.float64)))[..., None]
    np.testing.assert_allclose(got, ref, atol=1e-12)


def test_folded_linear_layout():
    w = np.arange(12, dtype=np.float32).reshape(4, 3)  # PyTorch [out=4, in=3]
    scale = np.array([1, 2, 3], np.float32)
    wf, bf = O.folded_linear(w, 3, range(1, 3), scale, 0.5, bias=np.array([9, 8, 7, 6], np.float32))
    np.testing.assert_array_equal(wf, (w[1:3] * scale).T * 0.5)
    np.testing.assert_array_equal(bf, [4, 3.5])


def block_weights(dim, heads, hidden, seed=100, normalized=True):
    inner = heads * 64
    shapes = {
        "attn_gamma": (dim,), "to_qkv": (3 * inner, dim), "to_gates": (heads, dim),
        "to_gates_bias": (heads,), "to_out": (dim, inner), "ff_gamma": (dim,),
        "ff_in": (hidden, dim), "ff_in_bias": (hidden,), "ff_out": (dim, hidden),
        "ff_out_bias": (dim,),
    }
    if normalized:
        shapes["output_gamma"] = (dim,)
    w = {"heads": heads, "freqs": W.rope_freqs()}
    for i, (name, shape) in enumerate(sorted(shapes.items())):
        if name.endswith("gamma"):
            w[name] = 1.0 + W.normal(shape, seed + i, 0.1)
        else:
            w[name] = W.normal(shape, seed + i, 0.02)
    return w


@pytest.mark.parametrize("normalized", [True, False])
def test_transformer_kernel_path_matches_burn_path(normalized):
    # cuda_contracts.rs:404-460 / runtime_contracts.rs: the packed-GEMM + gated-attention block
    # equals the separate-projection Burn block.
    w = block_weights(128, 2, 512, normalized=normalized)
    x = W.normal((3, 37, 128), 4)
    a = O.transformer_forward(w, x, kernels=True)
    b = O.transformer_forward(w, x, kernels=False, threads=2)
    np.testing.assert_allclose(a, b, atol=2e-5)
    assert np.isfinite(a).all() and np.abs(a - x).max() > 1e-3
