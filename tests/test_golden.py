"""The oracle against the committed golden fixtures (tests/golden/*.npz).

The fixtures hold float64 results of an independent torch restatement of each op (written in
tests/golden/make_golden.py), rounded to float32, for the reference's own closed-form test
inputs (tests/cuda_contracts.rs:183-295) and single-group slices of the two production shapes.
Inputs are regenerated here and matched against the stored checksums first.
"""
import os

import numpy as np
import pytest

import oracle as O
from tests.golden import cases as C

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def fixture(name):
    return np.load(os.path.join(HERE, name), allow_pickle=False)


def close(got, want, tol):
    err = float(np.abs(np.asarray(got, np.float64) - np.asarray(want, np.float64)).max())
    assert err <= tol, err


@pytest.mark.parametrize("shape", C.ATTENTION_SHAPES)
def test_attention_cases(shape):
    f = fixture("attention_cases.npz")
    q, k, v, gates, packed = C.attention_case(*shape)
    tag = "x".join(map(str, shape))
    np.testing.assert_allclose(C.checksum(q, k, v, packed), f[f"checksum_{tag}"], rtol=1e-12)
    if f"attention_{tag}" in f:
        close(O.attention_op(q, k, v), f[f"attention_{tag}"], 2e-7)
        close(O.attention_op(q, k, v, precision="f32"), f[f"attention_{tag}"], 2e-6)
    close(O.gated_attention(packed, shape[2]), f[f"gated_{tag}"], 2e-7)
    close(O.gated_attention(packed, shape[2], precision="f32"), f[f"gated_{tag}"], 2e-6)


def test_linear_epilogues():
    f = fixture("linear_epilogue.npz")
    x, w, b, r, table, _ = C.linear_case()
    np.testing.assert_allclose(C.checksum(x, w, b, r), f["checksum"], rtol=1e-12)
    for precision, tol in (("f64", 1e-6), ("f32", 1e-5)):
        got = O.linear(x, w, bias=b, gelu=True, residual=r, precision=precision)
        close(got[C.LINEAR_GELU_ROWS], f["gelu_rows"], tol)
        got = O.linear(x, w, bias=b, rope=table, tokens=C.LINEAR_TOKENS, width=C.LINEAR_WIDTH,
                       precision=precision)
        close(got[C.LINEAR_ROTARY_ROWS], f["rotary_rows"], tol)


@pytest.mark.parametrize("name", sorted(C.SLICES))
def test_production_slices(name):
    f = fixture("production_slices.npz")
    shape, rows, heads = C.SLICES[name]
    q, k, v, table, _ = C.slice_case(shape)
    np.testing.assert_allclose(C.checksum(q, k, v), f[f"checksum_{name}"], rtol=1e-12)
    close(O.attention_op(q, k, v, rope=table)[0][np.ix_(rows, heads)], f[name], 2e-7)
    got = O.attention_op(q, k, v, rope=table, precision="f32")
    close(got[0][np.ix_(rows, heads)], f[name], 2e-6)


@pytest.mark.parametrize("kernels", [True, False])
def test_layer(kernels):
    f = fixture("layer.npz")
    w, x = C.layer_case()
    np.testing.assert_allclose(
        C.checksum(x, *(w[n] for n in sorted(w) if n not in ("heads", "freqs"))), f["checksum"],
        rtol=1e-12)
    close(O.transformer_forward(w, x, kernels=kernels), f["out"], 5e-5)


def test_fixtures_reject_a_planted_mistake():
    # A dropped sign in the rotation (sin instead of signed sin) must fail the slice fixture.
    f = fixture("production_slices.npz")
    shape, rows, heads = C.SLICES["band"]
    q, k, v, table, _ = C.slice_case(shape)
    bad = table.copy()
    bad[1] = np.abs(bad[1])
    bad[3] = np.abs(bad[3])
    err = np.abs(O.attention_op(q, k, v, rope=bad)[0][np.ix_(rows, heads)] - f["band"]).max()
    assert err > 1e-4
