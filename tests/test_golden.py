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


@pytest.mark.parametrize("name", C.NETWORKS)
def test_network_forward(name):
    """The oracle's network end (band split, axis loop, final norm, mask heads with GLU and the
    overlapping-band average) against the torch float64 restatement of Roformer::forward in
    tests/golden/make_golden.py, with non-zero weights, non-unit gammas and per-layer rotary
    frequencies."""
    import oracle.mel as M
    f = fixture("network.npz")
    config, tensors, spectrum = C.network_case(name)
    np.testing.assert_allclose(C.checksum(spectrum, *(tensors[k] for k in sorted(tensors))),
                               f[f"checksum_{name}"], rtol=1e-12)
    got = M.model_forward(spectrum, config, M.weights_from_tensors(config, tensors), threads=4)
    want = f[name]
    sub = got[:, C.NETWORK_ROWS][..., C.NETWORK_FRAMES]
    close(sub, want, 1e-5 * float(np.abs(want).max()))
    np.testing.assert_allclose(C.moments(got), f[f"moments_{name}"], rtol=1e-4)


def test_network_fixture_rejects_planted_mistakes():
    """Mistakes a restatement of network.rs could plausibly make each move the masks far
    outside the fixture's tolerance: counting Mel mask depth like BS (one hidden layer fewer),
    swapping the GLU halves, and skipping the overlapping-band average."""
    import oracle.mel as M
    f = fixture("network.npz")
    config, tensors, spectrum = C.network_case("mel")
    want = f["mel"]
    scale = float(np.abs(want).max())

    def masks(cfg, weights):
        out = M.model_forward(spectrum, cfg, weights, threads=4)
        return out[:, C.NETWORK_ROWS][..., C.NETWORK_FRAMES]

    weights = M.weights_from_tensors(config, tensors)
    # GLU halves swapped: value <-> gate rows of every band's output projection.
    swapped = dict(weights, masks=[
        {"hidden": h["hidden"],
         "out": [(np.concatenate([w[w.shape[0] // 2:], w[:w.shape[0] // 2]]),
                  np.concatenate([b[b.shape[0] // 2:], b[:b.shape[0] // 2]])) for w, b in h["out"]]}
        for h in weights["masks"]])
    assert np.abs(masks(config, swapped) - want).max() > 1e-2 * scale
    # One hidden layer dropped (the BS count applied to a Mel network).
    shallow = dict(weights, masks=[{"hidden": h["hidden"][:1], "out": h["out"]}
                                   for h in weights["masks"]])
    fewer = dict(config, mask_depth=1)
    assert np.abs(masks(fewer, shallow) - want).max() > 1e-2 * scale
    # Sum instead of average over the covering bands: rows 2*300.. are covered twice.
    got = M.model_forward(spectrum, config, weights, threads=4)
    cover = np.zeros(2050)
    for band in config["bands"]:
        for fb in band:
            cover[2 * fb:2 * fb + 2] += 1
    summed = got * cover[None, :, None, None]
    assert np.abs(summed[:, C.NETWORK_ROWS][..., C.NETWORK_FRAMES] - want).max() > 1e-2 * scale
