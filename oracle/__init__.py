"""The oracle: a C restatement of Ancha's reference CPU path for the fused RoFormer
attention ops. TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline leg import this
package, and only as the checker (or the timed CPU baseline). The product path in
``ancha_amd`` never imports it.

Each wrapper takes and returns numpy arrays; ``precision`` selects the fp32 restatement
("f32", the reference's operation order) or the fp64 run of the same steps ("f64").
Errors raise :class:`OracleError` with the reference's error string.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "_build", "libancha_oracle.so")

ERRORS = {
    -1: "all dimensions must be positive",
    -3: "non-finite input",
    -4: "score overflow",
    -5: "output overflow",
    -6: "tiles must be positive",
    -7: "invalid shape",
    -8: "norm overflow",
}


class OracleError(RuntimeError):
    pass


def build() -> str:
    """Compile the oracle library with its Makefile (gcc only)."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    return LIB_PATH


_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        _lib = ctypes.CDLL(LIB_PATH)
        _declare(_lib)
    return _lib


_sz = ctypes.c_size_t
_p = ctypes.c_void_p


def _declare(l: ctypes.CDLL) -> None:
    l.anc_fill_normal.argtypes = [_p, _sz, ctypes.c_uint64, ctypes.c_double, _sz]
    l.anc_axis_rope_packed.argtypes = [_p, _sz, _sz, _p]
    l.anc_rope_tables.argtypes = [_p, _sz, _sz, _sz, ctypes.c_float, _p, _p]
    for s in ("f32", "f64"):
        getattr(l, f"anc_attention_dense_{s}").argtypes = [_p, _p, _p] + [_sz] * 5 + [_p]
        getattr(l, f"anc_attention_tiled_{s}").argtypes = [_p, _p, _p] + [_sz] * 7 + [_p]
        getattr(l, f"anc_token_major_attention_{s}").argtypes = [_p, _p, _p] + [_sz] * 10 + [_p]
        getattr(l, f"anc_attention_op_{s}").argtypes = [_p, _p, _p] + [_sz] * 6 + [_p, _p]
        getattr(l, f"anc_gated_attention_{s}").argtypes = [_p] + [_sz] * 4 + [_p, _p]
        getattr(l, f"anc_unit_norm_{s}").argtypes = [_p, _sz, _sz, _p, _p]
        getattr(l, f"anc_unit_norm_{s}").restype = None
        getattr(l, f"anc_linear_{s}").argtypes = (
            [_p, _sz, _sz, _sz, _p, _sz, _p, ctypes.c_int, _p, _sz, _sz, _p, _p])
        getattr(l, f"anc_linear_{s}").restype = None
    l.anc_residual_l2norm.argtypes = [_p, _p, _p, _sz, _sz, ctypes.c_float, _p, _p]
    l.anc_pack_qkv_gate.argtypes = [_p, _sz, _p, _sz, _p, _sz, _sz, _p, _p]
    l.anc_fold_norm_scale.argtypes = [_p, _sz, _p, _sz, _p]
    l.anc_folded_linear.argtypes = [_p, _sz, _sz, _sz, _p, ctypes.c_float, _p, _p, _p]
    l.anc_folded_linear.restype = None
    l.anc_transformer_forward.argtypes = [_p, _p, _sz, _sz, ctypes.c_int, _sz, _p]


def _dtype(precision: str):
    if precision not in ("f32", "f64"):
        raise ValueError(precision)
    return np.float32 if precision == "f32" else np.float64


def _arr(x, dtype) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(x, dtype=dtype))


def _ptr(a) -> int | None:
    return None if a is None else a.ctypes.data


def _check(rc: int) -> None:
    if rc:
        raise OracleError(ERRORS.get(rc, f"error {rc}"))


# ---- seeded inputs -------------------------------------------------------------------------

def normal(shape, seed: int, scale: float = 1.0, first: int = 0) -> np.ndarray:
    """splitmix64 -> Box-Muller N(0, scale^2) stream, elements [first, first + size)."""
    n = int(np.prod(shape))
    out = np.empty(n, dtype=np.float32)
    lib().anc_fill_normal(out.ctypes.data, n, seed, scale, first)
    return out.reshape(shape)


# ---- rotary tables -------------------------------------------------------------------------

def axis_rope_packed(freqs, tokens: int) -> np.ndarray:
    """[4, tokens, 2*len(freqs)] packed table (roformer.rs:282-302)."""
    f = _arr(freqs, np.float32)
    out = np.empty((4, tokens, 2 * f.size), dtype=np.float32)
    lib().anc_axis_rope_packed(f.ctypes.data, f.size, tokens, out.ctypes.data)
    return out


def rope_tables(freqs, tokens: int, heads: int, scale: float):
    """RopeTables::new (roformer.rs:156-175): cos, signed sin, each [tokens * heads * 2nf]."""
    f = _arr(freqs, np.float32)
    width = heads * 2 * f.size
    cos = np.empty(tokens * width, dtype=np.float32)
    sin = np.empty(tokens * width, dtype=np.float32)
    lib().anc_rope_tables(f.ctypes.data, f.size, tokens, heads, scale, cos.ctypes.data,
                          sin.ctypes.data)
    return cos, sin


# ---- attention -----------------------------------------------------------------------------

def attention_dense(q, k, v, groups, queries, keys, head_dim, value_dim, precision="f64"):
    dt = _dtype(precision)
    q, k, v = _arr(q, dt), _arr(k, dt), _arr(v, dt)
    out = np.zeros(max(groups * queries * value_dim, 1), dtype=dt)
    _check(getattr(lib(), f"anc_attention_dense_{precision}")(
        q.ctypes.data, k.ctypes.data, v.ctypes.data, groups, queries, keys, head_dim, value_dim,
        out.ctypes.data))
    return out


def attention_tiled(q, k, v, groups, queries, keys, head_dim, value_dim, query_tile, key_tile,
                    precision="f64"):
    dt = _dtype(precision)
    q, k, v = _arr(q, dt), _arr(k, dt), _arr(v, dt)
    out = np.zeros(max(groups * queries * value_dim, 1), dtype=dt)
    _check(getattr(lib(), f"anc_attention_tiled_{precision}")(
        q.ctypes.data, k.ctypes.data, v.ctypes.data, groups, queries, keys, head_dim, value_dim,
        query_tile, key_tile, out.ctypes.data))
    return out


def token_major_attention(q, k, v, query_tile=None, threads=1, precision="f32"):
    """Prescaled attention over [G, T, H, d] inputs, the Flex CPU path (roformer.rs:324-363)."""
    dt = _dtype(precision)
    q, k, v = _arr(q, dt), _arr(k, dt), _arr(v, dt)
    g, t, h, d = q.shape
    out = np.empty_like(q)
    _check(getattr(lib(), f"anc_token_major_attention_{precision}")(
        q.ctypes.data, k.ctypes.data, v.ctypes.data, g, t, h, d, h * d, h * d, h * d, g,
        query_tile or t, threads, out.ctypes.data))
    return out


def attention_op(q, k, v, rope=None, precision="f64"):
    """The fused::attention contract: q pre-scaled, [G, T, H, 64] in and out; ``rope`` is the
    optional packed [4, T, 64] table applied to q and k first."""
    dt = _dtype(precision)
    q, k, v = _arr(q, dt), _arr(k, dt), _arr(v, dt)
    g, t, h, d = q.shape
    assert d == 64
    table = None if rope is None else _arr(rope, np.float32)
    out = np.empty_like(q)
    _check(getattr(lib(), f"anc_attention_op_{precision}")(
        q.ctypes.data, k.ctypes.data, v.ctypes.data, g, t, h, h * d, h * d, h * d,
        _ptr(table), out.ctypes.data))
    return out


def gated_attention(packed, heads, rope=None, precision="f64"):
    """fused::gated_attention on packed [G, T, C] -> [G, T, H, 64]."""
    dt = _dtype(precision)
    p = _arr(packed, dt)
    g, t, c = p.shape
    table = None if rope is None else _arr(rope, np.float32)
    out = np.empty((g, t, heads, 64), dtype=dt)
    _check(getattr(lib(), f"anc_gated_attention_{precision}")(
        p.ctypes.data, g, t, c, heads, _ptr(table), out.ctypes.data))
    return out


# ---- norm / projections --------------------------------------------------------------------

def unit_norm(x, scale=None, precision="f64"):
    dt = _dtype(precision)
    x = _arr(x, dt)
    dim = x.shape[-1]
    rows = x.size // dim
    s = None if scale is None else _arr(scale, dt)
    out = np.empty_like(x)
    getattr(lib(), f"anc_unit_norm_{precision}")(x.ctypes.data, rows, dim, _ptr(s),
                                                 out.ctypes.data)
    return out


def linear(x, w, bias=None, gelu=False, rope=None, tokens=1, width=0, residual=None,
           precision="f64"):
    """fused::linear: x [n, k] . w [k, m] with the bias/GELU/rotary/residual epilogue."""
    dt = _dtype(precision)
    x, w = _arr(x, dt), _arr(w, dt)
    n, k = x.shape
    m = w.shape[1]
    b = None if bias is None else _arr(bias, dt)
    r = None if residual is None else _arr(residual, dt)
    table = None if rope is None else _arr(rope, np.float32)
    out = np.empty((n, m), dtype=dt)
    getattr(lib(), f"anc_linear_{precision}")(
        x.ctypes.data, n, k, k, w.ctypes.data, m, _ptr(b), int(gelu), _ptr(table), tokens, width,
        _ptr(r), out.ctypes.data)
    return out


def residual_l2norm(x, residual, gamma, rows, dim, eps):
    x, r, g = (_arr(a, np.float32) for a in (x, residual, gamma))
    s = np.zeros(max(rows * dim, 1), np.float32)
    n = np.zeros(max(rows * dim, 1), np.float32)
    _check(lib().anc_residual_l2norm(x.ctypes.data, r.ctypes.data, g.ctypes.data, rows, dim,
                                     eps, s.ctypes.data, n.ctypes.data))
    return s, n


def pack_qkv_gate(qkv, gate, gate_bias, dim):
    qkv, gate, gb = (_arr(a, np.float32) for a in (qkv, gate, gate_bias))
    w = np.zeros(qkv.size + gate.size, np.float32)
    b = np.zeros(qkv.size // dim + gb.size, np.float32)
    _check(lib().anc_pack_qkv_gate(qkv.ctypes.data, qkv.size, gate.ctypes.data, gate.size,
                                   gb.ctypes.data, gb.size, dim, w.ctypes.data, b.ctypes.data))
    return w, b


def fold_norm_scale(weights, gamma):
    w, g = _arr(weights, np.float32), _arr(gamma, np.float32)
    out = np.zeros_like(w)
    _check(lib().anc_fold_norm_scale(w.ctypes.data, w.size, g.ctypes.data, g.size,
                                     out.ctypes.data))
    return out


def folded_linear(weight, input_dim, rows, input_scale, output_scale=1.0, bias=None):
    """weights.rs:149-176 -> (W' [input, len(rows)], b' or None)."""
    w, s = _arr(weight, np.float32), _arr(input_scale, np.float32)
    r0, r1 = rows.start, rows.stop
    wo = np.empty((input_dim, r1 - r0), np.float32)
    b = None if bias is None else _arr(bias, np.float32)
    bo = None if bias is None else np.empty(r1 - r0, np.float32)
    lib().anc_folded_linear(w.ctypes.data, input_dim, r0, r1, s.ctypes.data, output_scale,
                            _ptr(b), wo.ctypes.data, _ptr(bo))
    return wo, bo


class _BlockWeights(ctypes.Structure):
    _fields_ = [("dim", _sz), ("heads", _sz), ("head_dim", _sz), ("hidden", _sz)] + [
        (name, _p) for name in (
            "attn_gamma", "to_qkv", "to_gates", "to_gates_bias", "to_out", "freqs", "ff_gamma",
            "ff_in", "ff_in_bias", "ff_out", "ff_out_bias", "output_gamma")]


def transformer_forward(weights: dict, x, kernels=True, threads=1):
    """One RoFormer block on x [groups, tokens, dim]; ``weights`` holds the PyTorch-layout
    tensors under the names of :class:`_BlockWeights` (output_gamma optional)."""
    x = _arr(x, np.float32)
    groups, tokens, dim = x.shape
    keep = {k: _arr(v, np.float32) for k, v in weights.items()
            if v is not None and k != "heads"}
    bw = _BlockWeights(dim=dim, heads=int(weights["heads"]), head_dim=64,
                       hidden=keep["ff_in"].shape[0])
    for name, _ in _BlockWeights._fields_[4:]:
        setattr(bw, name, keep[name].ctypes.data if name in keep else None)
    out = np.empty_like(x)
    _check(lib().anc_transformer_forward(ctypes.byref(bw), x.ctypes.data, groups, tokens,
                                         int(kernels), threads, out.ctypes.data))
    return out
