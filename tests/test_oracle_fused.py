"""The fused-ops oracle (oracle/fused_ops.py) against the reference's compiled fused_ops.cpp
(committed golden vectors), the float64 mathematics and closed forms."""

from __future__ import annotations

import numpy as np
import pytest

from conftest import GOLDEN
from oracle import fused_ops as ofo

F32 = np.float32


@pytest.fixture(scope="module")
def fg():
    return dict(np.load(GOLDEN / "fused_golden.npz"))


def _rel(a, b):
    return float(np.abs(np.asarray(a, np.float64) - b).max() / max(np.abs(b).max(), 1e-30))


@pytest.mark.parametrize("T,H", [(3, 1024), (2, 200), (1, 2048)])
def test_norms_match_reference(fg, T, H):
    k = f"norm_T{T}_H{H}"
    x, r, w = fg[k + "_x"], fg[k + "_r"], fg[k + "_w"]
    assert _rel(ofo.rmsnorm(x, w, 1e-6), fg[k + "_out"]) < 2e-6
    assert _rel(ofo.rmsnorm(x, w, 1e-6), ofo.rmsnorm_f64(x, w, 1e-6)) < 2e-6
    xa, o = ofo.add_rmsnorm(x, r, w, 1e-6)
    assert np.array_equal(xa, fg[k + "_xadd"])  # a single fp32 add: bit-exact
    assert _rel(o, fg[k + "_outadd"]) < 2e-6


@pytest.mark.parametrize("T,I", [(2, 300), (4, 3072)])
def test_silu_mul_matches_reference(fg, T, I):
    gu = fg[f"silu_T{T}_I{I}_gu"]
    assert _rel(ofo.silu_mul(gu), fg[f"silu_T{T}_I{I}_out"]) < 2e-6
    assert _rel(ofo.silu_mul(gu), ofo.silu_mul_f64(gu)) < 2e-6


@pytest.mark.parametrize("name", ["rope_d128", "rope_d64"])
def test_rope_matches_reference(fg, name):
    nq, nk, D, norms = (int(v) for v in fg[f"{name}_meta"])
    qw = fg.get(f"{name}_qw") if norms else None
    kw = fg.get(f"{name}_kw") if norms else None
    args = (fg[f"{name}_qkv"], fg[f"{name}_cos"], fg[f"{name}_sin"], nq, nk, D, qw, kw, 1e-6)
    out = ofo.rope_qk(*args)
    assert _rel(out, fg[f"{name}_out"]) < 2e-6
    assert _rel(out, ofo.rope_qk_f64(*args)) < 2e-6
    # the v heads are untouched
    assert np.array_equal(out[:, (nq + nk) * D:], fg[f"{name}_qkv"][:, (nq + nk) * D:])


def test_closed_forms():
    # a constant row normalizes to sign * w (mean(x^2) = c^2)
    w = np.linspace(0.5, 1.5, 64).astype(F32)
    for c in (3.0, -0.25):
        y = ofo.rmsnorm(np.full((1, 64), c, F32), w, 0.0)
        assert np.allclose(y, np.sign(c) * w, rtol=1e-6)
    # RoPE at position 0 is the identity; it preserves each pair's norm
    D = 128
    rng = np.random.default_rng(0)
    qkv = rng.standard_normal((2, 3 * D)).astype(F32)
    c0, s0 = ofo.rope_tables(np.array([0, 0]), D, 1e6)
    assert np.array_equal(ofo.rope_qk(qkv, c0, s0, 1, 1, D), qkv)
    c, s = ofo.rope_tables(np.array([5, 1000]), D, 1e6)
    out = ofo.rope_qk(qkv, c, s, 1, 1, D)
    for h in range(2):
        a, b = qkv[:, h * D:(h + 1) * D], out[:, h * D:(h + 1) * D]
        na = a[:, :D // 2] ** 2 + a[:, D // 2:] ** 2
        nb = b[:, :D // 2] ** 2 + b[:, D // 2:] ** 2
        assert np.allclose(na, nb, rtol=1e-5)
    # silu(0) * u = 0; silu(g) ~ g for large g
    gu = np.array([[0.0, 30.0, 2.0, 3.0]], F32)
    y = ofo.silu_mul(gu)
    assert y[0, 0] == 0.0 and abs(y[0, 1] - 30.0 * 3.0) < 1e-4
