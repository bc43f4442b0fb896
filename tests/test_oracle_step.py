"""The decode-step oracle (oracle/decode_step.py): the reference's fused order in float32 from
the pinned parts, against a plain float64 forward of the same model (the reference's own
fused-vs-plain check, tests/test_fused_ops.py:31-40, tolerance 1e-4)."""

from __future__ import annotations

from types import SimpleNamespace

import numpy as np
import pytest

from oracle import decode_step as ods
from oracle import fused_ops as ofo

TINY = SimpleNamespace(vocab_size=512, hidden_size=256, intermediate_size=512,
                       num_hidden_layers=2, num_attention_heads=4, num_key_value_heads=2,
                       head_dim=128, rms_norm_eps=1e-6, rope_theta=1e6, qk_norm=True)
BS = 16


def _batch(seed, ctx):
    rng = np.random.default_rng(seed)
    ctx = np.asarray(ctx, np.int64)
    width = -(-int(ctx.max()) // BS)
    nblk = len(ctx) * width + 3
    perm = rng.permutation(nblk)
    bt = perm[: len(ctx) * width].reshape(len(ctx), width).astype(np.int64)
    ids = rng.integers(0, TINY.vocab_size, len(ctx)).astype(np.int64)
    return ids, ctx, bt, nblk * BS


def _run(cfg, W, ids, ctx, bt, slots, seed, smooth=True):
    caches = ods.random_caches(cfg, slots, seed, smooth)
    c32 = [c.copy() for c in caches]
    c64 = [c.copy() for c in caches]
    cos, sin = ofo.rope_tables(np.arange(int(ctx.max())), cfg.head_dim, cfg.rope_theta)
    logits, nxt, _ = ods.decode_step(W, cfg, ids, ctx, bt, c32, BS, cos, sin)
    ref = ods.decode_step_plain_f64(W, cfg, ids, ctx, bt, c64, BS)
    return caches, c32, c64, logits, nxt, ref


def _rel(a, b):
    return float(np.abs(np.asarray(a, np.float64) - b).max() / np.abs(b).max())


@pytest.mark.parametrize("lm_int4,smooth,awq", [(False, True, True), (True, False, True),
                                                (False, False, False)])
def test_fused_order_matches_plain_f64(lm_int4, smooth, awq):
    W = ods.random_model(TINY, 128, seed=1, lm_int4=lm_int4, awq=awq)
    ids, ctx, bt, slots = _batch(2, [1, 16, 17, 200, 77])
    caches, c32, c64, logits, nxt, ref = _run(TINY, W, ids, ctx, bt, slots, 3, smooth)
    assert _rel(logits, ref) < 1e-4
    top2 = np.sort(ref, -1)[:, -2:]
    clear = top2[:, 1] - top2[:, 0] > 1e-3 * np.abs(ref).max()
    assert np.array_equal(nxt[clear], np.argmax(ref, -1)[clear])
    # this step's K/V rows: written at the token's slot, equal up to a rounding step; every
    # other slot untouched
    tok = ods.token_slots(bt, ctx, BS)
    for a, b, c0 in zip(c32, c64, caches):
        for fa, fb, f0 in ((a.kd, b.kd, c0.kd), (a.vd, b.vd, c0.vd)):
            assert np.abs(fa[tok].astype(int) - fb[tok].astype(int)).max() <= 1
            keep = np.setdiff1d(np.arange(len(f0)), tok)
            assert np.array_equal(fa[keep], f0[keep])
        assert np.allclose(a.ks[tok], b.ks[tok], rtol=1e-5)


def test_step_is_sensitive():
    """The 1e-4 bar separates real mistakes: an off-by-one position, a missing smoothing
    product on q, or a skipped layer each move the logits by far more."""
    W = ods.random_model(TINY, 128, seed=4)
    ids, ctx, bt, slots = _batch(5, [40, 90, 33])
    _, _, _, logits, _, ref = _run(TINY, W, ids, ctx, bt, slots, 6)
    assert _rel(logits, ref) < 1e-4
    cos, sin = ofo.rope_tables(np.arange(200), TINY.head_dim, TINY.rope_theta)
    # position shifted by one (RoPE row and the slot written)
    caches = ods.random_caches(TINY, slots, 6)
    bad, *_ = ods.decode_step(W, TINY, ids, ctx, bt, caches, BS, cos[1:], sin[1:])
    assert _rel(bad, ref) > 1e-2
    # q not multiplied by the smoothing vector
    caches = ods.random_caches(TINY, slots, 6)
    saved = ods.q_mult
    try:
        ods.q_mult = lambda s, n: np.ones((n, s.shape[1]), np.float32)
        bad, *_ = ods.decode_step(W, TINY, ids, ctx, bt, caches, BS, cos, sin)
    finally:
        ods.q_mult = saved
    assert _rel(bad, ref) > 1e-3
    # one layer dropped
    caches = ods.random_caches(TINY, slots, 6)
    W1 = ods.Weights(W.embed, W.norm, W.lm_head, W.layers[1:])
    bad, *_ = ods.decode_step(W1, TINY, ids, ctx, bt, caches[1:], BS, cos, sin)
    assert _rel(bad, ref) > 1e-2


def test_argmax_first():
    lg = np.array([[1, 3, 3, 0], [np.nan, 1, np.nan, 2], [-np.inf] * 4], np.float32)
    assert ods.argmax_first(lg).tolist() == [1, 0, 0]
