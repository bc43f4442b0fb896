"""One greedy decode step of the quantized model (llmserve.transformer + llmserve.model_runner)
against the decode-step oracle (oracle/decode_step.py), and graph replays against eager steps.

Tolerances: logits max-abs <= 2e-5 x max|logits|, float32 through two layers in different
reduction orders, with the GEMV linears (<= 4 rows) and with the matrix-core linears above
(x split into bf16 hi + mid + lo, exact to ~2^-26 per element, exact products); the oracle
reads the K/V rows the HIP step wrote, so a
one-step rounding difference of a quantized value cannot enter. This step's int8 K/V rows are
within one quantization step of the oracle's (under 1% of them off by one), their scales within
the same relative tolerance, at the oracle's slots; every other slot is unchanged;
greedy ids equal wherever the top two logits are apart by more than the tolerance. Graph
replays are bit-identical to eager steps.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import decode_step as ods

pytestmark = pytest.mark.gpu
BS = 16


def tol(rows: int) -> float:
    return 2e-5  # the GEMV up to 4 rows and the matrix-core kernel above: fp32 arithmetic


def tiny_cfg(vocab=512):
    from llmserve.transformer import ModelConfig

    return ModelConfig(vocab_size=vocab, hidden_size=256, intermediate_size=512,
                       num_hidden_layers=2, num_attention_heads=4, num_key_value_heads=2,
                       head_dim=128, max_position_embeddings=1024)


def _np(t):
    return None if t is None else t.detach().cpu().numpy()


def oracle_weights(m) -> ods.Weights:
    def w4(lin):
        return ods.Int4W(_np(lin.nibbles), _np(lin.g_scale), _np(lin.g_zero),
                         _np(lin.inv_act_scale), lin.group_size)

    layers = [ods.Layer(_np(L.input_layernorm), _np(L.post_attention_layernorm), _np(L.q_norm),
                        _np(L.k_norm), w4(L.qkv_proj), w4(L.o_proj), w4(L.gate_up_proj),
                        w4(L.down_proj)) for L in m.layers]
    lm = w4(m.lm_head) if m.lm_head is not None else _np(m.lm_weight)
    return ods.Weights(_np(m.embed), _np(m.norm), lm, layers)


def setup(cfg, ctx, seed, lm_int4=False, smooth=True, extra=4):
    from llmserve.kv_cache import KVCache
    from llmserve.model_runner import DecodeRunner
    from llmserve.transformer import QuantCausalLM

    rng = np.random.default_rng(seed)
    ctx = np.asarray(ctx, np.int64)
    width = -(-(int(ctx.max()) + extra) // BS)
    nblk = len(ctx) * width + 5
    bt = rng.permutation(nblk)[: len(ctx) * width].reshape(len(ctx), width).astype(np.int64)
    ids = rng.integers(0, cfg.vocab_size, len(ctx)).astype(np.int64)
    model = QuantCausalLM(cfg, 128, quantize_lm_head=lm_int4, seed=seed)
    cache = KVCache(cfg, nblk, BS, device="cuda", kv_dtype="int8")
    host = ods.random_caches(cfg, nblk * BS, seed + 1, smooth)
    for (k, v), c in zip(cache.layers, host):
        k.data.copy_(torch.from_numpy(c.kd))
        k.scale.copy_(torch.from_numpy(c.ks))
        v.data.copy_(torch.from_numpy(c.vd))
        v.scale.copy_(torch.from_numpy(c.vs))
        if smooth:
            k.set_smoothing(torch.from_numpy(c.smooth), cfg.num_attention_heads)
    runner = DecodeRunner(model, cache, torch.from_numpy(ids), torch.from_numpy(ctx),
                          torch.from_numpy(bt))
    return model, cache, runner, host, ids, ctx, bt


def _rel(a, b):
    return float(np.abs(np.asarray(a, np.float64) - b).max() / np.abs(b).max())


def check_step(cfg, model, cache, runner, host, ids, ctx, bt):
    runner.step()
    got = _np(runner.logits)
    nxt = _np(runner.ids)
    assert np.array_equal(_np(runner.context_lens), ctx + 1)
    tok = ods.token_slots(bt, ctx, BS)
    after = [ods.LayerCache(_np(k.data), _np(k.scale), _np(v.data), _np(v.scale),
                            c.smooth) for (k, v), c in zip(cache.layers, host)]
    W = oracle_weights(model)
    cos, sin = _np(model.rope_cos), _np(model.rope_sin)
    logits, want_ids, rows = ods.decode_step(W, cfg, ids, ctx, bt, [c.copy() for c in after], BS,
                                             cos, sin, write_kv=False)
    assert _rel(got, logits) < tol(len(ids))
    top2 = np.sort(logits, -1)[:, -2:]
    clear = top2[:, 1] - top2[:, 0] > 10 * tol(len(ids)) * np.abs(logits).max()
    assert clear.sum() >= len(ids) // 2
    assert np.array_equal(nxt[clear], want_ids[clear])
    keep = np.setdiff1d(np.arange(host[0].kd.shape[0]), tok)
    for a, c0, (kq, ks, vq, vs) in zip(after, host, rows):
        for d, dq in ((a.kd, kq), (a.vd, vq)):
            diff = np.abs(d[tok].astype(np.int32) - dq.astype(np.int32))
            assert diff.max() <= 1 and (diff > 0).mean() < 0.01
        r = tol(len(ids))  # the scales carry the relative error of the qkv rows
        assert np.allclose(a.ks[tok], ks, rtol=r) and np.allclose(a.vs[tok], vs, rtol=r)
        assert np.array_equal(a.kd[keep], c0.kd[keep]) and np.array_equal(a.vd[keep], c0.vd[keep])
        assert np.array_equal(a.ks[keep], c0.ks[keep]) and np.array_equal(a.vs[keep], c0.vs[keep])


@pytest.mark.parametrize("ctx,lm_int4,smooth", [
    ([1, 16, 17, 300, 77], False, True),     # 5 rows: the matrix-core linears
    ([1, 16, 17, 300], True, False),         # 4 rows: the GEMV linears, int4 LM head
    ([9, 300], False, True),                 # 2 rows: the decode chain
    ([700], True, True),                     # 1 row: the decode chain
    (list(range(20, 500, 20)), False, True),  # 24 rows: the matrix-core linears
    (list(range(20, 500, 20)), True, True),
])
def test_step_matches_oracle(gpu, ctx, lm_int4, smooth):
    cfg = tiny_cfg()
    model, cache, runner, host, ids, ctx, bt = setup(cfg, ctx, 11, lm_int4, smooth)
    check_step(cfg, model, cache, runner, host, ids, ctx, bt)


def test_graph_replays_equal_eager_steps(gpu):
    cfg = tiny_cfg()
    _, cache, runner, _, _, _, _ = setup(cfg, list(range(30, 30 + 24 * 9, 9)), 21, extra=8)
    start = runner.snapshot()
    eager = []
    for _ in range(3):
        runner.step()
        eager.append((runner.ids.clone(), runner.logits.clone(), runner.context_lens.clone()))
    eager_cache = runner.snapshot()[2]
    runner.restore(start)
    runner.capture(keep_state=True)
    for i in range(3):
        runner.replay()
        torch.cuda.synchronize()
        _ = torch.randn(1000, device="cuda").sum().item()  # unrelated eager work between replays
        ids, logits, ctx = eager[i]
        assert torch.equal(runner.ids, ids)
        assert torch.equal(runner.logits, logits)
        assert torch.equal(runner.context_lens, ctx)
    for (k, v), (kd, ks, vd, vs) in zip(cache.layers, eager_cache):
        assert torch.equal(k.data, kd) and torch.equal(k.scale, ks)
        assert torch.equal(v.data, vd) and torch.equal(v.scale, vs)


@pytest.mark.parametrize("lm_int4", [False, True])
def test_fragment_path_equals_plain_path(gpu, lm_int4):
    """Above 16 rows the step fuses each linear's x * inv_act_scale and bf16 split into the
    producing norm / silu kernel; the logits, tokens and caches equal the unfused step's bit
    for bit."""
    cfg = tiny_cfg()
    ctx = list(range(20, 500, 20))
    model, cache, runner, host, ids, ctx, bt = setup(cfg, ctx, 31, lm_int4)
    start = runner.snapshot()
    assert model._xfrag_ok(len(ids))
    model.fp32_head_kernel = False  # both runs take torch.mm for the fp32 head
    runner.step()
    fused = (runner.logits.clone(), runner.ids.clone(), runner.snapshot()[2])
    runner.restore(start)
    model.fuse_xfrag = False
    runner.step()
    assert torch.equal(runner.logits, fused[0]) and torch.equal(runner.ids, fused[1])
    for a, b in zip(runner.snapshot()[2], fused[2]):
        for u, v in zip(a, b):
            assert torch.equal(u, v)


def test_embed_rmsnorm(gpu):
    from llmserve.kernels import load_fused_ops
    from oracle import fused_ops as ofo

    rng = np.random.default_rng(0)
    V, H = 300, 1024
    emb = rng.standard_normal((V, H)).astype(np.float32)
    w = rng.standard_normal(H).astype(np.float32)
    ids = np.array([0, 299, 17, 17, 300, -1], np.int64)
    x, h = load_fused_ops().embed_rmsnorm(torch.from_numpy(ids).cuda(), torch.from_numpy(emb).cuda(),
                                          torch.from_numpy(w).cuda(), 1e-6)
    x, h = _np(x), _np(h)
    assert np.array_equal(x[:4], emb[ids[:4]])
    ref = ofo.rmsnorm_f64(emb[ids[:4]], w, 1e-6)
    assert np.abs(h[:4] - ref).max() <= 2e-6 * np.abs(ref).max()
    assert np.isnan(x[4:]).all() and np.isnan(h[4:]).all()  # ids outside [0, V)
