"""ModelRunner.execute on ragged batches, and key-smoothing calibration on this package's model.

* A mixed step (prompt chunks with and without a cached prefix, decode tokens) runs the
  ragged forward (QuantCausalLM.forward, the reference's _forward_fused order) with the native
  attention backend (device metadata + one row launch per layer); the same step with the torch
  backend (the reference's gather + SDPA) gives logits within 1e-4 (the reference's
  fused-vs-plain bar, tests/test_fused_ops.py:40) where both runs attend over identical cache
  rows (one layer, or an fp32 cache), 2e-3 with two layers over an int8 cache (see
  logit_tol), and the same cache contents up to one int8 step in under 1% of the values.
* A decode-only step takes the fused decode step; it equals the ragged forward's logits
  to the same tolerances and writes the same K/V rows.
* calibrate_k_smoothing runs on QuantCausalLM: factors have mean 1 per head, layer 0's equal
  max|K|^alpha / mean computed from the layer-0 keys directly (bit for bit), alpha = 0 gives
  ones, and the native and torch attention backends agree.
"""

from __future__ import annotations

from types import SimpleNamespace

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu
BS = 16


def tiny_cfg(layers=2):
    from llmserve.transformer import ModelConfig

    return ModelConfig(vocab_size=512, hidden_size=256, intermediate_size=512,
                       num_hidden_layers=layers, num_attention_heads=4, num_key_value_heads=2,
                       head_dim=128, max_position_embeddings=2048)


# Logit tolerances. With one layer (or an fp32 cache) both runs attend over bit-identical
# cache rows and differ only by the attention kernels' float32 rounding: 1e-4, the
# reference's fused-vs-plain bar. With an int8 cache and two layers, layer 1's new K/V rows
# are quantized from activations that differ by ~1e-6, so a value near a rounding boundary can
# land one int8 step apart (checked below: under 1% of values), and one such step moves a short
# prompt's attention weights by up to a few 1e-3: 2e-3.
def logit_tol(layers, kv_dtype):
    return 1e-4 if layers == 1 or kv_dtype == "auto" else 2e-3


class _Seq:
    def __init__(self, toks, computed, table):
        self._toks, self.num_computed_tokens, self.block_table = toks, computed, table

    def token_ids(self):
        return self._toks


def _sched(seqs, news):
    return SimpleNamespace(scheduled=[SimpleNamespace(seq=s, num_new_tokens=n)
                                      for s, n in zip(seqs, news)], block_copies=[])


def _setup(seed, backend, ctx_lens, kv_dtype="int8", layers=2):
    from llmserve.kv_cache import KVCache
    from llmserve.model_runner import ModelRunner
    from llmserve.transformer import QuantCausalLM

    cfg = tiny_cfg(layers)
    rng = np.random.default_rng(seed)
    model = QuantCausalLM(cfg, 128, seed=seed)
    need = [-(-c // BS) for c in ctx_lens]
    total = sum(need) + 4
    cache = KVCache(cfg, total, BS, device="cuda", kv_dtype=kv_dtype)
    g = torch.Generator(device="cuda").manual_seed(seed)
    for k, v in cache.layers:
        if kv_dtype == "int8":
            for t in (k, v):
                t.data.random_(-127, 128, generator=g)
                t.scale.uniform_(0.005, 0.05, generator=g)
            s = torch.rand(cfg.num_key_value_heads, cfg.head_dim, device="cuda", generator=g) + 0.5
            k.set_smoothing(s / s.mean(-1, keepdim=True), cfg.num_attention_heads)
        else:
            k.normal_(generator=g)
            v.normal_(generator=g)
    perm = rng.permutation(total).tolist()
    tables, used = [], 0
    for n in need:
        tables.append(perm[used:used + n])
        used += n
    return cfg, model, cache, ModelRunner(model, cache, backend), tables, rng


def _int8_close(a, b):
    d = (a.data.to(torch.int32) - b.data.to(torch.int32)).abs()
    return int(d.max()) <= 1 and float((d > 0).float().mean()) < 0.01


@pytest.mark.parametrize("kv_dtype,layers", [("int8", 1), ("int8", 2), ("auto", 2)])
def test_mixed_batch_native_vs_torch(gpu, kv_dtype, layers):
    ctx = [40, 70, 301, 17, 5]
    new = [40, 30, 1, 1, 5]  # fresh prompt, chunk after 40 cached, decodes, fresh prompt
    logits, caches = [], []
    for backend in ("hip", "torch"):
        cfg, model, cache, runner, tables, rng = _setup(7, backend, ctx, kv_dtype, layers)
        seqs = [_Seq(rng.integers(0, cfg.vocab_size, c).tolist(), c - n, t)
                for c, n, t in zip(ctx, new, tables)]
        out = runner.execute(_sched(seqs, new), [0, 1, 2, 3, 4], {1: 3})
        assert out.shape == (7, cfg.vocab_size) and out.device.type == "cpu"
        logits.append(out)
        caches.append(cache)
    ref = logits[1].double()
    err = float((logits[0].double() - ref).abs().max() / ref.abs().max())
    assert err < logit_tol(layers, kv_dtype), err
    for (k0, v0), (k1, v1) in zip(caches[0].layers, caches[1].layers):
        if kv_dtype == "int8":
            assert _int8_close(k0, k1) and _int8_close(v0, v1)
        else:
            for a, b in ((k0, k1), (v0, v1)):
                assert float((a - b).abs().max()) <= 1e-4 * float(b.abs().max())


@pytest.mark.parametrize("layers", [1, 2])
def test_decode_step_equals_ragged_forward(gpu, layers):
    ctx = [33, 1, 300, 129, 64, 17]
    runs = []
    for fused in (True, False):
        cfg, model, cache, runner, tables, rng = _setup(9, "hip", ctx, layers=layers)
        runner.fused_decode = fused
        seqs = [_Seq(rng.integers(0, cfg.vocab_size, c).tolist(), c - 1, t)
                for c, t in zip(ctx, tables)]
        out = runner.execute(_sched(seqs, [1] * len(ctx)), [5, 0, 2])
        runs.append((out, cache))
    ref = runs[1][0].double()
    err = float((runs[0][0].double() - ref).abs().max() / ref.abs().max())
    assert err < logit_tol(layers, "int8"), err
    for (k0, v0), (k1, v1) in zip(runs[0][1].layers, runs[1][1].layers):
        assert _int8_close(k0, k1) and _int8_close(v0, v1)


def test_calibrate_k_smoothing(gpu):
    from llmserve import attention as att
    from llmserve.kernels import load_fused_ops
    from llmserve.transformer import QuantCausalLM

    cfg = tiny_cfg()
    model = QuantCausalLM(cfg, 128, seed=3)
    ids = np.random.default_rng(3).integers(0, cfg.vocab_size, 70).tolist()
    f_hip = att.calibrate_k_smoothing(model, ids, 1.0)
    assert len(f_hip) == cfg.num_hidden_layers
    for f in f_hip:
        assert f.shape == (cfg.num_key_value_heads, cfg.head_dim) and bool((f > 0).all())
        torch.testing.assert_close(f.mean(-1), torch.ones(f.shape[0], device=f.device),
                                   rtol=1e-6, atol=1e-6)
    ones = att.calibrate_k_smoothing(model, ids, 0.0)
    assert all(bool((f == 1).all()) for f in ones)
    # layer 0's keys, computed directly: embedding + norm, qkv projection, q/k norm + RoPE
    fo = load_fused_ops()
    nq, nk, D = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
    L0 = model.layers[0]
    dev_ids = torch.tensor(ids, device="cuda")
    _, h = fo.embed_rmsnorm(dev_ids, model.embed, L0.input_layernorm, cfg.rms_norm_eps)
    qkv = L0.qkv_proj(h).contiguous()
    pos = torch.arange(len(ids), device="cuda")
    fo.rope_qk_(qkv, model.rope_cos[pos].contiguous(), model.rope_sin[pos].contiguous(), nq, nk,
                D, L0.q_norm, L0.k_norm, cfg.rms_norm_eps)
    k0 = qkv[:, nq * D:(nq + nk) * D].reshape(len(ids), nk, D)
    want = att.smoothing_from_stats([k0.abs().amax(0)], 1.0)[0]
    assert torch.equal(f_hip[0], want)
    # the torch attention backend gives the same factors (layer 1 within attention rounding)
    orig = att.resolve_backend
    try:
        att.resolve_backend = lambda name, device="cpu": "torch"
        f_torch = att.calibrate_k_smoothing(model, ids, 1.0)
    finally:
        att.resolve_backend = orig
    assert torch.equal(f_torch[0], f_hip[0])
    torch.testing.assert_close(f_torch[1], f_hip[1], rtol=1e-4, atol=1e-6)


def _prompt_runs(kv_dtype, layers, chunks, first_rows, seed=13, prompt=300):
    """A ``prompt``-token prompt prefilled in ``chunks`` (new-token counts, one execute each;
    every chunk but the last samples ``first_rows``), then one decode step through the fused
    step. Returns (final prefill logits, decode logits, cache snapshots after each execute)."""
    cfg, model, cache, runner, tables, rng = _setup(seed, "hip", [prompt + 1], kv_dtype, layers)
    toks = rng.integers(0, cfg.vocab_size, prompt + 1).tolist()
    snaps, done, out = [], 0, None
    for i, n in enumerate(chunks):
        seq = _Seq(toks[:prompt], done, tables[0])
        rows = [0] if i == len(chunks) - 1 else first_rows
        out = runner.execute(_sched([seq], [n]), rows)
        assert out.shape == (len(rows), cfg.vocab_size)
        done += n
        snaps.append([[t.clone() for t in _cache_tensors(k) + _cache_tensors(v)]
                      for k, v in cache.layers])
    seq = _Seq(toks, prompt, tables[0])
    dec = runner.execute(_sched([seq], [1]), [0])
    return out, dec, snaps


def _cache_tensors(c):
    return [c.data, c.scale] if hasattr(c, "scale") else [c]


@pytest.mark.parametrize("kv_dtype,layers", [("int8", 1), ("int8", 2), ("auto", 2)])
def test_chunked_prefill_step_without_sampled_rows(gpu, kv_dtype, layers):
    """A step made only of a non-final prompt chunk samples nothing (the reference engine's
    execute(sched, []) during chunked prefill, engine.py:323-333) but must still run the
    forward and write the chunk's K/V (model_runner.py:66-83)."""
    quiet, _, snaps_q = _prompt_runs(kv_dtype, layers, [160, 140], [])
    loud, _, snaps_l = _prompt_runs(kv_dtype, layers, [160, 140], [0])
    # the step that samples nothing writes exactly what the same step sampling a row writes
    for a, b in zip(snaps_q, snaps_l):
        for la, lb in zip(a, b):
            assert all(torch.equal(x, y) for x, y in zip(la, lb))
    assert torch.equal(quiet, loud)
    # and the result equals a one-chunk prefill. Its 300-row linears run another kernel than
    # the 160- and 140-row chunks (rounding ~1e-6 apart), so even layer 0's int8 K/V rows can
    # land one step apart (checked below): the two-layer int8 tolerance for every int8 case.
    one, dec_one, snaps_one = _prompt_runs(kv_dtype, layers, [300], [])
    _, dec_two, _ = _prompt_runs(kv_dtype, layers, [160, 140], [])
    tol = logit_tol(2, kv_dtype)
    for x, y in ((quiet, one), (dec_two, dec_one)):
        err = float((x.double() - y.double()).abs().max() / y.double().abs().max())
        assert err < tol, err
    for layer, (la, lb) in enumerate(zip(snaps_q[-1], snaps_one[-1])):
        if kv_dtype == "int8":
            # layer 0 sees only the linears' rounding; deeper layers also the attention over
            # layer 0's differing int8 steps
            share = 0.01 if layer == 0 else 0.05
            for x, y in ((la[0], lb[0]), (la[2], lb[2])):
                d = (x.to(torch.int32) - y.to(torch.int32)).abs()
                assert int(d.max()) <= 1 and float((d > 0).float().mean()) < share
        else:
            for x, y in zip(la, lb):
                assert float((x - y).abs().max()) <= 1e-4 * float(y.abs().max())


def test_execute_raises_when_the_decode_chain_gives_up(gpu):
    """A decode chain whose hand-off waits get a single poll gives up (error word set, rows
    unwritten): execute raises instead of returning logits from unwritten rows, clears the
    word, and a step with the normal poll budget then runs."""
    cfg, model, cache, runner, tables, rng = _setup(17, "hip", [90], "int8", 2)
    assert model._chain_ok(1)
    seq = _Seq(rng.integers(0, cfg.vocab_size, 90).tolist(), 89, tables[0])
    model.chain_spin_limit = 0
    raised = 0
    for _ in range(20):  # a single poll is rarely enough for every wait of a step
        try:
            runner.execute(_sched([seq], [1]), [0])
        except RuntimeError as e:
            assert "ran out of polls" in str(e)
            raised += 1
    assert raised > 0
    model.chain_spin_limit = 1 << 22
    out = runner.execute(_sched([seq], [1]), [0])
    assert torch.isfinite(out).all() and model.chain_error() == 0
