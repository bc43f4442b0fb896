"""Host-side logic of the drop-in modules, CPU only: attention metadata, KV-cache sizing,
smoothing factors, backend resolution and loud failure when the native build is missing."""

from __future__ import annotations

from types import SimpleNamespace

import numpy as np
import pytest
import torch

from llmserve.attention import AttentionMetadata, QuantizedKV, resolve_backend, smoothing_from_stats
from llmserve.kv_cache import KVCache
from oracle import quant as oq


def test_metadata_native_tables():
    meta = AttentionMetadata.build([1, 1, 3], [5, 9, 3], [[4, 2], [7, 1, 3], [0]], 4, backend="cpp")
    assert meta.backend == "hip"
    assert meta.decode_block_tables.tolist() == [[4, 2, 0], [7, 1, 3]]  # zero-padded
    assert meta.decode_ctx_lens.tolist() == [5, 9]
    assert meta.decode_token_idx.tolist() == [0, 1]
    # slots of the new tokens: last token of each decode seq, all 3 of the prefill
    assert meta.slot_mapping.tolist() == [2 * 4 + 0, 3 * 4 + 0, 0, 1, 2]
    assert len(meta.prefills) == 1 and meta.prefills[0].q_start == 2


def test_metadata_torch_tables_and_errors():
    meta = AttentionMetadata.build([1, 1], [2, 6], [[3], [5, 6]], 4)
    assert meta.decode_slots.tolist() == [[12, 13, 0, 0, 0, 0], [20, 21, 22, 23, 24, 25]]
    assert meta.decode_mask[:, 0, 0].tolist() == [[True, True] + [False] * 4, [True] * 6]
    with pytest.raises(ValueError):
        AttentionMetadata.build([1], [9], [[1, 2]], 4)


def test_kv_cache_int8_sizing():
    cfg = SimpleNamespace(num_hidden_layers=28, num_key_value_heads=8, head_dim=128)
    fp = KVCache.blocks_for_memory(cfg, 1 << 30, 16)
    i8 = KVCache.blocks_for_memory(cfg, 1 << 30, 16, kv_dtype="int8")
    D = cfg.head_dim
    assert i8 >= 0.95 * 4 * D / (D + 4) * fp  # reference tests/test_engine.py:159-182
    c = KVCache(cfg, 4, 16, kv_dtype="int8")
    k, v = c.layers[0]
    assert isinstance(k, QuantizedKV) and k.data.shape == (64, 8, 128) and k.scale.shape == (64, 8)
    assert c.nbytes() == 28 * 2 * (64 * 8 * 128 + 64 * 8 * 4)
    with pytest.raises(ValueError):
        KVCache(cfg, 4, 16, kv_dtype="fp8")


def test_smoothing_factors_match_oracle_and_invariants():
    rng = np.random.default_rng(0)
    m = np.abs(rng.standard_normal((8, 128))).astype(np.float32) * 3
    m[:, 5] = 0.0
    s = smoothing_from_stats([torch.from_numpy(m)], alpha=1.0)[0]
    np.testing.assert_allclose(s.numpy(), oq.smoothing_from_stats(m, 1.0), rtol=1e-6)
    np.testing.assert_allclose(s.mean(-1).numpy(), 1.0, rtol=1e-5)
    # monotone in max|K| within a head
    order = np.argsort(m[0])
    assert np.all(np.diff(s[0].numpy()[order]) >= 0)


def test_set_smoothing_repeats_per_gqa_group():
    kv = QuantizedKV(8, 2, 4)
    s = torch.arange(1, 9, dtype=torch.float32).view(2, 4)
    kv.set_smoothing(s, num_q_heads=6)
    assert kv._q_mult.shape == (6, 4)
    assert torch.equal(kv._q_mult[:3], s[0].expand(3, 4)) and torch.equal(kv._q_mult[3:], s[1].expand(3, 4))


def test_resolve_backend_on_cpu():
    assert resolve_backend("torch", "cpu") == "torch"
    assert resolve_backend("auto", "cpu") == "torch"
    with pytest.raises(RuntimeError):
        resolve_backend("hip", "cpu")
    with pytest.raises(ValueError):
        resolve_backend("cuda-graphs", "cpu")


def test_missing_native_library_fails_loudly(monkeypatch, tmp_path):
    from llmserve import _native

    monkeypatch.setattr(_native, "TORCH_LIB", tmp_path / "absent.so")
    _native.ops.cache_clear()
    try:
        with pytest.raises(_native.NativeLibraryMissing):
            _native.ops()
    finally:
        _native.ops.cache_clear()


def test_quantized_ops_reject_cpu_tensors():
    from llmserve.kernels import load_int8_gemv

    k = load_int8_gemv()
    with pytest.raises((NotImplementedError, RuntimeError)):
        k.int8_linear(torch.zeros(1, 16), torch.zeros(4, 16, dtype=torch.int8), torch.zeros(4))
