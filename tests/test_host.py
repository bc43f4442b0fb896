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


@pytest.fixture
def hidden_library(monkeypatch, tmp_path):
    """The native op library made unloadable for the duration of a test (loader caches
    cleared before and after)."""
    from llmserve import _native, attention, kernels

    def clear():
        _native.ops.cache_clear()
        for f in (kernels.load_int8_gemv, kernels.load_paged_attention, kernels.load_quant,
                  kernels.load_fused_ops, attention._ops_namespace, attention.resolve_backend):
            f.cache_clear()

    monkeypatch.setattr(_native, "TORCH_LIB", tmp_path / "absent.so")
    clear()
    yield
    monkeypatch.undo()
    clear()


def test_loaders_return_none_without_library(hidden_library):
    """The reference's loader contract (kernels/__init__.py:31-35): None, not an exception."""
    from llmserve import kernels

    assert kernels.load_int8_gemv() is None and kernels.load_paged_attention() is None
    assert kernels.load_quant() is None and kernels.load_fused_ops() is None
    assert not kernels.native_available()
    assert resolve_backend("auto", "cuda") == "torch"
    with pytest.raises(RuntimeError):
        resolve_backend("hip", "cuda")


def _linear(n_out, n_in, seed, bias=False):
    g = torch.Generator().manual_seed(seed)
    lin = torch.nn.Linear(n_in, n_out, bias=bias)
    with torch.no_grad():
        lin.weight.copy_(torch.randn(n_out, n_in, generator=g) * 0.02)
        if bias:
            lin.bias.copy_(torch.randn(n_out, generator=g))
    return lin


@pytest.mark.parametrize("hide", [False, True])
def test_quant_modules_compute_with_torch_on_cpu(request, hide):
    """On CPU tensors (and without the library) the modules run the reference's formulas as
    torch ops: buffers bit-exact with the oracle quantizers, outputs within the reference
    tests' 1e-4 / 2e-4 of the float64 product."""
    if hide:
        request.getfixturevalue("hidden_library")
    from llmserve.quant import Int4Linear, Int8Linear
    from oracle import math_ref as mr

    lin = _linear(96, 256, 0, bias=True)
    w = lin.weight.detach().numpy()
    m8 = Int8Linear(lin)
    q, s = oq.int8_quantize(w)
    assert np.array_equal(m8.qweight.numpy(), q) and np.array_equal(m8.scale.numpy(), s)
    x = torch.randn(3, 256, generator=torch.Generator().manual_seed(1))
    y_ref = mr.int8_linear_f64(x.numpy(), q, s) + lin.bias.detach().numpy()[None]
    for kernel in ("auto", "dequant", "w8a8"):
        Int8Linear.kernel = kernel
        try:
            y = m8(x).detach().numpy()
        finally:
            Int8Linear.kernel = "auto"
        tol = 2e-2 if kernel == "w8a8" else 1e-4  # W8A8 rounds activations (test_quant.py:22-28)
        assert np.abs(y - y_ref).max() <= tol * np.abs(y_ref).max(), kernel
    act = np.abs(np.random.default_rng(2).standard_normal(256)).astype(np.float32) + 0.1
    m4 = Int4Linear(lin, 64, torch.from_numpy(act))
    nib, gs, gz, inv = oq.int4_quantize_pack(w, 64, act)
    for a, b in ((m4.nibbles, nib), (m4.g_scale, gs), (m4.g_zero, gz), (m4.inv_act_scale, inv)):
        assert np.array_equal(a.numpy(), b)
    assert m4.gemm_packed is None
    y4 = m4(x).detach().numpy()
    y4_ref = mr.int4_linear_f64(x.numpy(), nib, gs, gz, 64, inv) + lin.bias.detach().numpy()[None]
    assert np.abs(y4 - y4_ref).max() <= 2e-4 * np.abs(y4_ref).max()
    np.testing.assert_array_equal(m4.dequantize().numpy(), oq.int4_dequantize(nib, gs, gz, 64))


def test_quantized_kv_torch_path_bit_exact():
    rng = np.random.default_rng(4)
    x = rng.standard_normal((12, 2, 32)).astype(np.float32)
    x[0] = 0.0
    sm = (np.abs(rng.standard_normal((2, 32))) + 0.5).astype(np.float32)
    kv = QuantizedKV(40, 2, 32)
    slots = torch.tensor([3, 7, 0, 39, 12, 5, 6, 8, 9, 10, 11, 1])
    kv.write(slots, torch.from_numpy(x), torch.from_numpy(sm))
    qd, qs = oq.kv_quantize(oq.kv_smooth(x, sm))
    assert np.array_equal(kv.data[slots].numpy(), qd) and np.array_equal(kv.scale[slots].numpy(), qs)
    d, s = QuantizedKV.quantize(torch.from_numpy(x))
    qd, qs = oq.kv_quantize(x)
    assert np.array_equal(d.numpy(), qd) and np.array_equal(s.numpy(), qs)
    kv.copy_rows(torch.tensor([20, 21]), torch.tensor([3, 7]))
    assert torch.equal(kv.data[20], kv.data[3]) and torch.equal(kv.scale[21], kv.scale[7])
    assert kv.nbytes() == 40 * 2 * 32 + 40 * 2 * 4


def test_metadata_host_plan_matches_step_rows():
    """Slots of a ragged batch against the reference's construction (attention.py:68-84),
    prefill context slots, the decode slot table / mask, the causal prefill masks."""
    from oracle import math_ref as mr

    q_lens, ctx_lens = [1, 6, 1, 3], [9, 6, 2, 11]
    tables = [[4, 2, 7], [5, 0], [3, 9], [1, 6, 8]]
    meta = AttentionMetadata.build(q_lens, ctx_lens, tables, 4)
    slots, _, _ = mr.step_rows(q_lens, ctx_lens, tables, 4)
    assert meta.slot_mapping.tolist() == slots.tolist()
    assert [(p.q_start, p.q_len, p.ctx_len) for p in meta.prefills] == [(1, 6, 6), (8, 3, 11)]
    for p, t in zip(meta.prefills, (tables[1], tables[3])):
        assert p.slots.tolist() == mr.context_slots(np.array(t), p.ctx_len, 4).tolist()
    assert meta.prefill_mask(0) is None
    mask = meta.prefill_mask(1)
    assert mask.shape == (3, 11) and mask.sum(1).tolist() == [9, 10, 11]
    assert meta.decode_token_idx.tolist() == [0, 7]
    assert meta.decode_slots.tolist()[1][:2] == [12, 13] and meta.decode_mask.shape == (2, 1, 1, 9)


@pytest.mark.parametrize("kv_dtype", ["int8", "auto"])
def test_paged_attention_torch_backend_cpu(kv_dtype):
    """The torch backend on the CPU (the path a build without the library takes) equals the
    float64 attention over the written cache, for a mixed batch."""
    from llmserve.attention import paged_attention
    from oracle import math_ref as mr

    rng = np.random.default_rng(8)
    Hq, Hk, D, bs = 4, 2, 32, 4
    q_lens, ctx_lens = [1, 5, 1], [10, 7, 3]
    tables = [[2, 5, 7], [1, 0], [4]]
    cfg = SimpleNamespace(num_hidden_layers=1, num_key_value_heads=Hk, head_dim=D)
    cache = KVCache(cfg, 8, bs, kv_dtype=kv_dtype)
    kc, vc = cache.layers[0]
    base = torch.from_numpy(rng.standard_normal((32, Hk, D)).astype(np.float32))
    if kv_dtype == "int8":
        kc.write(torch.arange(32), base)
        vc.write(torch.arange(32), base * 0.5)
    else:
        kc.copy_(base)
        vc.copy_(base * 0.5)
    T = sum(q_lens)
    q, k, v = (torch.from_numpy(rng.standard_normal((T, h, D)).astype(np.float32))
               for h in (Hq, Hk, Hk))
    for backend in ("torch", "cpp"):
        meta = AttentionMetadata.build(q_lens, ctx_lens, tables, bs, backend=backend)
        out = paged_attention(q, k, v, kc, vc, meta, D ** -0.5).numpy()
        if kv_dtype == "int8":
            kd, vd = kc.rows(torch.arange(32)).numpy(), vc.rows(torch.arange(32)).numpy()
        else:
            kd, vd = kc.numpy(), vc.numpy()
        _, rows, rctx = mr.step_rows(q_lens, ctx_lens, tables, bs)
        bt = np.zeros((3, 3), np.int64)
        for i, t in enumerate(tables):
            bt[i, :len(t)] = t
        ref = mr.paged_rows_f64(q.numpy(), kd, vd, bt, rows, rctx, bs, D ** -0.5)
        assert np.abs(out - ref).max() <= 1e-5 * np.abs(ref).max(), backend


def test_quantize_model_and_calibration_inputs_cpu():
    from llmserve.quant import (Int4Linear, Int8Linear, _row_sample, collect_linear_inputs,
                                quantize_model, weight_bytes)

    class Tiny(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.up = _linear(64, 128, 1)
            self.down = _linear(128, 64, 2)
            self.lm_head = _linear(32, 128, 3)
            self.register_buffer("rope_cos", torch.zeros(10, 4))

        def forward(self, x):
            return self.lm_head(self.down(torch.relu(self.up(x))))

    m = Tiny()
    before = weight_bytes(m)
    assert before == 4 * (64 * 128 + 128 * 64 + 32 * 128)  # rope tables excluded
    x = torch.randn(3000, 128, generator=torch.Generator().manual_seed(5))
    acts = collect_linear_inputs(m, lambda: m(x), max_rows=512)
    assert set(acts) == {"up", "down", "lm_head"} and acts["up"].shape == (512, 128)
    # the reference's row choice: the first max_rows of a seed-0 permutation
    perm = torch.randperm(3000, generator=torch.Generator().manual_seed(0))[:512]
    assert torch.equal(acts["up"], x[perm]) and torch.equal(_row_sample(x[:10], 512), x[:10])
    with pytest.raises(ValueError):
        quantize_model(Tiny(), "int4-awq")
    with pytest.raises(ValueError):
        quantize_model(Tiny(), "fp8")
    q8 = quantize_model(Tiny(), "int8")
    assert isinstance(q8.up, Int8Linear) and isinstance(q8.lm_head, torch.nn.Linear)
    q4 = quantize_model(m, "int4-awq", 64, calib_acts=acts)
    assert isinstance(q4.up, Int4Linear) and q4.up.inv_act_scale is not None
    assert isinstance(q4.lm_head, torch.nn.Linear) and q4.quantization == "int4-awq"
    assert weight_bytes(q4) < before
    tied = Tiny()
    tied.extra = torch.nn.Linear(128, 32, bias=False)
    tied.extra.weight = tied.lm_head.weight  # a tied weight is counted once
    assert weight_bytes(tied) == before


def test_awq_search_cpu_equals_golden():
    """The product's _search_awq_scale on the CPU (torch ops, the reference's arithmetic) picks
    the golden alpha and bit-identical scales."""
    from conftest import GOLDEN
    from llmserve.quant import _search_awq_scale

    g = np.load(GOLDEN / "quant_golden.npz")
    s = _search_awq_scale(torch.from_numpy(g["awq_w"]), torch.from_numpy(g["awq_x"]),
                          int(g["awq_group"]))
    assert np.array_equal(s.numpy(), g["awq_s"])


def test_decode_runner_context_guard():
    """A step that would pass the block tables or the RoPE table raises before it runs."""
    from llmserve.model_runner import DecodeRunner

    cfg = SimpleNamespace(num_hidden_layers=1, num_key_value_heads=2, head_dim=16)
    model = SimpleNamespace(embed=torch.zeros(4, 8), rope_cos=torch.zeros(100, 16))
    cache = KVCache(cfg, 8, 16, kv_dtype="int8")
    bt = torch.zeros(2, 4, dtype=torch.long)  # 64 slots per sequence
    r = DecodeRunner(model, cache, torch.tensor([1, 2]), torch.tensor([60, 10]), bt)
    assert r.max_context == 64 and r.steps_left() == 5
    for _ in range(5):
        r._advance()
    with pytest.raises(RuntimeError):
        r._advance()
    with pytest.raises(ValueError):
        DecodeRunner(model, cache, torch.tensor([1]), torch.tensor([65]), bt[:1])
    short_rope = SimpleNamespace(embed=torch.zeros(4, 8), rope_cos=torch.zeros(62, 16))
    assert DecodeRunner(short_rope, cache, torch.tensor([1]), torch.tensor([60]), bt[:1]).steps_left() == 3


def test_model_runner_rejects_blocks_past_the_cache():
    """A block table naming a block past the cache (or a negative one) raises on the host, as
    the reference's index_copy_ write does; blocks past the context are not checked."""
    from llmserve.model_runner import ModelRunner

    cfg = SimpleNamespace(num_hidden_layers=1, num_key_value_heads=2, head_dim=16)
    r = ModelRunner.__new__(ModelRunner)
    r.cache = KVCache(cfg, 8, 16, kv_dtype="int8")  # blocks 0..7
    r.block_size = 16
    r._check_tables([[0, 7], [3]], [32, 5])
    r._check_tables([[0, 99]], [16])  # block 99 lies past the context: unused
    r._check_tables([[]], [0])
    with pytest.raises(IndexError, match="out of bounds"):
        r._check_tables([[0, 8]], [17])
    with pytest.raises(IndexError, match="out of bounds"):
        r._check_tables([[1], [-1]], [3, 3])


def test_model_runner_rejects_token_ids_outside_the_vocabulary():
    """A token id outside [0, vocab) raises on the host, as the reference's embedding does
    (the native gather would write a NaN row)."""
    from llmserve.model_runner import ModelRunner

    ModelRunner._check_ids([0, 5, 99], 100)
    ModelRunner._check_ids([], 100)
    with pytest.raises(IndexError, match="index out of range"):
        ModelRunner._check_ids([3, 100], 100)
    with pytest.raises(IndexError, match="index out of range"):
        ModelRunner._check_ids([-1], 100)


_STUB_KERNELS = '''"""Stub laid out as the reference's src/llmserve/kernels/__init__.py (its imports, logger,
csrc path and functools-cached JIT loaders that return a module or None)."""

from __future__ import annotations

import functools
import logging
import os
from pathlib import Path

import torch

log = logging.getLogger(__name__)
_CSRC = Path(__file__).parent / "csrc"


@functools.cache
def load_paged_attention():
    """Return the compiled extension module, or None if it cannot be built."""
    return "reference-cpu:paged_attention"


@functools.cache
def load_fused_ops():
    """Fused ops, or None."""
    return "reference-cpu:fused_ops"


@functools.cache
def load_int8_gemv():
    """Weight-only int8 small-batch matmul, or None."""
    return "reference-cpu:int8_gemv"
'''

_BINDING_CHECK = r'''
import os, sys
import torch
torch.cuda.is_available = lambda: {cuda}  # a ROCm host, as the binding expects (or not)
sys.path.insert(0, {stub!r})
import llmserve.kernels as k
assert os.path.dirname(k.__file__).startswith({stub!r}), k.__file__  # the reference's package
gemv, attn, fused = k.load_int8_gemv(), k.load_paged_attention(), k.load_fused_ops()
if {expect_build}:
    assert sys.modules["llmserve_mi355x.kernels"].__file__.startswith({pkg!r})
    assert "llmserve_hip.int8_linear" in repr(gemv.int8_linear), gemv
    assert "llmserve_hip.int4_linear" in repr(gemv.int4_linear), gemv
    assert "llmserve_hip.paged_attention_decode_int8" in repr(attn.paged_attention_decode_int8)
    assert attn.simd_available() is False and attn.set_simd(True) is None
    assert callable(attn.paged_attention_decode_v1)
    assert "llmserve_hip.rope_qk_" in repr(fused.rope_qk_)
else:
    assert (gemv, attn, fused) == ("reference-cpu:int8_gemv", "reference-cpu:paged_attention",
                                   "reference-cpu:fused_ops"), (gemv, attn, fused)
assert k.load_int8_gemv() is gemv  # cached, as the reference's loaders are
print("binding ok")
'''


@pytest.mark.parametrize("case", ["rocm", "no-device", "no-package"])
def test_reference_binding_from_integration_doc(tmp_path, case):
    """The documented reference-side binding block (the one ``python`` block of the
    repository's integration guide that defines ``_mi355x``), appended verbatim to a stub
    package named ``llmserve`` (laid out as the reference's kernels/__init__.py,
    kernels/__init__.py:19-72), loads this
    build under its alias and returns its namespaces on a ROCm host with no recursion; with no
    device, or no package at the configured path, the reference's own loaders answer."""
    import re
    import subprocess
    import sys

    from conftest import REPO
    from llmserve.kernels import native_available

    doc = (REPO / "INTEGRATION.md").read_text()
    blocks = [b for b in re.findall(r"```python\n(.*?)```", doc, re.S) if "def _mi355x" in b]
    assert len(blocks) == 1
    pkg = tmp_path / "llmserve"
    (pkg / "kernels").mkdir(parents=True)
    (pkg / "__init__.py").write_text('"""Stub of the reference package."""\n')
    (pkg / "kernels" / "__init__.py").write_text(_STUB_KERNELS + "\n\n" + blocks[0])
    ours = REPO / "llm-serving-engine_amd" / "llmserve"
    env = dict(__import__("os").environ)
    env["LLMSERVE_MI355X"] = str(ours if case != "no-package" else tmp_path / "absent")
    env["PYTHONPATH"] = ""
    expect = case == "rocm" and native_available()
    code = _BINDING_CHECK.format(cuda=case != "no-device", stub=str(tmp_path), pkg=str(ours),
                                 expect_build=expect)
    r = subprocess.run([sys.executable, "-c", code], env=env, cwd=tmp_path,
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 0 and "binding ok" in r.stdout, r.stderr[-3000:]
    assert "RecursionError" not in r.stderr
