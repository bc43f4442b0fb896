"""Paged attention over fp32 caches, over the query rows of ragged batches, and the device-side
step metadata, through the C ABI and the drop-in ``paged_attention`` / ``ModelRunner``.

Tolerance as for the int8 decode: max-abs <= 1e-5 * max|out| and rel-L2 <= 1e-5 against the
float64 attention (the reference's SDPA pin, tests/test_attention.py:146-152, is 1e-5), and
2e-5 against the reference's compiled fp32 kernel (committed outputs). The metadata kernel is
bit-exact against the step-row oracle, which walks the batch the way the reference's
AttentionMetadata.build does.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import capi_util as cu
from conftest import GOLDEN
from oracle import math_ref as mr
from oracle import quant as oq

pytestmark = pytest.mark.gpu
F32 = np.float32
TOL = 1e-5


@pytest.mark.parametrize("name,parts", [("f32_small", [0, 8, 10000]), ("f32_d128", [0, 32]),
                                        ("f32_g1", [0, 16])])
def test_fp32_decode_reference_goldens(gpu, name, parts):
    g = dict(np.load(GOLDEN / "attention_f32_golden.npz"))
    bs, sc = g[f"{name}_meta"]
    bs, sc = int(bs), float(sc)
    arrays = [g[f"{name}_{k}"] for k in ("q", "k", "v", "bt", "cl")]
    ref64 = mr.paged_decode_f64(*arrays, bs, sc)
    q, k, v, bt, cl = (cu.dev(a) for a in arrays)
    for p in parts:
        out = cu.paged_decode_f32(q, k, v, bt, cl, bs, sc, p)
        cu.assert_rel_close(out, g[f"{name}_out_p{p}"], 2 * TOL, f"{name} p={p} vs reference")
        cu.assert_rel_close(out, ref64, TOL, f"{name} p={p} vs f64")


def _batch(seed, q_lens, ctx_lens, bs, slack=2):
    """Block tables (a random permutation of the physical blocks) for a ragged batch."""
    rng = np.random.default_rng(seed)
    need = [-(-c // bs) for c in ctx_lens]
    total = sum(need) + slack
    perm = rng.permutation(total).tolist()
    tables, used = [], 0
    for n in need:
        extra = int(rng.integers(0, 2))  # tables may be longer than the context needs
        tables.append(perm[used:used + n] + [0] * extra)
        used += n
    return rng, tables, total


def _packed(tables, ctx_lens, bs):
    need = [-(-c // bs) for c in ctx_lens]
    width = max(need)
    bt = np.zeros((len(tables), width), np.int64)
    for i, (t, n) in enumerate(zip(tables, need)):
        bt[i, :n] = t[:n]
    return bt


# decode rows, a prompt from scratch, a chunk after a cached prefix, a chunk ending mid-block
MIXED = ([1, 37, 1, 12, 1, 5], [300, 37, 1, 80, 1000, 21])


def test_metadata_kernel_matches_step_rows(gpu):
    q_lens, ctx_lens = MIXED
    bs = 16
    _, tables, _ = _batch(3, q_lens, ctx_lens, bs)
    bt = _packed(tables, ctx_lens, bs)
    q = np.array(q_lens, np.int64)
    info = np.stack([q, np.array(ctx_lens, np.int64), np.cumsum(q) - q])
    slots, rows, ctx = cu.attention_metadata(cu.dev(info), cu.dev(bt), bs, int(q.sum()))
    r_slots, r_rows, r_ctx = mr.step_rows(q_lens, ctx_lens, tables, bs)
    np.testing.assert_array_equal(slots.cpu().numpy(), r_slots)
    np.testing.assert_array_equal(rows.cpu().numpy(), r_rows)
    np.testing.assert_array_equal(ctx.cpu().numpy(), r_ctx)


@pytest.mark.parametrize("kv", ["int8", "f32"])
@pytest.mark.parametrize("geom", [(16, 8, 128, 16), (8, 2, 64, 4), (4, 4, 32, 8)])
def test_rows_match_f64(gpu, kv, geom):
    """Every token of a mixed batch (decode rows and prefill rows with their causal prefixes)
    in one launch, int8 cache with key smoothing or fp32 cache."""
    Hq, Hk, D, bs = geom
    q_lens, ctx_lens = MIXED
    rng, tables, total = _batch(11 + D, q_lens, ctx_lens, bs)
    bt = _packed(tables, ctx_lens, bs)
    _, r_rows, r_ctx = mr.step_rows(q_lens, ctx_lens, tables, bs)
    R = r_rows.size
    k = rng.standard_normal((total * bs, Hk, D), dtype=F32)
    k[..., 3] *= 30
    v = rng.standard_normal((total * bs, Hk, D), dtype=F32)
    q = rng.standard_normal((R, Hq, D), dtype=F32)
    sc = D ** -0.5
    if kv == "int8":
        sm = np.maximum(np.abs(k).max(0), F32(1e-5)).astype(F32)
        sm = (sm / sm.mean(-1, keepdims=True)).astype(F32)
        kq, ks = oq.kv_quantize(oq.kv_smooth(k, sm))
        vq, vs = oq.kv_quantize(v)
        qm = np.repeat(sm, Hq // Hk, axis=0).astype(F32)
        ref = mr.paged_rows_f64((q * qm[None]).astype(F32), mr.kv_dequantize(kq, ks),
                                mr.kv_dequantize(vq, vs), bt, r_rows, r_ctx, bs, sc)
        out = cu.paged_rows(cu.dev(q), cu.dev(kq), cu.dev(vq), cu.dev(ks), cu.dev(vs), cu.dev(bt),
                            cu.dev(r_rows), cu.dev(r_ctx), bs, sc, cu.dev(qm))
    else:
        ref = mr.paged_rows_f64(q, k, v, bt, r_rows, r_ctx, bs, sc)
        out = cu.paged_rows(cu.dev(q), cu.dev(k), cu.dev(v), None, None, cu.dev(bt),
                            cu.dev(r_rows), cu.dev(r_ctx), bs, sc)
    cu.assert_rel_close(out, ref, TOL, f"rows {kv} {geom}")


def test_rows_edge_cases(gpu):
    """A row whose table row is outside the table gives NaN (like a zero context) and leaves
    the other rows' values; a decode batch given as rows equals the decode entry point bit for
    bit; R = 0 is a no-op."""
    rng = np.random.default_rng(5)
    Hq, Hk, D, bs = 4, 2, 64, 16
    k = rng.standard_normal((64 * bs, Hk, D), dtype=F32)
    v = rng.standard_normal((64 * bs, Hk, D), dtype=F32)
    bt = rng.permutation(64).reshape(4, 16).astype(np.int64)
    cl = np.array([200, 1, 77, 256], np.int64)
    q = rng.standard_normal((4, Hq, D), dtype=F32)
    dq, dk, dv, dbt, dcl = (cu.dev(a) for a in (q, k, v, bt, cl))
    dec = cu.paged_decode_f32(dq, dk, dv, dbt, dcl, bs, 0.1)
    rows = cu.paged_rows(dq, dk, dv, None, None, dbt, cu.dev(np.arange(4, dtype=np.int64)), dcl,
                         bs, 0.1)
    assert torch.equal(dec, rows)
    bad = cu.paged_rows(dq, dk, dv, None, None, dbt, cu.dev(np.array([0, 9, -1, 3], np.int64)),
                        dcl, bs, 0.1).cpu()
    assert torch.isnan(bad[1]).all() and torch.isnan(bad[2]).all()
    # the split of the work line depends on the whole batch, so the valid rows agree to
    # rounding, not bit for bit
    for i in (0, 3):
        torch.testing.assert_close(bad[i], rows[i].cpu(), rtol=1e-5, atol=1e-6)
    empty = cu.paged_rows(dq[:0], dk, dv, None, None, dbt, dcl[:0], dcl[:0], bs, 0.1)
    assert empty.shape == (0, Hq, D)


@pytest.mark.parametrize("kv_dtype", ["int8", "auto"])
def test_paged_attention_module_native_vs_torch(gpu, kv_dtype):
    """The drop-in paged_attention on a mixed batch: the native backend (device metadata, one
    row launch) against the torch backend (the reference's gather + SDPA), int8 cache with
    key smoothing and fp32 cache; written caches bit-identical."""
    from types import SimpleNamespace

    from llmserve.attention import AttentionMetadata, paged_attention
    from llmserve.kv_cache import KVCache

    Hq, Hk, D, bs = 16, 8, 128, 16
    q_lens, ctx_lens = MIXED
    rng, tables, total = _batch(17, q_lens, ctx_lens, bs)
    cfg = SimpleNamespace(num_hidden_layers=1, num_key_value_heads=Hk, head_dim=D)
    caches = []
    for _ in range(2):
        c = KVCache(cfg, total, bs, device="cuda", kv_dtype=kv_dtype)
        caches.append(c)
    g = torch.Generator(device="cuda").manual_seed(3)
    kv_prefill = torch.randn(total * bs, Hk, D, device="cuda", generator=g)
    sm = None
    if kv_dtype == "int8":
        sm = kv_prefill.abs().amax(0).clamp_min(1e-5)
        sm = sm / sm.mean(-1, keepdim=True)
    for c in caches:
        kc, vc = c.layers[0]
        slots = torch.arange(total * bs, device="cuda")
        if kv_dtype == "int8":
            kc.set_smoothing(sm, Hq)
            kc.write(slots, kv_prefill, kc.smooth)
            vc.write(slots, kv_prefill * 0.5)
        else:
            kc.copy_(kv_prefill)
            vc.copy_(kv_prefill * 0.5)
    T = sum(q_lens)
    q = torch.randn(T, Hq, D, device="cuda", generator=g)
    k = torch.randn(T, Hk, D, device="cuda", generator=g)
    v = torch.randn(T, Hk, D, device="cuda", generator=g)
    outs = []
    for backend, c in zip(("hip", "torch"), caches):
        meta = AttentionMetadata.build(q_lens, ctx_lens, tables, bs, "cuda", backend)
        assert (meta.row_table is not None) == (backend == "hip")
        kc, vc = c.layers[0]
        outs.append(paged_attention(q, k, v, kc, vc, meta, D ** -0.5))
    cu.assert_rel_close(outs[0], outs[1], 4 * TOL, f"native vs torch ({kv_dtype})")
    (k0, v0), (k1, v1) = caches[0].layers[0], caches[1].layers[0]
    if kv_dtype == "int8":
        assert torch.equal(k0.data, k1.data) and torch.equal(k0.scale, k1.scale)
        assert torch.equal(v0.data, v1.data) and torch.equal(v0.scale, v1.scale)
    else:
        assert torch.equal(k0, k1) and torch.equal(v0, v1)


@pytest.mark.parametrize("simd", [True, False])
@pytest.mark.parametrize("partition", [0, 4, 8, 10_000])
def test_loader_v1_entry_and_simd_switch(gpu, simd, partition):
    """The reference's own v1-vs-v2 check (tests/test_attention.py:84-101) through this
    build's loader: paged_attention_decode at every partition size, with set_simd either way,
    equals paged_attention_decode_v1 (one partition per sequence) at 1e-5, and both equal the
    float64 attention."""
    from llmserve.kernels import load_paged_attention

    m = load_paged_attention()
    g = dict(np.load(GOLDEN / "attention_f32_golden.npz"))
    bs, sc = (float(x) for x in g["f32_small_meta"])
    bs = int(bs)
    arrays = [g[f"f32_small_{k}"] for k in ("q", "k", "v", "bt", "cl")]
    q, k, v, bt, cl = (torch.from_numpy(a).to(gpu) for a in arrays)
    ref = m.paged_attention_decode_v1(q, k, v, bt, cl, bs, sc)
    m.set_simd(simd)
    try:
        out = m.paged_attention_decode(q, k, v, bt, cl, bs, sc, partition)
    finally:
        m.set_simd(True)
    torch.testing.assert_close(out, ref, atol=1e-5, rtol=1e-5)
    ref64 = mr.paged_decode_f64(*arrays, bs, sc)
    cu.assert_rel_close(ref, ref64, TOL, "v1 vs f64")
