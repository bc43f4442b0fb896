"""HIP int8-KV paged decode through the C ABI and the drop-in attention module.

Tolerance: max-abs <= 1e-5 * max|out| and rel-L2 <= 1e-5 against the float64 attention over
the dequantized cache (the reference's strongest pin, tests/test_attention.py:146-152, is
1e-5), and against the reference kernel's own outputs (committed goldens) and the C
restatement. At the BASELINE size (config 4) the C restatement is the checker, plus
size-independent properties: partition-size invariance and relabelling of physical blocks.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import capi_util as cu
from conftest import GOLDEN
from oracle import cpu as ocpu
from oracle import math_ref as mr
from oracle import quant as oq

pytestmark = pytest.mark.gpu
F32 = np.float32
TOL = 1e-5


@pytest.fixture(scope="module")
def kg():
    return dict(np.load(GOLDEN / "kernels_golden.npz"))


def _golden_case(kg, name):
    bs, sc = kg[f"{name}_meta"]
    arrays = [kg[f"{name}_{k}"] for k in ("q", "kq", "vq", "ks", "vs", "bt", "cl")]
    return arrays, int(bs), float(sc)


@pytest.mark.parametrize("name,parts", [("pa_small", [0, 4, 8, 10000]), ("pa_d128", [0, 32, 64]),
                                        ("pa_g1", [0, 16])])
def test_reference_goldens(gpu, kg, name, parts):
    arrays, bs, sc = _golden_case(kg, name)
    q, kq, vq, ks, vs, bt, cl = arrays
    ref64 = mr.paged_decode_f64(q, mr.kv_dequantize(kq, ks), mr.kv_dequantize(vq, vs), bt, cl, bs, sc)
    dq = [cu.dev(a) for a in arrays]
    for p in parts:
        out = cu.paged_decode_int8(*dq, bs, sc, p)
        cu.assert_rel_close(out, kg[f"{name}_out_p{p}"], 2 * TOL, f"{name} p={p} vs reference")
        cu.assert_rel_close(out, ref64, TOL, f"{name} p={p} vs f64")


def make_case(seed, B, Hq, Hk, D, bs, ctx_lo, ctx_hi, outlier=True, slack_blocks=3):
    rng = np.random.default_rng(seed)
    ctx = rng.integers(ctx_lo, ctx_hi + 1, B)
    nblk = [-(-int(c) // bs) for c in ctx]
    total = sum(nblk) + slack_blocks
    perm = rng.permutation(total)
    width = max(nblk)
    bt = np.zeros((B, width), np.int64)
    used = 0
    for b, n in enumerate(nblk):
        bt[b, :n] = perm[used:used + n]
        used += n
    k = rng.standard_normal((total * bs, Hk, D), dtype=F32)
    if outlier:
        k[..., 3] *= 40
        k[..., D // 2 + 1] *= 25
    v = rng.standard_normal((total * bs, Hk, D), dtype=F32)
    sm = np.maximum(np.abs(k).max(0), F32(1e-5)).astype(F32)
    sm = (sm / sm.mean(-1, keepdims=True)).astype(F32)
    kq, ks = oq.kv_quantize(oq.kv_smooth(k, sm))
    vq, vs = oq.kv_quantize(v)
    q = rng.standard_normal((B, Hq, D)).astype(F32)
    q_mult = np.repeat(sm, Hq // Hk, axis=0).astype(F32)
    return dict(q=q, kq=kq, vq=vq, ks=ks, vs=vs, bt=bt, cl=ctx.astype(np.int64), q_mult=q_mult)


@pytest.mark.parametrize("Hq,Hk,D,bs", [(16, 8, 128, 16), (8, 2, 32, 4), (9, 3, 64, 16),
                                        (4, 4, 16, 8), (8, 1, 256, 16), (32, 4, 128, 32)])
def test_geometries_vs_f64(gpu, Hq, Hk, D, bs):
    c = make_case(Hq * 31 + D, 5, Hq, Hk, D, bs, 1, 300)
    ref = mr.paged_decode_f64(oq.q_smooth(c["q"], c["q_mult"]), mr.kv_dequantize(c["kq"], c["ks"]),
                              mr.kv_dequantize(c["vq"], c["vs"]), c["bt"], c["cl"], bs, D ** -0.5)
    args = [cu.dev(c[k]) for k in ("q", "kq", "vq", "ks", "vs", "bt", "cl")]
    for p in (0, bs, 64, 100000):
        out = cu.paged_decode_int8(*args, bs, D ** -0.5, p, cu.dev(c["q_mult"]))
        cu.assert_rel_close(out, ref, TOL, f"H{Hq}/{Hk} D{D} bs{bs} p{p}")


def test_baseline_config4_size(gpu):
    """16q/8kv heads, D=128, block 16, batch 32, ctx ~ U[512, 8192],
    permuted blocks, outlier key channels with smoothing. Checked against the C restatement;
    partition sizes agree and relabelling the physical blocks changes nothing."""
    c = make_case(2024, 32, 16, 8, 128, 16, 512, 8192)
    args = [cu.dev(c[k]) for k in ("q", "kq", "vq", "ks", "vs", "bt", "cl")]
    qm = cu.dev(c["q_mult"])
    sc = 128 ** -0.5
    out = cu.paged_decode_int8(*args, 16, sc, 0, qm)
    ref = ocpu.paged_decode_int8(c["q"], c["kq"], c["vq"], c["ks"], c["vs"], c["bt"], c["cl"], 16,
                                 sc, 0, c["q_mult"])
    cu.assert_rel_close(out, ref, 2 * TOL, "config 4 vs C restatement")
    out2 = cu.paged_decode_int8(*args, 16, sc, 1024, qm)
    cu.assert_rel_close(out2, out, 2 * TOL, "partition 1024 vs auto")
    # relabel physical blocks: move every block to a new id
    nb = c["kq"].shape[0] // 16
    relabel = np.random.default_rng(1).permutation(nb)
    inv = np.argsort(relabel)
    kq2 = c["kq"].reshape(nb, 16, 8, 128)[inv].reshape(c["kq"].shape)
    vq2 = c["vq"].reshape(nb, 16, 8, 128)[inv].reshape(c["vq"].shape)
    ks2 = c["ks"].reshape(nb, 16, 8)[inv].reshape(c["ks"].shape)
    vs2 = c["vs"].reshape(nb, 16, 8)[inv].reshape(c["vs"].shape)
    bt2 = relabel[c["bt"]]
    args2 = [cu.dev(a) for a in (c["q"], kq2, vq2, ks2, vs2, bt2, c["cl"])]
    out3 = cu.paged_decode_int8(*args2, 16, sc, 0, qm)
    assert torch.equal(out3, out)


@pytest.mark.parametrize("B,lo,hi", [(32, 512, 8192), (64, 1024, 4096), (7, 1, 3000)])
def test_balanced_plan_is_a_64_token_partition(gpu, B, lo, hi):
    """The default split (partition_size 0) cuts every (sequence, kv head group) into ranges
    of Q tokens, the last one the rest, with Q a multiple of 64 chosen from the contexts: its
    output equals, bit for bit, that of a fixed partition size of some multiple of 64 (same
    ranges, same per-range arithmetic, the partials merged in the same order)."""
    c = make_case(B + lo, B, 16, 8, 128, 16, lo, hi)
    args = [cu.dev(c[k]) for k in ("q", "kq", "vq", "ks", "vs", "bt", "cl")]
    qm = cu.dev(c["q_mult"])
    sc = 128 ** -0.5
    out = cu.paged_decode_int8(*args, 16, sc, 0, qm)
    ref = ocpu.paged_decode_int8(c["q"], c["kq"], c["vq"], c["ks"], c["vs"], c["bt"], c["cl"], 16,
                                 sc, 0, c["q_mult"])
    cu.assert_rel_close(out, ref, 2 * TOL, f"B={B}: balanced plan vs C restatement")
    top = -(-int(c["cl"].max()) // 64) * 64
    same = [P for P in range(64, top + 65, 64)
            if torch.equal(cu.paged_decode_int8(*args, 16, sc, P, qm), out)]
    assert same, f"B={B}: no 64-token multiple reproduces the balanced plan"


def test_skewed_batch_within_unit_slots(gpu):
    """One long sequence among 255 short ones: the workspace holds a few times each unit's
    fair share of ranges, so the plan widens the ranges until the long unit fits; the result
    still matches float64 and a fixed partition size."""
    c = make_case(77, 256, 16, 8, 64, 16, 1, 24, outlier=False, slack_blocks=300)
    bs = 16
    long_blocks = 250  # 4000 tokens in blocks past the short rows' blocks
    nb = c["kq"].shape[0] // bs
    width = max(c["bt"].shape[1], long_blocks)
    bt = np.zeros((256, width), np.int64)
    bt[:, :c["bt"].shape[1]] = c["bt"]
    bt[100, :long_blocks] = np.random.default_rng(3).permutation(nb)[:long_blocks]
    cl = c["cl"].copy()
    cl[100] = long_blocks * bs
    ref = mr.paged_decode_f64(oq.q_smooth(c["q"], c["q_mult"]), mr.kv_dequantize(c["kq"], c["ks"]),
                              mr.kv_dequantize(c["vq"], c["vs"]), bt, cl, bs, 0.125)
    args = [cu.dev(a) for a in (c["q"], c["kq"], c["vq"], c["ks"], c["vs"], bt, cl)]
    out = cu.paged_decode_int8(*args, bs, 0.125, 0, cu.dev(c["q_mult"]))
    cu.assert_rel_close(out, ref, TOL, "skewed batch, balanced plan")
    out64 = cu.paged_decode_int8(*args, bs, 0.125, 64, cu.dev(c["q_mult"]))
    cu.assert_rel_close(out64, ref, TOL, "skewed batch, 64-token partitions")


@pytest.mark.parametrize("seed", range(12))
def test_random_batches_vs_f64(gpu, seed):
    """Seeded random batches across the split's regimes: 1 to 300 rows (one or several
    64-row windows of the plan), contexts uniform, skewed (one long row) or with empty rows,
    several head geometries and block sizes, the balanced split or a random fixed partition
    size. Rows with an empty context must be NaN, every other row within 1e-5 of float64."""
    rng = np.random.default_rng(1000 + seed)
    Hq, Hk, D = [(16, 8, 128), (8, 8, 64), (32, 4, 128), (12, 4, 64)][seed % 4]
    bs = [16, 32, 8][seed % 3]
    B = int(rng.choice([1, 3, 17, 64, 65, 130, 300]))
    c = make_case(seed, B, Hq, Hk, D, bs, 1, 300, outlier=seed % 2 == 0, slack_blocks=40)
    cl = c["cl"].copy()
    kind = seed % 3
    nb = c["kq"].shape[0] // bs
    bt = c["bt"]
    if kind == 1:  # one long row over blocks shared with the others
        long_blocks = min(nb, 120)
        bt = np.zeros((B, max(bt.shape[1], long_blocks)), np.int64)
        bt[:, :c["bt"].shape[1]] = c["bt"]
        r = int(rng.integers(B))
        bt[r, :long_blocks] = rng.permutation(nb)[:long_blocks]
        cl[r] = long_blocks * bs - int(rng.integers(bs))
    elif kind == 2:  # some empty rows
        cl[rng.random(B) < 0.2] = 0
    scale = D ** -0.5
    ref = mr.paged_decode_f64(oq.q_smooth(c["q"], c["q_mult"]), mr.kv_dequantize(c["kq"], c["ks"]),
                              mr.kv_dequantize(c["vq"], c["vs"]), bt, np.maximum(cl, 1), bs, scale)
    args = [cu.dev(a) for a in (c["q"], c["kq"], c["vq"], c["ks"], c["vs"], bt, cl)]
    part = 0 if seed % 4 < 2 else int(rng.integers(1, 200))
    out = cu.paged_decode_int8(*args, bs, scale, part, cu.dev(c["q_mult"])).cpu().numpy()
    empty = cl == 0
    assert np.isnan(out[empty]).all(), f"seed {seed}: empty rows must be NaN"
    if (~empty).any():
        cu.assert_rel_close(torch.from_numpy(out[~empty]), ref[~empty], TOL,
                            f"seed {seed}: B={B} H{Hq}/{Hk} D{D} bs{bs} part {part} kind {kind}")


def test_cache_beyond_4gb(gpu):
    """A cache tensor of more than 4 GB (num_slots * Hk * D > 2^32) takes the kernel variant
    with 64-bit slot addressing; its sequences live in blocks past the 4 GB mark. The used
    blocks are copied into the big cache on the device and checked against the oracle on a
    compact copy of the same blocks (same tokens, relabelled)."""
    c = make_case(41, 3, 16, 8, 128, 16, 20, 120, slack_blocks=0)
    bs, Hk, D = 16, 8, 128
    nb_small = c["kq"].shape[0] // bs
    nb_big = (1 << 32) // (bs * Hk * D) + 64  # 4.3 GB of K, as much of V
    dev_blocks = nb_big - 1 - np.arange(nb_small)  # block i of the small cache -> a high id
    kq = torch.zeros(nb_big * bs, Hk, D, dtype=torch.int8, device="cuda")
    vq = torch.zeros_like(kq)
    ks = torch.zeros(nb_big * bs, Hk, device="cuda")
    vs = torch.zeros_like(ks)
    rows = torch.from_numpy((dev_blocks[:, None] * bs + np.arange(bs)[None, :]).ravel()).cuda()
    kq[rows] = cu.dev(c["kq"])
    vq[rows] = cu.dev(c["vq"])
    ks[rows] = cu.dev(c["ks"])
    vs[rows] = cu.dev(c["vs"])
    bt_big = dev_blocks[c["bt"]]
    assert kq.numel() > (1 << 32)
    out = cu.paged_decode_int8(cu.dev(c["q"]), kq, vq, ks, vs, cu.dev(bt_big), cu.dev(c["cl"]), bs,
                               D ** -0.5, 0, cu.dev(c["q_mult"]))
    ref = mr.paged_decode_f64(oq.q_smooth(c["q"], c["q_mult"]), mr.kv_dequantize(c["kq"], c["ks"]),
                              mr.kv_dequantize(c["vq"], c["vs"]), c["bt"], c["cl"], bs, D ** -0.5)
    cu.assert_rel_close(out, ref, TOL, "cache > 4 GB")
    del kq, vq, ks, vs
    torch.cuda.empty_cache()


def test_edge_contexts(gpu):
    """ctx = 1 returns the token's value row; ctx = 0 gives NaN (the reference's 0 * (1/0))."""
    c = make_case(5, 3, 4, 2, 32, 4, 9, 9, outlier=False)
    c["cl"][:] = [1, 0, 9]
    args = [cu.dev(c[k]) for k in ("q", "kq", "vq", "ks", "vs", "bt", "cl")]
    for p in (0, 4):
        out = cu.paged_decode_int8(*args, 4, 0.2, p).cpu().numpy()
        slot = c["bt"][0, 0] * 4
        vrow = mr.kv_dequantize(c["vq"][slot], c["vs"][slot])
        np.testing.assert_allclose(out[0], np.repeat(vrow, 2, axis=0), rtol=1e-6, atol=1e-6)
        assert np.isnan(out[1]).all()
        assert np.isfinite(out[2]).all()


@pytest.mark.parametrize("B,Hq,Hk,D,bs,part,with_inv,zero_ctx", [
    (5, 4, 2, 128, 16, 0, True, False),     # 16-row padding of the fragments
    (20, 8, 4, 256, 16, 0, False, False),   # two 128-channel blocks per head
    (17, 16, 8, 128, 16, 64, True, False),  # fixed ranges: whole and split sequences
    (6, 4, 2, 128, 8, 0, True, True),       # a zero context: NaN rows
])
def test_merge_writes_oproj_fragments(gpu, B, Hq, Hk, D, bs, part, with_inv, zero_ctx):
    """The decode whose merge writes o_proj's input fragments: its output equals the plain
    decode's bit for bit, and its fragments (x' = out * inv_act_scale, bf16 hi / mid / lo,
    block sums) equal those the packed int4 linear's split pass makes of that output."""
    c = make_case(B * 7 + D, B, Hq, Hk, D, bs, 1, 700)
    if zero_ctx:
        c["cl"][1] = 0
    args = [cu.dev(c[k]) for k in ("q", "kq", "vq", "ks", "vs", "bt", "cl")]
    qm = cu.dev(c["q_mult"])
    rng = np.random.default_rng(B)
    inv = cu.dev((0.5 + rng.random(Hq * D)).astype(F32)) if with_inv else None
    ref = cu.paged_decode_int8(*args, bs, D ** -0.5, part, qm)
    out, xf = cu.paged_decode_int8_xfrag(*args, bs, D ** -0.5, part, qm, inv)
    assert torch.equal(out.view(torch.int32), ref.view(torch.int32))
    if zero_ctx:
        assert torch.isnan(out[1]).all() and torch.isfinite(out[0]).all()
    assert torch.equal(xf, cu.split_fragments(ref.view(B, Hq * D), inv))


def test_merge_fragments_reject_bad_head_dim(gpu):
    c = make_case(3, 2, 4, 2, 64, 16, 1, 50)
    args = [cu.dev(c[k]) for k in ("q", "kq", "vq", "ks", "vs", "bt", "cl")]
    with pytest.raises(RuntimeError, match="128 or 256"):
        cu.paged_decode_int8_xfrag(*args, 16, 0.125)


def test_invalid_block_ids_are_skipped(gpu):
    c = make_case(6, 2, 8, 2, 32, 4, 12, 12, outlier=False)
    bt = c["bt"].copy()
    bt[0, 1] = 10**9  # out of range: those 4 tokens contribute nothing
    args = [cu.dev(a) for a in (c["q"], c["kq"], c["vq"], c["ks"], c["vs"], bt, c["cl"])]
    out = cu.paged_decode_int8(*args, 4, 0.2).cpu().numpy()
    keep = np.array([0, 2])
    bt_ok = c["bt"][:1, keep]
    ref = mr.paged_decode_f64(c["q"][:1], mr.kv_dequantize(c["kq"], c["ks"]),
                              mr.kv_dequantize(c["vq"], c["vs"]), bt_ok, np.array([8]), 4, 0.2)
    cu.assert_rel_close(out[:1], ref, TOL)


# ---- drop-in module tests (mirroring the reference's tests/test_attention.py) --------------

def _int8_caches(kc, vc):
    from llmserve.attention import QuantizedKV

    kq, vq = QuantizedKV(*kc.shape, device=kc.device), QuantizedKV(*vc.shape, device=vc.device)
    all_slots = torch.arange(kc.shape[0], device=kc.device)
    kq.write(all_slots, kc)
    vq.write(all_slots, vc)
    return kq, vq


def test_quantized_kv_roundtrip_error_is_bounded(gpu):
    from llmserve.attention import QuantizedKV

    x = torch.randn(64, 2, 32, device="cuda")
    c = QuantizedKV(64, 2, 32, device="cuda")
    c.write(torch.arange(64, device="cuda"), x)
    err = (c.rows(torch.arange(64, device="cuda")) - x).abs()
    assert (err <= c.scale[..., None] / 2 + 1e-6).all()
    q, s = QuantizedKV.quantize(x)
    assert torch.equal(q, c.data) and torch.equal(s, c.scale)


@pytest.mark.parametrize("q_lens,ctx_lens", [([1, 1, 1], [5, 40, 17]), ([6, 1, 1], [6, 23, 9])])
def test_int8_kv_attention_close_to_fp32(gpu, q_lens, ctx_lens):
    from llmserve.attention import AttentionMetadata, QuantizedKV, paged_attention

    g = torch.Generator().manual_seed(4)
    hq, hk, d, bs = 8, 2, 32, 4
    kc = torch.randn(64 * bs, hk, d, generator=g).cuda()
    vc = torch.randn(64 * bs, hk, d, generator=g).cuda()
    tables, used = [], 0
    for c in ctx_lens:
        n = -(-c // bs)
        tables.append(list(range(used, used + n)))
        used += n
    T = sum(q_lens)
    q, k, v = (torch.randn(T, h, d, generator=g).cuda() for h in (hq, hk, hk))
    ref_meta = AttentionMetadata.build(q_lens, ctx_lens, tables, bs, device="cuda", backend="torch")
    ref = paged_attention(q, k, v, kc.clone(), vc.clone(), ref_meta, d**-0.5)
    meta = AttentionMetadata.build(q_lens, ctx_lens, tables, bs, device="cuda", backend="hip")
    kq, vq = _int8_caches(kc, vc)
    out = paged_attention(q, k, v, kq, vq, meta, d**-0.5)
    rel = (out - ref).norm() / ref.norm()
    assert rel < 0.02, rel
    # the int8 kernel equals attention over the dequantized cache (same math)
    all_slots = torch.arange(kc.shape[0], device="cuda")
    kd, vd = kq.rows(all_slots), vq.rows(all_slots)
    kr, vr = ((lambda t: t[0].float() * t[1][..., None])(QuantizedKV.quantize(x)) for x in (k, v))
    deq = paged_attention(q, kr, vr, kd, vd, ref_meta, d**-0.5)
    torch.testing.assert_close(out, deq, atol=1e-5, rtol=1e-5)


def test_k_smoothing_reduces_int8_error_with_outlier_channels(gpu):
    from llmserve.attention import AttentionMetadata, QuantizedKV, paged_attention

    g = torch.Generator().manual_seed(5)
    hq, hk, d, bs = 8, 2, 32, 4
    n = 40 * bs
    kc = torch.randn(n, hk, d, generator=g)
    kc[..., 3] *= 40.0
    kc[..., 17] *= 25.0
    kc = kc.cuda()
    vc = torch.randn(n, hk, d, generator=g).cuda()
    ctx = [37, 60, 11]
    tables, used = [], 0
    for c in ctx:
        m = -(-c // bs)
        tables.append(list(range(used, used + m)))
        used += m
    q = (torch.randn(len(ctx), hq, d, generator=g) * 0.2).cuda()
    k, v = torch.randn(len(ctx), hk, d, generator=g).cuda(), torch.randn(len(ctx), hk, d, generator=g).cuda()
    ref_meta = AttentionMetadata.build([1] * 3, ctx, tables, bs, device="cuda", backend="torch")
    ref = paged_attention(q, k, v, kc.clone(), vc.clone(), ref_meta, d**-0.5)
    meta = AttentionMetadata.build([1] * 3, ctx, tables, bs, device="cuda", backend="hip")

    def run(smooth):
        kq, vq = QuantizedKV(n, hk, d, device="cuda"), QuantizedKV(n, hk, d, device="cuda")
        if smooth is not None:
            kq.set_smoothing(smooth, hq)
        kq.write(torch.arange(n, device="cuda"), kc / (smooth if smooth is not None else 1.0))
        vq.write(torch.arange(n, device="cuda"), vc)
        out = paged_attention(q, k, v, kq, vq, meta, d**-0.5)
        return ((out - ref).norm() / ref.norm()).item()

    s = kc.abs().amax(0).sqrt()
    s = s / s.mean(-1, keepdim=True)
    assert run(s) < 0.5 * run(None)
