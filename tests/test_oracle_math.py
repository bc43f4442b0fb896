"""Pins of the float64 references (oracle/math_ref.py), CPU only: brute-force loops, torch
SDPA in float64 and closed forms."""

from __future__ import annotations

import numpy as np
import torch

from oracle import math_ref as mr
from oracle import quant as oq


def test_linear_brute_force():
    rng = np.random.default_rng(0)
    x = rng.standard_normal((3, 7)).astype(np.float32)
    q, s = oq.int8_quantize(rng.standard_normal((5, 7)).astype(np.float32))
    y = mr.int8_linear_f64(x, q, s)
    for m in range(3):
        for n in range(5):
            # the dequantized weight is the float32 product q * scale (quant.py:79)
            w = [float(np.float32(q[n, k]) * s[n]) for k in range(7)]
            assert abs(y[m, n] - sum(float(x[m, k]) * w[k] for k in range(7))) < 1e-9


def test_int4_awq_prescale_applied_once():
    rng = np.random.default_rng(1)
    w = (rng.standard_normal((4, 64)) * 0.02).astype(np.float32)
    act = np.abs(rng.standard_normal(64)).astype(np.float32) + 0.5
    nib, gs, gz, inv = oq.int4_quantize_pack(w, 32, act)
    x = rng.standard_normal((2, 64)).astype(np.float32)
    y = mr.int4_linear_f64(x, nib, gs, gz, 32, inv)
    # (x / s) @ Q(W s)^T ~= x @ W^T within int4 rounding of the scaled weight
    deq = oq.int4_dequantize(nib, gs, gz, 32) * inv[None, :]
    np.testing.assert_allclose(y, x.astype(np.float64) @ deq.T.astype(np.float64), rtol=1e-5, atol=1e-6)


def _paged_case(seed, B=3, Hq=4, Hk=2, D=16, bs=4, nblk=16):
    rng = np.random.default_rng(seed)
    k = rng.standard_normal((nblk * bs, Hk, D)).astype(np.float32)
    v = rng.standard_normal((nblk * bs, Hk, D)).astype(np.float32)
    bt = rng.permutation(nblk)[: B * 4].reshape(B, 4).astype(np.int64)
    cl = np.array([13, 1, 16], np.int64)[:B]
    q = rng.standard_normal((B, Hq, D)).astype(np.float32)
    return q, k, v, bt, cl, bs


def test_paged_decode_matches_sdpa():
    q, k, v, bt, cl, bs = _paged_case(0)
    out = mr.paged_decode_f64(q, k, v, bt, cl, bs, 0.3)
    G = q.shape[1] // k.shape[1]
    for b in range(q.shape[0]):
        slots = mr.context_slots(bt[b], int(cl[b]), bs)
        kb = torch.from_numpy(k[slots]).double().repeat_interleave(G, 1).transpose(0, 1)
        vb = torch.from_numpy(v[slots]).double().repeat_interleave(G, 1).transpose(0, 1)
        qb = torch.from_numpy(q[b]).double()[:, None, :]
        ref = torch.nn.functional.scaled_dot_product_attention(qb, kb, vb, scale=0.3)[:, 0]
        np.testing.assert_allclose(out[b], ref.numpy(), rtol=1e-12, atol=1e-12)


def test_paged_decode_closed_forms():
    q, k, v, bt, cl, bs = _paged_case(1)
    # one-token context: the output is that token's value row
    out = mr.paged_decode_f64(q, k, v, bt, cl, bs, 0.3)
    s0 = bt[1, 0] * bs
    np.testing.assert_allclose(out[1], np.repeat(v[s0], 2, axis=0), rtol=0, atol=1e-12)
    # identical keys: uniform weights -> mean of the value rows
    k_same = np.broadcast_to(k[:1], k.shape).copy()
    out = mr.paged_decode_f64(q, k_same, v, bt, cl, bs, 0.3)
    slots = mr.context_slots(bt[0], int(cl[0]), bs)
    np.testing.assert_allclose(out[0], np.repeat(v[slots].astype(np.float64).mean(0), 2, axis=0), atol=1e-12)


def test_bf16_round_matches_torch_cast():
    """bf16_round against torch's CPU float32 -> bfloat16 cast (round half to even)."""
    rng = np.random.default_rng(11)
    x = np.concatenate([
        rng.standard_normal(4096).astype(np.float32) * np.float32(10) ** rng.integers(-30, 30, 4096),
        # exact ties: low half 0x8000 with an even and an odd kept mantissa
        np.array([0x3F808000, 0x3F818000, 0xBF808000, 0xBF818000], np.uint32).view(np.float32),
        # just below / above a tie, rounding into the next binade, signed zeros, subnormals
        np.array([0x3F807FFF, 0x3F808001, 0x3FFFFFFF, 0x7F7FFFFF - 0x10000, 0x80000000, 0x00000000,
                  0x00000001, 0x8000FFFF, 0x007F8000], np.uint32).view(np.float32),
    ]).astype(np.float32)
    want = torch.from_numpy(x).to(torch.bfloat16).to(torch.float32).numpy()
    got = mr.bf16_round(x)
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))
    # a plausible mistake, truncation instead of rounding, is caught
    trunc = (x.view(np.uint32) & np.uint32(0xFFFF0000)).view(np.float32)
    assert not np.array_equal(trunc.view(np.uint32), want.view(np.uint32))


def test_prefill_reference_brute_force():
    """int8_linear_prefill_f64 = sum_k bf16(x) q scale, by loops on a tiny case; without the
    rounding it is the plain weight-only product."""
    rng = np.random.default_rng(12)
    M, N, K = 3, 5, 7
    x = rng.standard_normal((M, K)).astype(np.float32)
    q = rng.integers(-127, 128, (N, K)).astype(np.int8)
    s = (rng.random(N) * 0.01 + 1e-3).astype(np.float32)
    xr = torch.from_numpy(x).to(torch.bfloat16).to(torch.float64).numpy()
    want = np.array([[sum(xr[m, k] * float(q[n, k]) for k in range(K)) * float(s[n])
                      for n in range(N)] for m in range(M)])
    np.testing.assert_allclose(mr.int8_linear_prefill_f64(x, q, s), want, rtol=1e-13, atol=0)
    plain = mr.int8_linear_f64(x, q, s)
    np.testing.assert_allclose(mr.int8_linear_prefill_f64(x, q, s, round_x=False), plain,
                               rtol=1e-6, atol=1e-12)


def test_rows_oracle_is_causal_sdpa():
    """A prefill chunk's rows (contexts p + 1 over one block-table row) equal float64 SDPA with
    the reference's mask k_pos <= q_pos (attention.py:114-124), a chunk with no cached prefix
    equals is_causal, and a decode row equals paged_decode_f64."""
    rng = np.random.default_rng(21)
    Hq, Hk, D, bs, nblk = 4, 2, 16, 4, 12
    k = rng.standard_normal((nblk * bs, Hk, D))
    v = rng.standard_normal((nblk * bs, Hk, D))
    table = rng.permutation(nblk)
    for cached, q_len in ((0, 9), (11, 6)):
        ctx = cached + q_len
        q = rng.standard_normal((q_len, Hq, D))
        got = mr.paged_rows_f64(q, k, v, table[None, :], np.zeros(q_len, np.int64),
                                np.arange(cached + 1, ctx + 1), bs, D ** -0.5)
        slots = mr.context_slots(table, ctx, bs)
        kt = torch.from_numpy(k[slots]).transpose(0, 1)[None]  # [1, Hk, ctx, D]
        vt = torch.from_numpy(v[slots]).transpose(0, 1)[None]
        qt = torch.from_numpy(q).transpose(0, 1)[None]
        mask = torch.arange(ctx)[None, :] <= torch.arange(cached, ctx)[:, None]
        ref = torch.nn.functional.scaled_dot_product_attention(
            qt, kt.repeat_interleave(2, 1), vt.repeat_interleave(2, 1), attn_mask=mask,
            scale=D ** -0.5)[0].transpose(0, 1).numpy()
        np.testing.assert_allclose(got, ref, rtol=1e-12, atol=1e-12)
        if cached == 0:
            ref_c = torch.nn.functional.scaled_dot_product_attention(
                qt, kt.repeat_interleave(2, 1), vt.repeat_interleave(2, 1), is_causal=True,
                scale=D ** -0.5)[0].transpose(0, 1).numpy()
            np.testing.assert_allclose(got, ref_c, rtol=1e-12, atol=1e-12)
    q1 = rng.standard_normal((1, Hq, D))
    np.testing.assert_allclose(
        mr.paged_rows_f64(q1, k, v, table[None, :], [0], [17], bs, 0.3),
        mr.paged_decode_f64(q1, k, v, table[None, :], [17], bs, 0.3), rtol=0, atol=0)


def test_step_rows_oracle():
    """The step-row oracle on a hand-checked batch: block size 4, a decode token at position
    9 of table [5, 2, 7], a 3-token chunk after 2 cached tokens of table [1], a fresh 2-token
    prompt on table [3]."""
    slots, rows, ctx = mr.step_rows([1, 3, 2], [10, 5, 2], [[5, 2, 7], [1, 6], [3]], 4)
    np.testing.assert_array_equal(slots, [7 * 4 + 1, 4 + 2, 4 + 3, 6 * 4 + 0, 12, 13])
    np.testing.assert_array_equal(rows, [0, 1, 1, 1, 2, 2])
    np.testing.assert_array_equal(ctx, [10, 3, 4, 5, 1, 2])
