"""The allocation-free paged decode (llmserve_paged_attention_decode_int8_noalloc) through the
C ABI: two calls in a row, the second on a smaller batch, each bit-identical to
llmserve_paged_attention_decode_int8 with a caller workspace (the same kernels and split), and
a size past the library's scratch array rejected with an error before anything runs."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

import capi_util as cu
from llmserve._native import capi, check

pytestmark = pytest.mark.gpu


def _case(seed, B, Hq=16, Hk=8, D=128, bs=16, lo=100, hi=3000):
    rng = np.random.default_rng(seed)
    ctx = rng.integers(lo, hi + 1, B).astype(np.int64)
    nblk = [-(-int(c) // bs) for c in ctx]
    total = sum(nblk) + 2
    perm = rng.permutation(total)
    bt = np.zeros((B, max(nblk)), np.int64)
    used = 0
    for b, n in enumerate(nblk):
        bt[b, :n] = perm[used:used + n]
        used += n
    kq = rng.integers(-127, 128, (total * bs, Hk, D), dtype=np.int8)
    vq = rng.integers(-127, 128, (total * bs, Hk, D), dtype=np.int8)
    ks = (rng.random((total * bs, Hk)) * 0.05).astype(np.float32)
    vs = (rng.random((total * bs, Hk)) * 0.05).astype(np.float32)
    q = rng.standard_normal((B, Hq, D)).astype(np.float32)
    qm = (rng.random((Hq, D)) + 0.5).astype(np.float32)
    return [cu.dev(a) for a in (q, kq, vq, ks, vs, bt, ctx, qm)], bs


def _noalloc(q, kq, vq, ks, vs, bt, cl, qm, bs, scale, partition=0):
    B, Hq, D = q.shape
    out = torch.full_like(q, float("nan"))
    check(capi().llmserve_paged_attention_decode_int8_noalloc(
        cu._p(q), cu._p(kq), cu._p(vq), cu._p(ks), cu._p(vs), cu._p(bt), cu._p(cl), cu._p(out), B,
        Hq, kq.shape[1], D, kq.shape[0], bt.shape[1], bs, ctypes.c_float(scale), partition,
        cu._p(qm), cu._stream()))
    return out


def test_noalloc_equals_workspace_entry(gpu):
    for seed, B in ((1, 64), (2, 7)):  # the second call smaller than the first
        (q, kq, vq, ks, vs, bt, cl, qm), bs = _case(seed, B)
        scale = 128 ** -0.5
        got = _noalloc(q, kq, vq, ks, vs, bt, cl, qm, bs, scale)
        want = cu.paged_decode_int8(q, kq, vq, ks, vs, bt, cl, bs, scale, 0, qm)
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"seed {seed}, B={B}"
    # a forced partition size (more partials) still fits and matches
    (q, kq, vq, ks, vs, bt, cl, qm), bs = _case(3, 5)
    got = _noalloc(q, kq, vq, ks, vs, bt, cl, qm, bs, 0.1, 256)
    assert torch.equal(got, cu.paged_decode_int8(q, kq, vq, ks, vs, bt, cl, bs, 0.1, 256, qm))


def test_noalloc_rejects_sizes_past_its_scratch(gpu):
    """A valid call whose partials would not fit the scratch array (a partition of one token
    over 2 x ~3000 tokens) is rejected with an error and writes nothing."""
    L = capi()
    limit = L.llmserve_paged_attention_noalloc_scratch_bytes()
    assert limit > 0
    (q, kq, vq, ks, vs, bt, cl, qm), bs = _case(4, 2, lo=2900, hi=3000)
    need = L.llmserve_paged_attention_workspace_bytes(2, 16, 8, 128, bt.shape[1], bs, 1)
    assert need > limit
    out = torch.full_like(q, 7.0)
    rc = L.llmserve_paged_attention_decode_int8_noalloc(
        cu._p(q), cu._p(kq), cu._p(vq), cu._p(ks), cu._p(vs), cu._p(bt), cu._p(cl), cu._p(out), 2,
        16, 8, 128, kq.shape[0], bt.shape[1], bs, ctypes.c_float(0.1), 1, cu._p(qm), cu._stream())
    torch.cuda.synchronize()
    assert rc != 0 and b"scratch" in L.llmserve_last_error()
    assert bool((out == 7.0).all())
