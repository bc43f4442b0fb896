"""HIP quantizers through the C ABI: bit-exact against the torch-CPU golden vectors and the
numpy oracle, at fixture size and at the BASELINE shapes."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import capi_util as cu
from conftest import GOLDEN
from oracle import quant as oq

pytestmark = pytest.mark.gpu
F32 = np.float32


@pytest.fixture(scope="module")
def gold():
    return dict(np.load(GOLDEN / "quant_golden.npz"))


def bits(t):
    return np.asarray(t.cpu() if isinstance(t, torch.Tensor) else t, F32).view(np.uint32)


def test_int8_golden(gpu, gold):
    q, s = cu.int8_quantize(cu.dev(gold["int8_w"]))
    np.testing.assert_array_equal(q.cpu().numpy(), gold["int8_q"])
    np.testing.assert_array_equal(bits(s), bits(gold["int8_scale"]))


@pytest.mark.parametrize("group", [32, 64, 128])
def test_int4_golden(gpu, gold, group):
    nib, gs, gz, inv = cu.int4_quantize(cu.dev(gold[f"int4_g{group}_w"]), group)
    assert inv is None
    np.testing.assert_array_equal(nib.cpu().numpy(), gold[f"int4_g{group}_nib"])
    np.testing.assert_array_equal(bits(gs), bits(gold[f"int4_g{group}_scale"]))
    np.testing.assert_array_equal(bits(gz), bits(gold[f"int4_g{group}_zero"]))


def test_awq_fold_golden(gpu, gold):
    g = int(gold["awq_group"])
    nib, gs, gz, inv = cu.int4_quantize(cu.dev(gold["awq_w"]), g, cu.dev(gold["awq_s"]))
    np.testing.assert_array_equal(nib.cpu().numpy(), gold["awq_nib"])
    np.testing.assert_array_equal(bits(gs), bits(gold["awq_scale"]))
    np.testing.assert_array_equal(bits(gz), bits(gold["awq_zero"]))
    np.testing.assert_array_equal(bits(inv), bits(gold["awq_inv"]))


def test_kv_golden(gpu, gold):
    x = cu.dev(gold["kv_x"])
    T, Hk, D = x.shape
    slots = torch.arange(T, device=x.device)
    data = torch.zeros(T, Hk, D, dtype=torch.int8, device=x.device)
    scale = torch.zeros(T, Hk, device=x.device)
    cu.kv_quantize_write(x, slots, data, scale)
    np.testing.assert_array_equal(data.cpu().numpy(), gold["kv_q"])
    np.testing.assert_array_equal(bits(scale), bits(gold["kv_s"]))
    cu.kv_quantize_write(x, slots, data, scale, cu.dev(gold["kv_smooth"]))
    np.testing.assert_array_equal(data.cpu().numpy(), gold["kv_q_smoothed"])
    np.testing.assert_array_equal(bits(scale), bits(gold["kv_s_smoothed"]))


@pytest.mark.parametrize("N,K", [(6144, 1024), (2048, 8192), (77, 200)])
def test_int8_baseline_shapes(gpu, N, K):
    rng = np.random.default_rng(N + K)
    w = (rng.standard_normal((N, K)) * 0.02).astype(F32)
    q, s = cu.int8_quantize(cu.dev(w))
    qo, so = oq.int8_quantize(w)
    np.testing.assert_array_equal(q.cpu().numpy(), qo)
    np.testing.assert_array_equal(bits(s), bits(so))


@pytest.mark.parametrize("N,K,group", [(4096, 1024, 128), (1024, 2048, 128), (6144, 1024, 128),
                                       (1024, 3072, 128), (80, 256, 64), (48, 96, 32)])
def test_int4_awq_baseline_shapes(gpu, N, K, group):
    rng = np.random.default_rng(N * 7 + K)
    w = (rng.standard_normal((N, K)) * 0.02).astype(F32)
    act = np.abs(rng.standard_normal(K)).astype(F32) + F32(0.1)
    act[rng.choice(K, max(1, K // 100), replace=False)] *= 20
    for a in (None, act):
        nib, gs, gz, inv = cu.int4_quantize(cu.dev(w), group, None if a is None else cu.dev(a))
        no, so, zo, io = oq.int4_quantize_pack(w, group, a)
        np.testing.assert_array_equal(nib.cpu().numpy(), no)
        np.testing.assert_array_equal(bits(gs), bits(so))
        np.testing.assert_array_equal(bits(gz), bits(zo))
        if a is not None:
            np.testing.assert_array_equal(bits(inv), bits(io))


def test_kv_write_scatter_and_bounds(gpu):
    """Random slot permutation with smoothing at the Qwen3 head shape; out-of-range slots are
    skipped and leave the cache untouched."""
    rng = np.random.default_rng(3)
    T, Hk, D, S = 200, 8, 128, 512
    x = rng.standard_normal((T, Hk, D)).astype(F32)
    x[..., 5] *= 30
    sm = np.abs(rng.standard_normal((Hk, D))).astype(F32) + F32(0.5)
    slots = rng.permutation(S)[:T].astype(np.int64)
    slots[7], slots[11] = -1, S  # invalid: skipped
    data = torch.full((S, Hk, D), 99, dtype=torch.int8, device="cuda")
    scale = torch.full((S, Hk), -1.0, device="cuda")
    cu.kv_quantize_write(cu.dev(x), cu.dev(slots), data, scale, cu.dev(sm))
    qo, so = oq.kv_quantize(oq.kv_smooth(x, sm))
    d, s = data.cpu().numpy(), scale.cpu().numpy()
    ok = (slots >= 0) & (slots < S)
    np.testing.assert_array_equal(d[slots[ok]], qo[ok])
    np.testing.assert_array_equal(bits(s[slots[ok]]), bits(so[ok]))
    untouched = np.setdiff1d(np.arange(S), slots[ok])
    assert (d[untouched] == 99).all() and (s[untouched] == -1.0).all()


def test_torch_ops_match_capi(gpu):
    from llmserve.kernels import load_quant

    rng = np.random.default_rng(9)
    w = cu.dev((rng.standard_normal((256, 512)) * 0.02).astype(F32))
    q1, s1 = load_quant().int8_quantize(w)
    q2, s2 = cu.int8_quantize(w)
    assert torch.equal(q1, q2) and torch.equal(s1, s2)
    a = cu.dev(np.abs(rng.standard_normal(512)).astype(F32) + F32(0.2))
    r1 = load_quant().int4_quantize(w, 128, a)
    r2 = cu.int4_quantize(w, 128, a)
    for t1, t2 in zip(r1, r2):
        assert torch.equal(t1, t2)
