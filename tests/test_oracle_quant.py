"""Pins of the numpy quantizer restatement (oracle/quant.py), CPU only.

* bit-exact against torch-CPU golden vectors (tests/golden/quant_golden.npz): random rows
  plus ties, zero/constant rows, subnormal and huge values, an outlier, the AWQ fold;
* hand-built cases whose answer is fixed by arithmetic (Python's round is half-to-even);
* the round-trip bound |deq - w| <= scale / 2 (reference tests/test_quant.py:21,
  tests/test_attention.py:114-122);
* mutation checks: plausible mistakes planted in a copy of the oracle must fail the pins.
"""

from __future__ import annotations

import numpy as np
import pytest

from conftest import GOLDEN
from oracle import quant as oq

F32 = np.float32


@pytest.fixture(scope="module")
def gold():
    return dict(np.load(GOLDEN / "quant_golden.npz"))


def bits(a):
    return np.asarray(a, F32).view(np.uint32)


def test_int8_matches_torch_golden(gold):
    q, s = oq.int8_quantize(gold["int8_w"])
    np.testing.assert_array_equal(q, gold["int8_q"])
    np.testing.assert_array_equal(bits(s), bits(gold["int8_scale"]))


@pytest.mark.parametrize("group", [32, 64, 128])
def test_int4_matches_torch_golden(gold, group):
    nib, s, z, inv = oq.int4_quantize_pack(gold[f"int4_g{group}_w"], group)
    assert inv is None
    np.testing.assert_array_equal(nib, gold[f"int4_g{group}_nib"])
    np.testing.assert_array_equal(bits(s), bits(gold[f"int4_g{group}_scale"]))
    np.testing.assert_array_equal(bits(z), bits(gold[f"int4_g{group}_zero"]))


def test_awq_fold_matches_torch_golden(gold):
    g = int(gold["awq_group"])
    nib, s, z, inv = oq.int4_quantize_pack(gold["awq_w"], g, gold["awq_s"])
    np.testing.assert_array_equal(nib, gold["awq_nib"])
    np.testing.assert_array_equal(bits(s), bits(gold["awq_scale"]))
    np.testing.assert_array_equal(bits(z), bits(gold["awq_zero"]))
    np.testing.assert_array_equal(bits(inv), bits(gold["awq_inv"]))


def test_awq_search_picks_torch_alpha(gold):
    s, alpha = oq.awq_search_scale(gold["awq_w"], gold["awq_x"], int(gold["awq_group"]))
    assert alpha == pytest.approx(float(gold["awq_alpha"]))
    # same alpha -> the same candidate vector up to the reduction order of mean|x| and the
    # last ulps of pow() in the two libraries (bits of s are not a contract: packing is
    # bit-exact *given* s, test_awq_fold_matches_torch_golden)
    np.testing.assert_allclose(s, gold["awq_s"], rtol=2e-6, atol=0)


def test_kv_matches_torch_golden(gold):
    q, s = oq.kv_quantize(gold["kv_x"])
    np.testing.assert_array_equal(q, gold["kv_q"])
    np.testing.assert_array_equal(bits(s), bits(gold["kv_s"]))
    qs, ss = oq.kv_quantize(oq.kv_smooth(gold["kv_x"], gold["kv_smooth"]))
    np.testing.assert_array_equal(qs, gold["kv_q_smoothed"])
    np.testing.assert_array_equal(bits(ss), bits(gold["kv_s_smoothed"]))


def test_int8_hand_built_ties_and_clamps():
    # amax 127 -> scale exactly 1; k + 0.5 rounds half to even (Python's round)
    vals = [127.0, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 126.5, -126.5, 3.4999, -3.5001]
    q, s = oq.int8_quantize(np.array([vals], F32))
    assert s[0] == F32(1.0)
    assert q[0].tolist() == [round(v) for v in vals]
    # zero row: scale clamps to float32(1e-8), q = 0
    q, s = oq.int8_quantize(np.zeros((1, 16), F32))
    assert s[0] == F32(1e-8) and not q.any()


def test_int4_hand_built():
    g = 8
    w = np.array([[0.25] * g, [0, 15, 0.5, 1.5, 2.5, 13.5, 14.5, 7.0]], F32)
    q, s, z = oq.int4_quantize(w.reshape(1, -1), g)
    # constant group: scale 1e-8, q 0, zero = 0.25 + 8e-8 in float32
    assert s[0, 0] == F32(1e-8) and not q[0, :g].any()
    assert z[0, 0] == F32(F32(0.25) + F32(8) * F32(1e-8))
    # range 15 -> scale 1; ties to even
    assert s[0, 1] == F32(1.0) and z[0, 1] == F32(8.0)
    assert q[0, g:].tolist() == [0, 15, 0, 2, 2, 14, 14, 7]
    # nibble order: even channel low, odd channel high
    assert oq.pack_nibbles(np.array([[1, 2, 3, 4, 15, 0]])).tolist() == [[0x21, 0x43, 0x0F]]
    np.testing.assert_array_equal(oq.unpack_nibbles(oq.pack_nibbles(q)), q)


def test_kv_hand_built():
    x = np.zeros((3, 1, 8), F32)
    x[1, 0] = [127.0, 0.5, 1.5, -2.5, 3.5, 0, 0, 0]
    q, s = oq.kv_quantize(x)
    # zero row: clamp first, then divide -> 1e-8 / 127 (not 1e-8 as for weights)
    assert s[0, 0] == F32(F32(1e-8) / F32(127.0))
    assert s[1, 0] == F32(1.0) and q[1, 0].tolist() == [127, 0, 2, -2, 4, 0, 0, 0]


@pytest.mark.parametrize("seed", [0, 1])
def test_roundtrip_bound(seed):
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((64, 192)) * 0.02).astype(F32)
    q, s = oq.int8_quantize(w)
    err = np.abs(oq.int8_dequantize(q, s) - w)
    assert (err <= s[:, None] / 2 * (1 + 1e-6) + 1e-12).all()
    x = rng.standard_normal((20, 4, 32)).astype(F32)
    kq, ks = oq.kv_quantize(x)
    assert (np.abs(kq * ks[..., None] - x) <= ks[..., None] / 2 * (1 + 1e-6)).all()
    nib, gs, gz, _ = oq.int4_quantize_pack(w, 64)
    deq = oq.int4_dequantize(nib, gs, gz, 64)
    assert (np.abs(deq - w).reshape(64, 3, 64) <= gs[..., None] / 2 * (1 + 1e-5) + 1e-9).all()


# ---- mutation checks: plausible mistakes must fail the pins --------------------------------

def _int8_reciprocal(w):
    w = np.asarray(w, F32)
    scale = np.maximum(np.abs(w).max(1) / F32(127), F32(1e-8)).astype(F32)
    inv = (F32(1) / scale).astype(F32)
    return np.clip(np.rint(w * inv[:, None]), -127, 127).astype(np.int8), scale


def _int8_half_up(w):
    w = np.asarray(w, F32)
    scale = np.maximum(np.abs(w).max(1) / F32(127), F32(1e-8)).astype(F32)
    return np.clip(np.floor(w / scale[:, None] + F32(0.5)), -127, 127).astype(np.int8), scale


def _kv_divide_then_clamp(x):
    x = np.asarray(x, F32)
    s = np.maximum(np.abs(x).max(-1) / F32(127), F32(1e-8)).astype(F32)
    return np.clip(np.rint(x / s[..., None]), -127, 127).astype(np.int8), s


def _int4_zero_fused(w, group):
    q, s, z = oq.int4_quantize(w, group)
    mn = np.asarray(w, F32).reshape(w.shape[0], -1, group).min(-1)
    z2 = (mn.astype(np.float64) + 8.0 * s.astype(np.float64) * (1 + 2**-20)).astype(F32)
    return q, s, z2


def test_mutations_fail_the_pins(gold):
    w = gold["int8_w"]
    q_ok = gold["int8_q"]
    assert not np.array_equal(_int8_half_up(w)[0], q_ok)
    # a reciprocal multiply instead of IEEE division changes the near-tie rows
    assert not np.array_equal(_int8_reciprocal(w)[0], q_ok)
    assert not np.array_equal(bits(_kv_divide_then_clamp(gold["kv_x"])[1]), bits(gold["kv_s"]))
    _, _, z2 = _int4_zero_fused(gold["int4_g64_w"], 64)
    assert not np.array_equal(bits(z2), bits(gold["int4_g64_zero"]))
    # swapped nibble order
    q4 = oq.unpack_nibbles(gold["int4_g32_nib"])
    swapped = (q4[:, 1::2].astype(np.uint8) | (q4[:, 0::2].astype(np.uint8) << 4))
    assert not np.array_equal(swapped, gold["int4_g32_nib"])
