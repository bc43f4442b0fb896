"""Pins of the C restatement of the reference's CPU kernels (oracle/cpu_kernels.c), CPU only.

* against the float64 mathematics (oracle/math_ref.py) at the reference tests' tolerances
  (tests/test_quant.py:90-118: 1e-4 int8, 2e-4 int4; tests/test_attention.py:146-152: 1e-5);
* against outputs of the reference's own compiled kernels committed in
  tests/golden/kernels_golden.npz, and live against oracle/_ref when it is built;
* split-context invariance: every partition size gives the same decode output
  (reference tests/test_attention.py:84-101).
"""

from __future__ import annotations

import numpy as np
import pytest

from conftest import GOLDEN
from oracle import cpu as ocpu
from oracle import math_ref as mr
from oracle import quant as oq

F32 = np.float32


@pytest.fixture(scope="module")
def kg():
    return dict(np.load(GOLDEN / "kernels_golden.npz"))


def close(a, b, rtol, atol):
    np.testing.assert_allclose(np.asarray(a, np.float64), np.asarray(b, np.float64), rtol=rtol, atol=atol)


@pytest.mark.parametrize("M,K,N", [(1, 200, 77), (3, 200, 77), (16, 200, 77), (4, 1024, 96)])
def test_int8_linear_vs_reference_kernel_and_f64(kg, M, K, N):
    key = f"i8_M{M}_K{K}_N{N}"
    x, q, s, y_ref = kg[key + "_x"], kg[key + "_q"], kg[key + "_s"], kg[key + "_y"]
    y = ocpu.int8_linear(x, q, s)
    close(y, y_ref, 2e-6, 2e-6)  # same algorithm; only the fp32 summation order differs
    close(y, mr.int8_linear_f64(x, q, s), 1e-4, 1e-4)


@pytest.mark.parametrize("M,K,N,g", [(1, 256, 80, 64), (5, 256, 80, 64), (16, 256, 80, 64),
                                     (4, 1024, 64, 128), (2, 512, 48, 32)])
def test_int4_linear_vs_reference_kernel_and_f64(kg, M, K, N, g):
    key = f"i4_M{M}_K{K}_N{N}_g{g}"
    x, nib, s, z, y_ref = (kg[key + k] for k in ("_x", "_nib", "_s", "_z", "_y"))
    y = ocpu.int4_linear(x, nib, s, z, g)
    close(y, y_ref, 2e-6, 2e-6)
    close(y, mr.int4_linear_f64(x, nib, s, z, g), 2e-4, 2e-4)


def _pa_case(kg, name):
    bs, sc = kg[f"{name}_meta"]
    return dict(q=kg[f"{name}_q"], k_cache=kg[f"{name}_kq"], v_cache=kg[f"{name}_vq"],
                k_scale=kg[f"{name}_ks"], v_scale=kg[f"{name}_vs"], block_tables=kg[f"{name}_bt"],
                context_lens=kg[f"{name}_cl"], block_size=int(bs), scale=float(sc))


@pytest.mark.parametrize("name,parts", [("pa_small", [0, 4, 8, 10000]), ("pa_d128", [0, 32, 64]),
                                        ("pa_g1", [0, 16])])
def test_paged_decode_vs_reference_kernel_and_f64(kg, name, parts):
    c = _pa_case(kg, name)
    kd = mr.kv_dequantize(c["k_cache"], c["k_scale"])
    vd = mr.kv_dequantize(c["v_cache"], c["v_scale"])
    ref64 = mr.paged_decode_f64(c["q"], kd, vd, c["block_tables"], c["context_lens"],
                                c["block_size"], c["scale"])
    outs = []
    for p in parts:
        o = ocpu.paged_decode_int8(**c, partition_size=p)
        close(o, kg[f"{name}_out_p{p}"], 2e-6, 2e-6)
        close(o, ref64, 1e-5, 1e-5)
        outs.append(o)
    for o in outs[1:]:
        close(o, outs[0], 1e-5, 1e-5)


def test_paged_decode_smoothing_fold_is_q_times_s():
    """q_mult folds the smoothing product into q before the dot (attention.py:243-244)."""
    rng = np.random.default_rng(5)
    B, Hq, Hk, D, bs = 3, 4, 2, 32, 4
    kc = rng.standard_normal((64, Hk, D)).astype(F32)
    kc[..., 3] *= 40.0
    vc = rng.standard_normal((64, Hk, D)).astype(F32)
    sm = np.sqrt(np.abs(kc).max(0)).astype(F32)
    sm = (sm / sm.mean(-1, keepdims=True)).astype(F32)
    kq, ks = oq.kv_quantize(oq.kv_smooth(kc, sm))
    vq, vs = oq.kv_quantize(vc)
    bt = rng.permutation(16).reshape(2, 8)[:, :5].repeat(1, 0)
    bt = np.concatenate([bt, bt[:1]]).astype(np.int64)
    cl = np.array([17, 20, 5], np.int64)
    q = rng.standard_normal((B, Hq, D)).astype(F32)
    q_mult = np.repeat(sm, Hq // Hk, axis=0)
    o = ocpu.paged_decode_int8(q, kq, vq, ks, vs, bt, cl, bs, D ** -0.5, 0, q_mult)
    ref = mr.paged_decode_f64(oq.q_smooth(q, q_mult), mr.kv_dequantize(kq, ks),
                              mr.kv_dequantize(vq, vs), bt, cl, bs, D ** -0.5)
    close(o, ref, 1e-5, 1e-5)


@pytest.mark.skipif(not ocpu.ref_available(), reason="oracle/_ref not built (needs /root/reference)")
def test_live_against_reference_build():
    import torch

    gemv = ocpu.ref_module("llmserve_int8_gemv")
    pa = ocpu.ref_module("llmserve_paged_attention")
    rng = np.random.default_rng(11)
    x = rng.standard_normal((4, 768)).astype(F32)
    q, s = oq.int8_quantize((rng.standard_normal((130, 768)) * 0.02).astype(F32))
    close(ocpu.int8_linear(x, q, s), gemv.int8_linear(*map(torch.from_numpy, (x, q, s))).numpy(),
          2e-6, 2e-6)
    nib, gs, gz, _ = oq.int4_quantize_pack((rng.standard_normal((96, 768)) * 0.02).astype(F32), 128)
    close(ocpu.int4_linear(x, nib, gs, gz, 128),
          gemv.int4_linear(*map(torch.from_numpy, (x, nib, gs, gz)), 128).numpy(), 2e-6, 2e-6)
    bs = 16  # 32 blocks of 16 slots; each table holds 8 blocks = 128 tokens
    kc = rng.standard_normal((32 * bs, 2, 64)).astype(F32)
    kq, ks = oq.kv_quantize(kc)
    vq, vs = oq.kv_quantize(rng.standard_normal((32 * bs, 2, 64)).astype(F32))
    bt = rng.permutation(32).reshape(4, 8).astype(np.int64)
    cl = np.array([100, 3, 128, 64], np.int64)
    qq = rng.standard_normal((4, 6, 64)).astype(F32)
    for p in (0, 16):
        mine = ocpu.paged_decode_int8(qq, kq, vq, ks, vs, bt, cl, bs, 0.125, p)
        theirs = pa.paged_attention_decode_int8(*map(torch.from_numpy, (qq, kq, vq, ks, vs, bt, cl)),
                                                bs, 0.125, p).numpy()
        close(mine, theirs, 2e-6, 2e-6)


def test_fp32_decode_golden_matches_f64():
    """The reference's compiled fp32-cache decode (committed outputs) agrees with the float64
    attention at every forced partition size: pins the fixture the GPU kernel is held to."""
    from conftest import GOLDEN
    from oracle import math_ref as mr

    g = dict(np.load(GOLDEN / "attention_f32_golden.npz"))
    for name in ("f32_small", "f32_d128", "f32_g1"):
        bs, sc = g[f"{name}_meta"]
        ref = mr.paged_decode_f64(g[f"{name}_q"], g[f"{name}_k"], g[f"{name}_v"], g[f"{name}_bt"],
                                  g[f"{name}_cl"], int(bs), float(sc))
        outs = [k for k in g if k.startswith(f"{name}_out_p")]
        assert outs
        for k in outs:
            err = np.abs(g[k] - ref).max() / np.abs(ref).max()
            assert err < 2e-6, (k, err)
