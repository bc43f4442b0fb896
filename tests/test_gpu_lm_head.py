"""fp32 LM head on activation fragments (llmserve_lm_head_f32_xfrag) against float64.

x and W are each split into bf16 hi + mid + lo (~2^-26 relative) and the six products whose
weight reaches 2^-16 of the leading one accumulate in fp32, so each product is the fp32
product up to fp32's own rounding (the reference's fp32 F.linear); the bound here is
max-abs <= 2e-5 * max|ref| and rel-L2 <= 2e-5 against x . W^T in float64. Shapes cover a
partial row tile (rows past M are zero fragments and are not stored), several 64-row passes
plus a remainder, vocab sizes that are not multiples of 64 or 4 (clamped loads, scalar
stores), and the Qwen3-0.6B head (V = 151936, K = 1024) at 8 and 64 rows. The 1-4 row head
(llmserve_lm_head_f32, an fp32 GEMV) is checked against float64 at 1e-5. The decode step's use of it is checked against the step oracle in test_gpu_step.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import capi_util as cu

pytestmark = pytest.mark.gpu
TOL = 2e-5


def _lm_head(xf, w, M):
    V, K = w.shape
    y = torch.empty(M, V, dtype=torch.float32, device=w.device)
    cu.check(cu.capi().llmserve_lm_head_f32_xfrag(cu._p(xf), cu._p(w), cu._p(y), M, V, K,
                                                   cu._stream()))
    return y


@pytest.mark.parametrize("M,V,K", [(5, 1000, 256), (64, 4096, 1024), (70, 777, 512),
                                   (130, 2050, 384), (16, 4099, 128),
                                   (8, 151936, 1024), (64, 151936, 1024)])  # Qwen3-0.6B head
def test_lm_head_f32_matches_f64(gpu, M, V, K):
    rng = np.random.default_rng(M * 7 + V)
    x = rng.standard_normal((M, K)).astype(np.float32)
    w = (0.02 * rng.standard_normal((V, K))).astype(np.float32)
    xd, wd = cu.dev(x), cu.dev(w)
    y = _lm_head(cu.split_fragments(xd), wd, M)
    ref = x.astype(np.float64) @ w.astype(np.float64).T
    cu.assert_rel_close(y, ref, TOL, f"M{M} V{V} K{K}")


def test_lm_head_op_and_rejects(gpu):
    from llmserve.kernels import load_fused_ops

    fo = load_fused_ops()
    rng = np.random.default_rng(3)
    x = cu.dev(rng.standard_normal((20, 256)).astype(np.float32))
    w = cu.dev(rng.standard_normal((300, 256)).astype(np.float32))
    xf = cu.split_fragments(x)
    y = fo.lm_head_f32_xfrag(xf, w, 20)
    assert torch.equal(y, _lm_head(xf, w, 20))
    with pytest.raises(RuntimeError, match="fewer than M rows"):
        fo.lm_head_f32_xfrag(xf[:100], w, 20)
    with pytest.raises(RuntimeError, match="multiple of 128"):
        _lm_head(xf, cu.dev(np.zeros((300, 200), np.float32)), 20)


@pytest.mark.parametrize("M,V,K", [(1, 151936, 1024), (2, 777, 512), (3, 4099, 256),
                                   (4, 151936, 1024), (4, 33, 1024)])
def test_lm_head_gemv_rows_matches_f64(gpu, M, V, K):
    """The 1-4 row fp32 head (llmserve_lm_head_f32): exact fp32 products and sums, so 1e-5 of
    float64 (a few ulps of the row sums); rows past V and groups that do not fill a
    wavefront's four rows are covered by the odd V."""
    rng = np.random.default_rng(M * 13 + V)
    x = rng.standard_normal((M, K)).astype(np.float32)
    w = (0.02 * rng.standard_normal((V, K))).astype(np.float32)
    xd, wd = cu.dev(x), cu.dev(w)
    y = torch.empty(M, V, dtype=torch.float32, device="cuda")
    cu.check(cu.capi().llmserve_lm_head_f32(cu._p(xd), cu._p(wd), cu._p(y), M, V, K, cu._stream()))
    ref = x.astype(np.float64) @ w.astype(np.float64).T
    cu.assert_rel_close(y, ref, 1e-5, f"gemv head M{M} V{V} K{K}")


def test_lm_head_gemv_op_and_rejects(gpu):
    from llmserve.kernels import load_fused_ops

    fo = load_fused_ops()
    x = torch.randn(2, 1024, device="cuda")
    w = torch.randn(500, 1024, device="cuda")
    torch.testing.assert_close(fo.lm_head_f32(x, w), x.double().mm(w.double().t()).float(),
                               rtol=1e-5, atol=1e-4)
    with pytest.raises(RuntimeError, match="1 to 4 rows"):
        fo.lm_head_f32(torch.randn(5, 1024, device="cuda"), w)
    with pytest.raises(RuntimeError, match="256, 512 or 1024"):
        fo.lm_head_f32(torch.randn(1, 2048, device="cuda"), torch.randn(10, 2048, device="cuda"))
