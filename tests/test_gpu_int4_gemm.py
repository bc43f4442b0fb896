"""int4 weight-only linear for M > 16 on the matrix cores (Int4Linear's large-M branch,
reference quant.py:141-142) through the C ABI, against the float64 oracle.

Tolerance: max-abs error <= 2e-5 * max|y| and rel-L2 <= 2e-5 against the float64 mathematics.
x' = x * inv_act_scale is carried as two bf16 terms (xh + xl equals x' to 2^-18 relative) and
every matrix-core product is exact, so the error is a few 1e-6; 2e-5 stays inside the
reference tests' own 2e-4 for int4 (tests/test_quant.py:116-118).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import capi_util as cu
from oracle import math_ref as mr
from oracle import quant as oq

pytestmark = pytest.mark.gpu
F32 = np.float32
TOL = 2e-5


def _case(M, N, K, g, seed, awq=True, outliers=True):
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((N, K)) * 0.02).astype(F32)
    x = rng.standard_normal((M, K)).astype(F32)
    if outliers:
        x[:, rng.choice(K, max(1, K // 100), replace=False)] *= 20
    act = None
    if awq:
        act = np.maximum(np.abs(x).mean(0), 1e-5).astype(F32) ** F32(0.5)
        act = (act / np.sqrt(act.max() * act.min())).astype(F32)
    nib, gs, gz, inv = oq.int4_quantize_pack(w, g, act)
    return x, nib, gs, gz, inv


QWEN = [(4096, 1024), (1024, 2048), (6144, 1024), (1024, 3072)]  # qkv, o, gate_up, down


@pytest.mark.parametrize("M", [17, 32, 64])
@pytest.mark.parametrize("N,K", QWEN)
def test_int4_gemm_qwen_shapes(gpu, M, N, K):
    """Config 5's batch-64 decode linears (and partial row tiles), g128 AWQ."""
    x, nib, gs, gz, inv = _case(M, N, K, 128, M * 31 + N + K)
    y = cu.int4_linear_gemm(cu.dev(x), cu.dev(nib), cu.dev(gs), cu.dev(gz), 128, cu.dev(inv))
    cu.assert_rel_close(y, mr.int4_linear_f64(x, nib, gs, gz, 128, inv), TOL, f"M={M} {N}x{K}")


@pytest.mark.parametrize("M,N,K,g", [(100, 48, 256, 128), (33, 16, 128, 128), (70, 160, 1536, 256),
                                     (1, 32, 512, 128), (129, 64, 384, 384), (257, 80, 640, 128)])
def test_int4_gemm_tails_and_groups(gpu, M, N, K, g):
    """Row tails (M not a multiple of 32), output-tile tails, groups of several 128 blocks,
    split counts that do not divide the blocks, no AWQ scale."""
    x, nib, gs, gz, inv = _case(M, N, K, g, M + N + K + g, awq=(M % 2 == 0))
    y = cu.int4_linear_gemm(cu.dev(x), cu.dev(nib), cu.dev(gs), cu.dev(gz), g,
                            None if inv is None else cu.dev(inv))
    cu.assert_rel_close(y, mr.int4_linear_f64(x, nib, gs, gz, g, inv), TOL, f"M={M} {N}x{K} g{g}")


def test_int4_gemm_matches_gemv(gpu):
    """The large-M kernel and the GEMV agree on the same rows (both within the fp32 bound)."""
    x, nib, gs, gz, inv = _case(16, 6144, 1024, 128, 7)
    args = (cu.dev(nib), cu.dev(gs), cu.dev(gz), 128, cu.dev(inv))
    a = cu.int4_linear_gemm(cu.dev(x), *args).cpu().numpy()
    b = cu.int4_linear(cu.dev(x), *args).cpu().numpy()
    assert np.abs(a - b).max() <= 4e-5 * np.abs(b).max()


def test_int4_gemm_rejects_bad_shapes(gpu):
    x, nib, gs, gz, inv = _case(20, 48, 256, 64, 3, awq=False)
    with pytest.raises(RuntimeError, match="multiples of 128"):
        cu.int4_linear_gemm(cu.dev(x), cu.dev(nib), cu.dev(gs), cu.dev(gz), 64)


def test_int4linear_large_batch_uses_gemm(gpu):
    """Int4Linear.forward above max_fused_rows runs the matrix-core kernel; its result equals
    the reference algorithm (dequantize + GEMM) to the stated bound."""
    from llmserve.quant import Int4Linear

    rng = np.random.default_rng(11)
    lin = torch.nn.Linear(1024, 4096, bias=False)
    with torch.no_grad():
        lin.weight.copy_(torch.from_numpy((rng.standard_normal((4096, 1024)) * 0.02).astype(F32)))
    act = torch.from_numpy((np.abs(rng.standard_normal(1024)) + 0.5).astype(F32))
    q = Int4Linear(lin, 128, act, device="cuda")
    x = torch.from_numpy(rng.standard_normal((64, 1024)).astype(F32)).cuda()
    y = q(x)
    q.kernel = "aten"
    ref = q(x)
    err = (y - ref).abs().max().item() / ref.abs().max().item()
    assert err < 2e-5, err
