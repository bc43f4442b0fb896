"""bf16 matrix-core prefill GEMM (Int8Linear's large-M path) through the C ABI.

Two oracles (oracle/math_ref.int8_linear_prefill_f64):
  * with x rounded to bfloat16 (ties to even), the product the kernel computes exactly up to
    its float32 accumulation: rel-L2 <= 2e-6 and max-abs <= 2e-5 * max|y|;
  * the plain weight-only product over float32 x (the reference's dequant GEMM, quant.py:71-72
    and :78-79): the stated bf16 tolerance, rel-L2 <= 5e-3.
At BASELINE config 3 sizes (M = 2048) the float64 oracles run on a seeded subset of rows.
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
TIGHT_L2, TIGHT_MAX, BF16_L2 = 2e-6, 2e-5, 5e-3


def rel_l2(got, ref):
    got = np.asarray(got, np.float64)
    return float(np.linalg.norm(got - ref) / np.linalg.norm(ref))


def check(y, x, q, s, rows=None):
    y = y.cpu().numpy()
    if rows is not None:
        x, y = x[rows], y[rows]
    exact = mr.int8_linear_prefill_f64(x, q, s)
    assert rel_l2(y, exact) <= TIGHT_L2, rel_l2(y, exact)
    assert np.abs(y - exact).max() <= TIGHT_MAX * np.abs(exact).max()
    plain = mr.int8_linear_prefill_f64(x, q, s, round_x=False)
    err = rel_l2(y, plain)
    assert err <= BF16_L2, err
    return err


def make(seed, M, N, K):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((M, K)).astype(F32)
    q, s = oq.int8_quantize((rng.standard_normal((N, K)) * 0.02).astype(F32))
    return x, q, s


@pytest.mark.parametrize("M,N,K", [(1, 1, 64), (37, 100, 64), (256, 256, 128), (300, 520, 192),
                                   (513, 257, 320), (64, 2048, 1024), (200, 300, 4096),
                                   (2048, 6000, 128)])  # 192-wide tiles, a 48-column last one
def test_shapes(gpu, M, N, K):
    x, q, s = make(M * 7 + N, M, N, K)
    y = cu.int8_linear_prefill(cu.dev(x), cu.dev(q), cu.dev(s))
    check(y, x, q, s)


@pytest.mark.parametrize("N,K", [(6144, 2048), (16384, 2048), (2048, 8192)])
def test_config3_shapes(gpu, N, K):
    """BASELINE config 3 (SmolLM2-1.7B qkv, gate_up, down) at M = 2048; 96 seeded rows checked
    against float64, every row against the torch bf16 product of the same operands."""
    M = 2048
    g = torch.Generator(device="cuda").manual_seed(N + K)
    xd = torch.randn(M, K, device="cuda", generator=g)
    wd = torch.randn(N, K, device="cuda", generator=g) * 0.02
    q, s = cu.int8_quantize(wd)
    y = cu.int8_linear_prefill(xd, q, s)
    rows = np.random.default_rng(N).choice(M, 96, replace=False)
    err = check(y, xd.cpu().numpy(), q.cpu().numpy(), s.cpu().numpy(), rows)
    print(f"config 3 N={N} K={K}: rel-L2 vs fp32-x weight-only product {err:.2e}")
    # all rows: float32 GEMM of the same bf16-rounded operands (torch, fp32 accumulate)
    ref = (xd.to(torch.bfloat16).float() @ q.float().t()) * s[None, :]
    assert torch.linalg.norm(y - ref) / torch.linalg.norm(ref) <= 1e-5


def test_module_prefill_and_dequant_agree(gpu):
    from torch import nn

    from llmserve.quant import Int8Linear

    torch.manual_seed(0)
    lin = nn.Linear(512, 384, bias=True)
    m = Int8Linear(lin, device="cuda")
    x = torch.randn(2, 150, 512, device="cuda")
    y = m(x)  # auto: 300 rows -> prefill GEMM
    Int8Linear.kernel = "dequant"
    try:
        y_ref = m(x)
    finally:
        Int8Linear.kernel = "auto"
    assert y.shape == (2, 150, 384)
    assert (torch.linalg.norm(y - y_ref) / torch.linalg.norm(y_ref)).item() <= BF16_L2


def test_rejects_bad_k(gpu):
    x = torch.randn(4, 96, device="cuda")
    q = torch.zeros(8, 96, dtype=torch.int8, device="cuda")
    s = torch.ones(8, device="cuda")
    with pytest.raises(RuntimeError, match="multiple of 64"):
        cu.int8_linear_prefill(x, q, s)
