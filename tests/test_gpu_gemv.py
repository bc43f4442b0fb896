"""HIP weight-only GEMVs through the C ABI against the oracle.

Tolerance (fp32 accumulation in a different order than the reference): max-abs error
<= 1e-5 * max|y| and rel-L2 <= 1e-5 against the float64 mathematics, and <= 2e-5 against the
reference's own CPU kernel outputs (committed goldens) and the C restatement — inside the
reference tests' own 1e-4 (int8) / 2e-4 (int4) (tests/test_quant.py:90-118).
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
TOL_F64 = 1e-5
TOL_REF = 2e-5


@pytest.fixture(scope="module")
def kg():
    return dict(np.load(GOLDEN / "kernels_golden.npz"))


@pytest.mark.parametrize("M,K,N", [(1, 200, 77), (3, 200, 77), (16, 200, 77), (4, 1024, 96)])
def test_int8_reference_goldens(gpu, kg, M, K, N):
    key = f"i8_M{M}_K{K}_N{N}"
    x, q, s = (kg[key + k] for k in ("_x", "_q", "_s"))
    y = cu.int8_linear(cu.dev(x), cu.dev(q), cu.dev(s))
    cu.assert_rel_close(y, kg[key + "_y"], TOL_REF, key)
    cu.assert_rel_close(y, mr.int8_linear_f64(x, q, s), TOL_F64, key)


@pytest.mark.parametrize("M,K,N,g", [(1, 256, 80, 64), (5, 256, 80, 64), (16, 256, 80, 64),
                                     (4, 1024, 64, 128), (2, 512, 48, 32)])
def test_int4_reference_goldens(gpu, kg, M, K, N, g):
    key = f"i4_M{M}_K{K}_N{N}_g{g}"
    x, nib, s, z = (kg[key + k] for k in ("_x", "_nib", "_s", "_z"))
    y = cu.int4_linear(cu.dev(x), cu.dev(nib), cu.dev(s), cu.dev(z), g)
    cu.assert_rel_close(y, kg[key + "_y"], TOL_REF, key)
    cu.assert_rel_close(y, mr.int4_linear_f64(x, nib, s, z, g), TOL_F64, key)


@pytest.mark.parametrize("M", [1, 2, 3, 4, 5, 8, 16, 17, 33, 64])
@pytest.mark.parametrize("N,K", [(6144, 1024), (1024, 3072), (96, 8192), (130, 448), (200, 4096),
                                 (300, 2048)])
def test_int8_shapes(gpu, M, N, K):
    rng = np.random.default_rng(M * 1000 + N + K)
    x = rng.standard_normal((M, K)).astype(F32)
    q, s = oq.int8_quantize((rng.standard_normal((N, K)) * 0.02).astype(F32))
    y = cu.int8_linear(cu.dev(x), cu.dev(q), cu.dev(s))
    cu.assert_rel_close(y, mr.int8_linear_f64(x, q, s), TOL_F64, f"M={M} N={N} K={K}")
    if M <= 4 and N * K <= 2**23:
        cu.assert_rel_close(y, ocpu.int8_linear(x, q, s), TOL_REF, "vs C restatement")


QWEN = [(4096, 1024), (1024, 2048), (6144, 1024), (1024, 3072)]  # qkv, o, gate_up, down


@pytest.mark.parametrize("M", [1, 2, 4, 16])
@pytest.mark.parametrize("N,K", QWEN)
def test_int4_awq_qwen_shapes(gpu, M, N, K):
    """g128 AWQ linears, activations with 1% outlier channels x20."""
    rng = np.random.default_rng(M * 7919 + N + K)
    w = (rng.standard_normal((N, K)) * 0.02).astype(F32)
    x = rng.standard_normal((M, K)).astype(F32)
    outl = rng.choice(K, K // 100, replace=False)
    x[:, outl] *= 20
    act = np.maximum(np.abs(x).mean(0), 1e-5).astype(F32) ** F32(0.5)
    act = (act / np.sqrt(act.max() * act.min())).astype(F32)
    nib, gs, gz, inv = oq.int4_quantize_pack(w, 128, act)
    y = cu.int4_linear(cu.dev(x), cu.dev(nib), cu.dev(gs), cu.dev(gz), 128, cu.dev(inv))
    cu.assert_rel_close(y, mr.int4_linear_f64(x, nib, gs, gz, 128, inv), TOL_F64, f"M={M} {N}x{K}")
    cu.assert_rel_close(y, ocpu.int4_linear(x, nib, gs, gz, 128, inv), TOL_REF, "vs C restatement")


@pytest.mark.parametrize("M,N,K,g", [(1, 64, 256, 64), (3, 96, 512, 32), (7, 40, 1536, 64),
                                     (16, 128, 2048, 64), (2, 33, 96, 32), (64, 64, 1024, 128),
                                     (20, 256, 4096, 128), (1, 8, 64, 2), (1, 100, 4096, 128),
                                     (2, 70, 2048, 32), (1, 50, 3072, 64)])
def test_int4_group_sizes_and_tails(gpu, M, N, K, g):
    rng = np.random.default_rng(M + N + K + g)
    w = (rng.standard_normal((N, K)) * 0.02).astype(F32)
    x = rng.standard_normal((M, K)).astype(F32)
    nib, gs, gz, _ = oq.int4_quantize_pack(w, g)
    y = cu.int4_linear(cu.dev(x), cu.dev(nib), cu.dev(gs), cu.dev(gz), g)
    cu.assert_rel_close(y, mr.int4_linear_f64(x, nib, gs, gz, g), TOL_F64, f"M={M} {N}x{K} g{g}")


def test_misaligned_inputs_take_generic_path(gpu):
    rng = np.random.default_rng(1)
    K, N = 1024, 64
    xb = torch.from_numpy(rng.standard_normal(K + 1).astype(F32)).cuda()
    x = xb[1:].view(1, K)  # 4-byte offset: not 16-byte aligned
    q, s = oq.int8_quantize((rng.standard_normal((N, K)) * 0.02).astype(F32))
    y = cu.int8_linear(x, cu.dev(q), cu.dev(s))
    cu.assert_rel_close(y, mr.int8_linear_f64(x.cpu().numpy(), q, s), TOL_F64)


def test_torch_op_signatures(gpu):
    """The reference's Python-visible calls: int8_linear(x, q, s) and
    int4_linear(x, nibbles, scale, zero, group_size)."""
    from llmserve.kernels import load_int8_gemv

    k = load_int8_gemv()
    rng = np.random.default_rng(2)
    x = rng.standard_normal((3, 256)).astype(F32)
    q, s = oq.int8_quantize((rng.standard_normal((80, 256)) * 0.02).astype(F32))
    cu.assert_rel_close(k.int8_linear(cu.dev(x), cu.dev(q), cu.dev(s)), mr.int8_linear_f64(x, q, s), TOL_F64)
    nib, gs, gz, _ = oq.int4_quantize_pack((rng.standard_normal((80, 256)) * 0.02).astype(F32), 64)
    y = k.int4_linear(cu.dev(x), cu.dev(nib), cu.dev(gs), cu.dev(gz), 64)
    cu.assert_rel_close(y, mr.int4_linear_f64(x, nib, gs, gz, 64), TOL_F64)
    with pytest.raises(RuntimeError, match="M <= 64"):
        k.int8_linear(torch.zeros(65, 256, device="cuda"), cu.dev(q), cu.dev(s))
    with pytest.raises(RuntimeError, match="K mismatch"):
        k.int8_linear(torch.zeros(2, 128, device="cuda"), cu.dev(q), cu.dev(s))
    with pytest.raises(RuntimeError, match="int4: shapes"):
        k.int4_linear(cu.dev(x), cu.dev(nib), cu.dev(gs), cu.dev(gz), 48)
