"""The drop-in modules on the GPU, through their own dispatch: Int8Linear's GEMV rows,
Int4Linear's GEMV and packed matrix-core rows, the product's AWQ search, and
quantize_model + collect_linear_inputs on a small model.

Tolerances: linears within 1e-5 of the float64 product over the oracle's dequantized weight
(max-abs relative to max|y| and rel-L2), 2e-5 for the packed matrix-core kernel (TOL_MC);
quantizer buffers bit-exact with the oracle given the scale; the AWQ search picks the golden alpha (computed with torch's CPU ops, the reference's
arithmetic) and a scale within 2e-6 of the golden one (the GPU's fp32 reductions differ in
order from the CPU's).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import capi_util as cu
from conftest import GOLDEN
from oracle import math_ref as mr
from oracle import quant as oq

pytestmark = pytest.mark.gpu
F32 = np.float32
TOL = 1e-5
# The packed matrix-core kernel (Int4Linear above 4 rows) multiplies x' split into bf16
# hi + mid + lo (x' to ~2^-26 relative) with exact products: fp32 arithmetic up to the
# summation order, so the GEMV's bar applies (inside the reference's int4 bar of 2e-4,
# tests/test_quant.py:116-118).
TOL_MC = 2e-5


def _linear(n_out, n_in, seed):
    g = torch.Generator().manual_seed(seed)
    lin = torch.nn.Linear(n_in, n_out, bias=False)
    with torch.no_grad():
        lin.weight.copy_(torch.randn(n_out, n_in, generator=g) * 0.02)
    return lin


@pytest.mark.parametrize("N,K", [(6144, 1024), (1000, 200)])
def test_int8linear_gemv_rows(gpu, N, K):
    """Int8Linear.forward at 1..16 rows runs the HIP GEMV (gemv_max_rows = 16)."""
    from llmserve.kernels import load_int8_gemv
    from llmserve.quant import Int8Linear

    lin = _linear(N, K, N + K)
    m = Int8Linear(lin, device="cuda")
    q, s = oq.int8_quantize(lin.weight.detach().numpy())
    assert np.array_equal(m.qweight.cpu().numpy(), q) and np.array_equal(m.scale.cpu().numpy(), s)
    rng = np.random.default_rng(N)
    for rows in (1, 2, 4, 5, 9, 16):
        assert m._path(rows, load_int8_gemv()) == "gemv"
        x = rng.standard_normal((rows, K)).astype(F32)
        y = m(cu.dev(x))
        cu.assert_rel_close(y, mr.int8_linear_f64(x, q, s), TOL, f"Int8Linear rows={rows}")
    # above 16 rows: the bf16 matrix-core GEMM, which steps K by 64 (else dequantize + GEMM)
    assert m._path(17, load_int8_gemv()) == ("prefill" if K % 64 == 0 else "dequant")


@pytest.mark.parametrize("N,K", [(4096, 1024), (1024, 2048), (6144, 1024), (1024, 3072)])
def test_int4linear_decode_rows(gpu, N, K):
    """Int4Linear.forward with AWQ at 1..16 rows: the GEMV up to 4 rows, the packed
    matrix-core kernel above, both against the float64 product."""
    from llmserve.quant import Int4Linear

    lin = _linear(N, K, N * 3 + K)
    rng = np.random.default_rng(K)
    act = (np.abs(rng.standard_normal(K)) + 0.2).astype(F32)
    m = Int4Linear(lin, 128, torch.from_numpy(act), device="cuda")
    nib, gs, gz, inv = oq.int4_quantize_pack(lin.weight.detach().numpy(), 128, act)
    assert np.array_equal(m.nibbles.cpu().numpy(), nib)
    for rows in (1, 2, 3, 4, 5, 9, 16):
        assert m.packed_path(rows) == (rows > 4)
        x = rng.standard_normal((rows, K)).astype(F32)
        x[:, rng.permutation(K)[: K // 100]] *= 20
        tol = TOL if rows <= 4 else TOL_MC
        cu.assert_rel_close(m(cu.dev(x)), mr.int4_linear_f64(x, nib, gs, gz, 128, inv), tol,
                            f"Int4Linear rows={rows} {N}x{K}")


def test_awq_search_on_gpu_picks_golden_alpha(gpu):
    from llmserve.quant import _awq_candidate, _search_awq_scale

    g = np.load(GOLDEN / "quant_golden.npz")
    w, x = torch.from_numpy(g["awq_w"]).cuda(), torch.from_numpy(g["awq_x"]).cuda()
    s = _search_awq_scale(w, x, int(g["awq_group"]))
    act = x.abs().mean(0).clamp_min(1e-5)
    picked = [a for a in (i / 10 for i in range(11)) if torch.equal(_awq_candidate(act, a), s)]
    assert picked == [float(g["awq_alpha"])]
    ref = g["awq_s"].astype(np.float64)
    assert np.abs(s.cpu().numpy() - ref).max() <= 2e-6 * np.abs(ref).max()


def test_quantize_model_awq_on_gpu(gpu):
    """quantize_model("int4-awq") with calibration rows from collect_linear_inputs: every
    linear but the LM head becomes an Int4Linear whose buffers are the oracle's quantization
    of W * s for the scale the search picks on those rows; outputs follow the float64
    product."""
    from llmserve.quant import Int4Linear, _search_awq_scale, collect_linear_inputs, quantize_model

    class Tiny(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.up = _linear(512, 256, 1)
            self.down = _linear(256, 512, 2)
            self.lm_head = _linear(64, 256, 3)

        def forward(self, x):
            return self.lm_head(self.down(torch.nn.functional.silu(self.up(x))))

    m = Tiny().cuda()
    x = torch.randn(700, 256, device="cuda", generator=torch.Generator(device="cuda").manual_seed(4))
    x[:, :3] *= 20
    acts = collect_linear_inputs(m, lambda: m(x), max_rows=512)
    assert acts["up"].shape == (512, 256) and acts["down"].shape == (512, 512)
    weights = {n: getattr(m, n).weight.detach().clone() for n in ("up", "down")}
    scales = {n: _search_awq_scale(weights[n], acts[n], 128) for n in ("up", "down")}
    quantize_model(m, "int4-awq", 128, calib_acts=acts)
    assert isinstance(m.lm_head, torch.nn.Linear)
    for n in ("up", "down"):
        mod = getattr(m, n)
        assert isinstance(mod, Int4Linear)
        s = scales[n].cpu().numpy()
        nib, gs, gz, inv = oq.int4_quantize_pack(weights[n].cpu().numpy(), 128, s)
        for a, b in ((mod.nibbles, nib), (mod.g_scale, gs), (mod.g_zero, gz), (mod.inv_act_scale, inv)):
            assert np.array_equal(a.cpu().numpy(), b), n
        xr = np.random.default_rng(9).standard_normal((3, mod.in_features)).astype(F32)
        cu.assert_rel_close(mod(cu.dev(xr)), mr.int4_linear_f64(xr, nib, gs, gz, 128, inv), TOL, n)
