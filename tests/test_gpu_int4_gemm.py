"""int4 weight-only linear for M > 16 on the matrix cores (Int4Linear's large-M branch,
reference quant.py:141-142) through the C ABI, against the float64 oracle: the kernel on the
reference [N, K/2] layout and the decode-batch kernel on the packed weight, whose packing is
checked byte for byte by unpacking it on the host.

Tolerance: max-abs error <= 2e-5 * max|y| and rel-L2 <= 2e-5 against the float64 mathematics.
x' = x * inv_act_scale is carried as bf16 terms (two by the reference-layout kernel: x' to
2^-17 relative; three by the packed decode-batch kernel: x' to ~2^-26) and every matrix-core
product is exact, so the error is a few 1e-6 or less; 2e-5 stays inside the reference tests'
own 2e-4 for int4 (tests/test_quant.py:116-118).
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


# ---- packed weight + decode-batch kernel ------------------------------------------------------

def unpack(packed: np.ndarray, N: int, K: int, G: int):
    """Inverse of llmserve_int4_gemm_pack, written from its documented layout."""
    slabs, nblk = -(-N // 64), K // 128
    wbytes = slabs * nblk * 4 * 1024
    wpk = packed[:wbytes].reshape(slabs, nblk, 4, 64, 16)
    nib = np.zeros((slabs * 64, K // 2), np.uint8)
    for u in range(4):
        for lane in range(64):
            rows = np.arange(slabs) * 64 + 16 * u + lane % 16
            for b in range(nblk):
                c = 64 * b + 16 * (lane // 16)
                nib[rows, c:c + 16] = wpk[:, b, u, lane]
    off = -(-wbytes // 256) * 256
    sz = packed[off:off + G * slabs * 16 * 8 * 4].view(np.float32).reshape(G, slabs, 16, 8)
    s = np.zeros((slabs * 64, G), np.float32)
    zz = np.zeros((slabs * 64, G), np.float32)
    for u in range(4):
        rows = np.arange(slabs)[:, None] * 64 + 16 * u + np.arange(16)[None, :]
        s[rows.ravel()] = sz[:, :, :, u].transpose(1, 2, 0).reshape(-1, G)
        zz[rows.ravel()] = sz[:, :, :, 4 + u].transpose(1, 2, 0).reshape(-1, G)
    return nib, s, zz


@pytest.mark.parametrize("N,K,g", [(4096, 1024, 128), (77, 256, 128), (1000, 1536, 256)])
def test_pack_layout(gpu, N, K, g):
    _, nib, gs, gz, _ = _case(4, N, K, g, N + K, awq=False)
    packed = cu.int4_gemm_pack(cu.dev(nib), cu.dev(gs), cu.dev(gz), g).cpu().numpy()
    G = K // g
    assert packed.size == cu.capi().llmserve_int4_gemm_pack_bytes(N, K, g)
    pn, ps, pz = unpack(packed, N, K, G)
    assert np.array_equal(pn[:N], nib) and not pn[N:].any()
    assert np.array_equal(ps[:N], gs) and not ps[N:].any()
    assert np.array_equal(pz[:N], (gz - F32(8) * gs).astype(F32)) and not pz[N:].any()


@pytest.mark.parametrize("M", [5, 16, 17, 32, 64])
@pytest.mark.parametrize("N,K", QWEN)
def test_packed_gemm_qwen_shapes(gpu, M, N, K):
    x, nib, gs, gz, inv = _case(M, N, K, 128, M * 37 + N + K)
    packed = cu.int4_gemm_pack(cu.dev(nib), cu.dev(gs), cu.dev(gz), 128)
    y = cu.int4_linear_gemm_packed(cu.dev(x), packed, N, 128, cu.dev(inv))
    cu.assert_rel_close(y, mr.int4_linear_f64(x, nib, gs, gz, 128, inv), TOL, f"M={M} {N}x{K}")


@pytest.mark.parametrize("M,N,K,g", [(1, 32, 512, 128), (5, 77, 256, 128), (64, 1000, 1536, 256),
                                     (33, 16, 128, 128), (100, 160, 4096, 128), (300, 72, 640, 128),
                                     (64, 151936 // 8, 1024, 128), (48, 64, 3200, 640),
                                     (16, 4200, 1024, 128), (7, 4213, 512, 256)])
def test_packed_gemm_tails(gpu, M, N, K, g):
    """Any N (packed slabs pad to 64 rows), K past one round of 24 blocks (4096, 3200),
    groups of several blocks, row tails, a wide output, no AWQ scale on odd M. Up to 16 rows,
    more 16-column tiles than CUs (N = 4200: 264 tiles) run two tiles per workgroup, with a
    last workgroup whose second tile is past N."""
    x, nib, gs, gz, inv = _case(M, N, K, g, M + N + K + g, awq=(M % 2 == 0))
    packed = cu.int4_gemm_pack(cu.dev(nib), cu.dev(gs), cu.dev(gz), g)
    y = cu.int4_linear_gemm_packed(cu.dev(x), packed, N, g, None if inv is None else cu.dev(inv))
    cu.assert_rel_close(y, mr.int4_linear_f64(x, nib, gs, gz, g, inv), TOL, f"M={M} {N}x{K} g{g}")


@pytest.mark.parametrize("M,N,K", [(64, 151936, 1024), (20, 2049 * 64 - 24, 512)])
def test_packed_gemm_wide_outputs(gpu, M, N, K):
    """Outputs of thousands of slabs (an LM head) run the slab-looping kernel that keeps each
    K block's x fragments in registers: against float64, and bit for bit against the same
    columns computed in chunks narrow enough for the per-slab kernel (same per-block
    arithmetic, same order of the partial sums)."""
    x, nib, gs, gz, inv = _case(M, N, K, 128, M + N + K)
    packed = cu.int4_gemm_pack(cu.dev(nib), cu.dev(gs), cu.dev(gz), 128)
    y = cu.int4_linear_gemm_packed(cu.dev(x), packed, N, 128, cu.dev(inv))
    cu.assert_rel_close(y, mr.int4_linear_f64(x, nib, gs, gz, 128, inv), TOL, f"M={M} {N}x{K}")
    chunk = 512 * 64 if M > 32 else 1024 * 64  # below the wide kernel's slab count
    parts = []
    for c0 in range(0, N, chunk):
        c1 = min(N, c0 + chunk)
        pk = cu.int4_gemm_pack(cu.dev(nib[c0:c1]), cu.dev(gs[c0:c1]), cu.dev(gz[c0:c1]), 128)
        parts.append(cu.int4_linear_gemm_packed(cu.dev(x), pk, c1 - c0, 128, cu.dev(inv)))
    assert torch.equal(y, torch.cat(parts, 1)), f"M={M} {N}x{K}: wide kernel != per-slab kernel"


def _gemm_xfrag_split(xf, packed, M, N, K, g, P):
    L = cu.capi()
    y = torch.full((P, M, N), float("nan"), dtype=torch.float32, device=xf.device)
    cu.check(L.llmserve_int4_linear_gemm_xfrag_split(cu._p(xf), cu._p(packed), cu._p(y), M, N, K,
                                                     g, P, cu._stream()))
    return y


@pytest.mark.parametrize("M", [17, 64])
@pytest.mark.parametrize("N,K", [(1024, 2048), (1024, 3072), (4096, 1024)])
def test_packed_gemm_split_planes(gpu, M, N, K):
    """The decode step's K-split linear (o_proj, down_proj): plane p of P is the product over
    the K blocks [p ceil(nb / P), ...) -- checked against the float64 mathematics of x with the
    other channels zeroed (an empty plane is exactly 0) -- and the planes added in order give
    the linear. P = 2, 3 (not dividing the blocks), 4 and the count the step uses."""
    x, nib, gs, gz, inv = _case(M, N, K, 128, M * 41 + N + K)
    packed = cu.int4_gemm_pack(cu.dev(nib), cu.dev(gs), cu.dev(gz), 128)
    xf = cu.split_fragments(cu.dev(x), cu.dev(inv))
    nb = K // 128
    step_p = cu.capi().llmserve_int4_xfrag_splits(M, N, K)
    # the rule: double P while the slab tiles of all planes still fit the CUs (256) and each
    # plane keeps >= 4 blocks
    tiles, want = (N // 64) * -(-M // 16), 1
    while want < 8 and tiles * 2 * want <= 256 and nb >= 8 * want:
        want *= 2
    assert step_p == want
    full = mr.int4_linear_f64(x, nib, gs, gz, 128, inv)
    for P in sorted({2, 3, 4, step_p}):
        y = _gemm_xfrag_split(xf, packed, M, N, K, 128, P)
        bpp = -(-nb // P)
        for p in range(P):
            lo, hi = min(p * bpp, nb) * 128, min((p + 1) * bpp, nb) * 128
            xp = np.zeros_like(x)
            xp[:, lo:hi] = x[:, lo:hi]
            ref = mr.int4_linear_f64(xp, nib, gs, gz, 128, inv)
            if hi == lo:
                assert not y[p].any(), f"P={P} plane {p} is empty and must be zero"
            else:
                cu.assert_rel_close(y[p], ref, TOL, f"M={M} {N}x{K} P={P} plane {p}")
        s = y[0].clone()
        for p in range(1, P):
            s = s + y[p]
        cu.assert_rel_close(s, full, TOL, f"M={M} {N}x{K} P={P} sum")
    with pytest.raises(RuntimeError, match="splits"):
        _gemm_xfrag_split(xf, packed, M, N, K, 128, 9)


@pytest.mark.parametrize("M,N,K,g", [(16, 1024, 2048, 128), (16, 1024, 3072, 128),
                                     (5, 1024, 2048, 128), (1, 1024, 3072, 128),
                                     (9, 200, 1536, 256), (16, 64, 3200, 640)])
def test_one_tile_k_planes(gpu, M, N, K, g):
    """Up to 16 rows a narrow output splits its K blocks over workgroups (config 2's o_proj
    and down_proj at 16 rows: 4 planes each; planes past the first must fit the workspace the
    call takes anyway): the result is within TOL of float64 and equals, bit for bit, the
    K-split fragment consumer's planes on the same x' added in order. The wide shapes keep one
    plane."""
    L = cu.capi()
    assert [L.llmserve_int4_packed_splits(16, n, k) for n, k in QWEN] == \
        [1 if n > 1024 else 4 for n, k in QWEN]
    P = int(L.llmserve_int4_packed_splits(M, N, K))
    assert P > 1
    x, nib, gs, gz, inv = _case(M, N, K, g, 5 * M + N + K)
    packed = cu.int4_gemm_pack(cu.dev(nib), cu.dev(gs), cu.dev(gz), g)
    y = cu.int4_linear_gemm_packed(cu.dev(x), packed, N, g, cu.dev(inv))
    cu.assert_rel_close(y, mr.int4_linear_f64(x, nib, gs, gz, g, inv), TOL, f"M={M} {N}x{K}")
    planes = _gemm_xfrag_split(cu.split_fragments(cu.dev(x), cu.dev(inv)), packed, M, N, K, g, P)
    s = planes[0].clone()
    for p in range(1, P):
        s = s + planes[p]
    assert torch.equal(y, s), f"M={M} {N}x{K}: one-launch planes != fragment planes"


def test_packed_gemm_rejects_bad_shapes(gpu):
    x, nib, gs, gz, _ = _case(20, 48, 256, 64, 3, awq=False)
    with pytest.raises(RuntimeError, match="multiples of 128"):
        cu.int4_gemm_pack(cu.dev(nib), cu.dev(gs), cu.dev(gz), 64)
    x, nib, gs, gz, _ = _case(20, 48, 256, 128, 3, awq=False)
    packed = cu.int4_gemm_pack(cu.dev(nib), cu.dev(gs), cu.dev(gz), 128)
    with pytest.raises(RuntimeError, match="workspace"):
        L = cu.capi()
        y = torch.empty(20, 48, device="cuda")
        xd = cu.dev(x)
        cu.check(L.llmserve_int4_linear_gemm_packed(cu._p(xd), None, cu._p(packed), cu._p(y), 20, 48,
                                                    256, 128, None, 0, cu._stream()))


@pytest.mark.parametrize("rows", [17, 64, 300])
def test_int4linear_packed_paths(gpu, rows):
    """Int4Linear's auto choice agrees with dequantize + GEMM: with 1000 outputs (not a
    multiple of 16) only the packed kernel applies at every batch, and forcing the
    reference-layout kernel is an error."""
    from llmserve.quant import Int4Linear

    rng = np.random.default_rng(rows)
    lin = torch.nn.Linear(1024, 1000, bias=False)
    with torch.no_grad():
        lin.weight.copy_(torch.from_numpy((rng.standard_normal((1000, 1024)) * 0.02).astype(F32)))
    act = torch.from_numpy((np.abs(rng.standard_normal(1024)) + 0.5).astype(F32))
    q = Int4Linear(lin, 128, act, device="cuda")
    assert q.gemm_packed is not None
    x = torch.from_numpy(rng.standard_normal((rows, 1024)).astype(F32)).cuda()
    q.kernel = "aten"
    ref = q(x)
    for k in ("auto", "gemm"):
        q.kernel = k
        y = q(x)
        err = (y - ref).abs().max().item() / ref.abs().max().item()
        assert err < 2e-5, (k, err)
    q.kernel = "gemm_ref"
    with pytest.raises(RuntimeError, match="multiple of 16"):
        q(x)


@pytest.mark.parametrize("M,N,K,g,awq", [(1, 40, 128, 128, True), (2, 1024, 4096, 128, False),
                                          (9, 200, 1536, 256, True), (15, 6144, 1024, 128, False),
                                          (16, 64, 3200, 640, True), (3, 1024, 2048, 1024, True)])
def test_one_tile_packed_gemm_odd_shapes(gpu, M, N, K, g, awq):
    """The one-launch kernel for up to 16 rows: one K block (four wavefronts, three idle
    blocks masked), two rounds of 16 blocks, groups spanning several blocks, a single
    partial slab, no AWQ scale."""
    x, nib, gs, gz, inv = _case(M, N, K, g, 11 * M + N + K, awq=awq)
    packed = cu.int4_gemm_pack(cu.dev(nib), cu.dev(gs), cu.dev(gz), g)
    y = cu.int4_linear_gemm_packed(cu.dev(x), packed, N, g, None if inv is None else cu.dev(inv))
    cu.assert_rel_close(y, mr.int4_linear_f64(x, nib, gs, gz, g, inv), TOL, f"M={M} {N}x{K} g{g}")
