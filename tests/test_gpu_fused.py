"""HIP fused decoder-layer ops and decode-step glue against the oracle.

Tolerances (fp32, a different reduction order than the reference's): max-abs <= 2e-6 x max|y|
against the float64 mathematics and the reference's compiled fused_ops (committed goldens).
The fused post-qkv decode kernel (norm + RoPE + int8 KV write) is compared bit for bit with
the composition of this build's rope_qk_ and llmserve_kv_quantize_write, whose quantizer is
bit-exact with the reference's (tests/test_gpu_quant.py).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import capi_util as cu
from conftest import GOLDEN
from oracle import fused_ops as ofo
from oracle import quant as oq

pytestmark = pytest.mark.gpu
F32 = np.float32
TOL = 2e-6


def fo():
    from llmserve.kernels import load_fused_ops

    return load_fused_ops()


@pytest.fixture(scope="module")
def fg():
    return dict(np.load(GOLDEN / "fused_golden.npz"))


def _rel(a, b):
    a = a.detach().cpu().numpy() if isinstance(a, torch.Tensor) else a
    return float(np.abs(np.asarray(a, np.float64) - b).max() / max(np.abs(b).max(), 1e-30))


@pytest.mark.parametrize("T,H", [(3, 1024), (2, 200), (1, 2048)])
def test_norms(gpu, fg, T, H):
    k = f"norm_T{T}_H{H}"
    x, r, w = fg[k + "_x"], fg[k + "_r"], fg[k + "_w"]
    out = fo().rmsnorm(cu.dev(x), cu.dev(w), 1e-6)
    assert _rel(out, fg[k + "_out"]) < 2 * TOL
    assert _rel(out, ofo.rmsnorm_f64(x, w, 1e-6)) < TOL
    xd = cu.dev(x)
    o = fo().add_rmsnorm_(xd, cu.dev(r), cu.dev(w), 1e-6)
    assert np.array_equal(xd.cpu().numpy(), fg[k + "_xadd"])  # x += r in place, one fp32 add
    assert _rel(o, fg[k + "_outadd"]) < 2 * TOL


@pytest.mark.parametrize("H", [200, 203, 2048, 3000, 4096, 5000, 5120])
def test_norm_forms_at_every_row_width(gpu, H):
    """Each row width's kernel form: rows of H % 4 == 0 channels up to 4096 keep 1, 2 or 4
    float4 chunks per thread in registers (200 and 3000 leave chunks partly or wholly past the
    row), anything else (203, 5000, 5120) runs one channel per thread. All of them: x += r is
    one fp32 add, the embedding row is copied exactly (an id outside the table gives a NaN row),
    the norm is within TOL of the float64 mathematics, and the fragment-writing form gives the
    bytes of the split pass over the plain form's output."""
    f = fo()
    T, V = 5, 40
    rng = np.random.default_rng(H)
    x = rng.standard_normal((T, H)).astype(F32)
    r = rng.standard_normal((T, H)).astype(F32)
    w = (1 + 0.1 * rng.standard_normal(H)).astype(F32)
    assert _rel(f.rmsnorm(cu.dev(x), cu.dev(w), 1e-6), ofo.rmsnorm_f64(x, w, 1e-6)) < TOL
    xd = cu.dev(x)
    out = f.add_rmsnorm_(xd, cu.dev(r), cu.dev(w), 1e-6)
    assert np.array_equal(xd.cpu().numpy(), x + r)
    assert _rel(out, ofo.rmsnorm_f64(x + r, w, 1e-6)) < TOL
    emb = rng.standard_normal((V, H)).astype(F32)
    ids = np.array([3, 0, V - 1, V, 7], np.int64)  # V: outside the table
    xe, he = f.embed_rmsnorm(cu.dev(ids), cu.dev(emb), cu.dev(w), 1e-6)
    xe, he = xe.cpu().numpy(), he.cpu().numpy()
    ok = ids < V
    assert np.array_equal(xe[ok], emb[ids[ok]])
    assert _rel(he[ok], ofo.rmsnorm_f64(emb[ids[ok]], w, 1e-6)) < TOL
    assert np.isnan(xe[~ok]).all() and np.isnan(he[~ok]).all()
    if H % 128 == 0:
        inv = cu.dev((rng.random(H) + 0.5).astype(F32))
        xa, xb = cu.dev(x), cu.dev(x)
        h = f.add_rmsnorm_(xa, cu.dev(r), cu.dev(w), 1e-6)
        xf = f.add_rmsnorm_xfrag_(xb, cu.dev(r), cu.dev(w), inv, 1e-6)
        assert torch.equal(xa, xb)
        assert torch.equal(xf, cu.split_fragments(h, inv))


@pytest.mark.parametrize("T,I", [(2, 300), (4, 3072)])
def test_silu_mul(gpu, fg, T, I):
    gu = fg[f"silu_T{T}_I{I}_gu"]
    out = fo().silu_mul(cu.dev(gu))
    assert _rel(out, fg[f"silu_T{T}_I{I}_out"]) < 2 * TOL
    assert _rel(out, ofo.silu_mul_f64(gu)) < TOL


@pytest.mark.parametrize("name", ["rope_d128", "rope_d64"])
def test_rope_qk_inplace(gpu, fg, name):
    nq, nk, D, norms = (int(v) for v in fg[f"{name}_meta"])
    qw = fg.get(f"{name}_qw") if norms else None
    kw = fg.get(f"{name}_kw") if norms else None
    qkv = cu.dev(fg[f"{name}_qkv"])
    fo().rope_qk_(qkv, cu.dev(fg[f"{name}_cos"]), cu.dev(fg[f"{name}_sin"]), nq, nk, D,
                  None if qw is None else cu.dev(qw), None if kw is None else cu.dev(kw), 1e-6)
    args = (fg[f"{name}_qkv"], fg[f"{name}_cos"], fg[f"{name}_sin"], nq, nk, D, qw, kw, 1e-6)
    assert _rel(qkv, fg[f"{name}_out"]) < 2 * TOL
    assert _rel(qkv, ofo.rope_qk_f64(*args)) < TOL


@pytest.mark.parametrize("D", [16, 32, 256])
def test_rope_other_head_dims(gpu, D):
    rng = np.random.default_rng(D)
    T, nq, nk = 3, 2, 1
    qkv = rng.standard_normal((T, (nq + 2 * nk) * D)).astype(F32)
    c, s = ofo.rope_tables(np.array([1, 9, 300]), D, 1e4)
    qw = (rng.random(D) + 0.5).astype(F32)
    t = cu.dev(qkv)
    fo().rope_qk_(t, cu.dev(c), cu.dev(s), nq, nk, D, cu.dev(qw), None, 1e-6)
    assert _rel(t, ofo.rope_qk_f64(qkv, c, s, nq, nk, D, qw, None, 1e-6)) < TOL


@pytest.mark.parametrize("smooth", [False, True])
def test_decode_qkv_kv_matches_composition(gpu, smooth):
    """Fused norm + RoPE + KV write == rope_qk_ (cos/sin rows at each position) followed by
    kv_quantize_write at the slots the block tables give, bit for bit."""
    rng = np.random.default_rng(5 + smooth)
    T, nq, nk, D, bs, nblk = 5, 4, 2, 128, 16, 40
    ctx = np.array([1, 16, 17, 300, 64], np.int64)  # positions 0, 15, 16, 299, 63
    width = -(-int(ctx.max()) // bs)
    perm = rng.permutation(nblk)
    bt = np.zeros((T, width), np.int64)
    used = 0
    for i, c in enumerate(ctx):
        n = -(-int(c) // bs)
        bt[i, :n] = perm[used:used + n] if used + n <= nblk else rng.integers(0, nblk, n)
        used += n
    qkv = rng.standard_normal((T, (nq + 2 * nk) * D)).astype(F32)
    qkv[:, nq * D + 5] *= 30  # an outlier key channel
    cos_t, sin_t = ofo.rope_tables(np.arange(512), D, 1e6)
    qw = (rng.random(D) + 0.5).astype(F32)
    kw = (rng.random(D) + 0.5).astype(F32)
    sm = (rng.random((nk, D)) + 0.5).astype(F32) if smooth else None
    kc = torch.zeros(nblk * bs, nk, D, dtype=torch.int8, device="cuda")
    vc, ks, vs = torch.zeros_like(kc), torch.zeros(nblk * bs, nk, device="cuda"), None
    vs = torch.zeros_like(ks)
    q = fo().decode_qkv_kv(cu.dev(qkv), cu.dev(cos_t), cu.dev(sin_t), cu.dev(ctx), cu.dev(bt), bs,
                           cu.dev(qw), cu.dev(kw), 1e-6, None if sm is None else cu.dev(sm),
                           kc, vc, ks, vs, nq, nk, D)
    # composition
    pos = ctx - 1
    ref = cu.dev(qkv)
    fo().rope_qk_(ref, cu.dev(cos_t[pos]), cu.dev(sin_t[pos]), nq, nk, D, cu.dev(qw), cu.dev(kw), 1e-6)
    refn = ref.cpu().numpy()
    assert np.array_equal(q.cpu().numpy().reshape(T, nq * D), refn[:, :nq * D])
    slots = cu.dev(np.array([bt[i, p // bs] * bs + p % bs for i, p in enumerate(pos)], np.int64))
    kc2, vc2 = torch.zeros_like(kc), torch.zeros_like(vc)
    ks2, vs2 = torch.zeros_like(ks), torch.zeros_like(vs)
    k_rows = torch.from_numpy(refn[:, nq * D:(nq + nk) * D].reshape(T, nk, D).copy()).cuda()
    v_rows = torch.from_numpy(qkv[:, (nq + nk) * D:].reshape(T, nk, D).copy()).cuda()
    cu.kv_quantize_write(k_rows, slots, kc2, ks2, None if sm is None else cu.dev(sm))
    cu.kv_quantize_write(v_rows, slots, vc2, vs2)
    for a, b in ((kc, kc2), (vc, vc2), (ks, ks2), (vs, vs2)):
        assert torch.equal(a, b)
    # and the quantized K rows equal the oracle quantizer on the oracle's RoPE output
    ko = ofo.rope_qk(qkv, cos_t[pos], sin_t[pos], nq, nk, D, qw, kw, 1e-6)[:, nq * D:(nq + nk) * D]
    kq, kss = oq.kv_quantize(oq.kv_smooth(ko.reshape(T, nk, D), sm) if sm is not None else ko.reshape(T, nk, D))
    got = kc[slots.cpu().numpy()].cpu().numpy()
    assert np.abs(got.astype(np.int32) - kq.astype(np.int32)).max() <= 1  # fp32 ulps may move a tie


def test_argmax_advance(gpu):
    """Greedy selection == torch.argmax on the CPU (sampling.py:170): first index among equal
    maxima, NaN above every number (the first NaN wins), an all -inf row gives 0."""
    rng = np.random.default_rng(3)
    T, V = 7, 151936
    logits = rng.standard_normal((T, V)).astype(F32)
    logits[1, 77] = logits[1, 150000] = 50.0  # tie: the first index wins
    logits[2, V - 1] = 60.0
    logits[3, 0] = 60.0
    logits[4, 12345] = logits[4, 99999] = np.nan
    logits[5] = -np.inf
    logits[6, 5000] = logits[6, 5256] = 70.0  # a tie inside one thread's unrolled loads
    ctx = np.arange(5, 5 + T, dtype=np.int64)
    c = cu.dev(ctx)
    ids = fo().argmax_advance(cu.dev(logits), c).cpu().numpy()
    want = torch.from_numpy(logits).argmax(-1).numpy()
    assert np.array_equal(ids, want)
    assert ids[1] == 77 and ids[4] == 12345 and ids[5] == 0 and ids[6] == 5000
    assert np.array_equal(c.cpu().numpy(), ctx + 1)


@pytest.mark.parametrize("V", [1, 31, 1000, 40000])
def test_argmax_small_vocab(gpu, V):
    rng = np.random.default_rng(V)
    logits = rng.integers(-3, 3, (4, V)).astype(F32)  # many ties
    c = cu.dev(np.zeros(4, np.int64))
    ids = fo().argmax_advance(cu.dev(logits), c).cpu().numpy()
    assert np.array_equal(ids, torch.from_numpy(logits).argmax(-1).numpy())


# ---- producers of the packed int4 linear's activation fragments ------------------------------

def _int4_packed(N, K, seed, awq=True):
    from llmserve.kernels import load_int8_gemv, load_quant

    g = torch.Generator(device="cuda").manual_seed(seed)
    w = torch.randn(N, K, device="cuda", generator=g) * 0.02
    act = (torch.rand(K, device="cuda", generator=g) + 0.5) if awq else None
    nib, gs, gz, inv = load_quant().int4_quantize(w, 128, act)
    return load_int8_gemv().int4_gemm_pack(nib, gs, gz, 128), (inv if awq else None)


@pytest.mark.parametrize("T", [17, 64, 70])
@pytest.mark.parametrize("awq", [True, False])
def test_xfrag_producers_equal_split_path(gpu, T, awq):
    """Norm / silu kernels writing fragments + the fragment GEMM give the same bits as the
    plain kernels followed by int4_linear_gemm_packed (its own split pass): the x' values,
    their bf16 split and the block sums are computed the same way."""
    from llmserve.kernels import load_int8_gemv

    f, lin = fo(), load_int8_gemv()
    H, I, N = 1024, 3072, 4096
    rng = np.random.default_rng(T + awq)
    x0 = rng.standard_normal((T, H)).astype(F32)
    r = rng.standard_normal((T, H)).astype(F32)
    w = (1 + 0.1 * rng.standard_normal(H)).astype(F32)
    pk, inv = _int4_packed(N, H, 1, awq)
    # add + rmsnorm
    xa, xb = cu.dev(x0), cu.dev(x0)
    h = f.add_rmsnorm_(xa, cu.dev(r), cu.dev(w), 1e-6)
    ref = lin.int4_linear_gemm_packed(h, pk, N, 128, inv)
    xf = f.add_rmsnorm_xfrag_(xb, cu.dev(r), cu.dev(w), inv, 1e-6)
    got = f.int4_linear_gemm_xfrag(xf, pk, T, N, H, 128)
    assert torch.equal(xa, xb) and torch.equal(got, ref)
    # embedding + rmsnorm
    V = 300
    emb = rng.standard_normal((V, H)).astype(F32)
    ids = cu.dev(rng.integers(0, V, T).astype(np.int64))
    xe, he = f.embed_rmsnorm(ids, cu.dev(emb), cu.dev(w), 1e-6)
    xe2, xfe = f.embed_rmsnorm_xfrag(ids, cu.dev(emb), cu.dev(w), inv, 1e-6)
    assert torch.equal(xe, xe2)
    assert torch.equal(f.int4_linear_gemm_xfrag(xfe, pk, T, N, H, 128),
                       lin.int4_linear_gemm_packed(he, pk, N, 128, inv))
    # silu * up -> down projection (K = 3072)
    pkd, invd = _int4_packed(1024, I, 2, awq)
    gu = cu.dev(rng.standard_normal((T, 2 * I)).astype(F32))
    ref = lin.int4_linear_gemm_packed(f.silu_mul(gu), pkd, 1024, 128, invd)
    got = f.int4_linear_gemm_xfrag(f.silu_mul_xfrag(gu, invd), pkd, T, 1024, I, 128)
    assert torch.equal(got, ref)


@pytest.mark.parametrize("T,P", [(17, 2), (64, 4), (70, 3)])
def test_add_rmsnorm_xfrag_adds_planes_in_order(gpu, T, P):
    """A residual given as P output planes [P, T, H] (a K-split linear's) is added plane by
    plane, then to x: the same x and fragments, bit for bit, as add_rmsnorm_xfrag_ with the
    planes summed in that order beforehand."""
    f = fo()
    H = 1024
    rng = np.random.default_rng(100 * T + P)
    x0 = rng.standard_normal((T, H)).astype(F32)
    planes = cu.dev(rng.standard_normal((P, T, H)).astype(F32))
    w = cu.dev((1 + 0.1 * rng.standard_normal(H)).astype(F32))
    inv = cu.dev((rng.random(H) + 0.5).astype(F32))
    r = planes[0].clone()
    for p in range(1, P):
        r = r + planes[p]
    xa, xb = cu.dev(x0), cu.dev(x0)
    ref = f.add_rmsnorm_xfrag_(xa, r, w, inv, 1e-6)
    got = f.add_rmsnorm_xfrag_(xb, planes, w, inv, 1e-6)
    assert torch.equal(xa, xb) and torch.equal(got, ref)
    with pytest.raises(RuntimeError, match="P, T, H"):
        f.add_rmsnorm_xfrag_(xb, planes[:, :-1].contiguous(), w, inv, 1e-6)


def test_xfrag_rejects_bad_shapes(gpu):
    f = fo()
    with pytest.raises(RuntimeError, match="multiple of 128"):
        f.silu_mul_xfrag(torch.zeros(4, 2 * 100, device="cuda"), None)
    pk, inv = _int4_packed(64, 256, 3)
    xf = f.add_rmsnorm_xfrag_(torch.zeros(8, 256, device="cuda"), torch.zeros(8, 256, device="cuda"),
                              torch.ones(256, device="cuda"), None, 1e-6)
    with pytest.raises(RuntimeError, match="fragments"):
        f.int4_linear_gemm_xfrag(xf, pk, 17, 64, 256, 128)  # buffer of one 16-row tile


@pytest.mark.parametrize("T", [1, 5, 16])
@pytest.mark.parametrize("awq", [True, False])
def test_one_tile_packed_gemm_equals_fragment_path(gpu, T, awq):
    """Up to 16 rows int4_linear_gemm_packed builds the fragments inside its GEMM launch; they
    and the products are the split pass's, so the result equals the fragment consumer on the
    fragments a norm or silu * up kernel writes, bit for bit (same per-wavefront blocks and
    the same fixed-order sum of the wavefronts at these shapes). A narrow output (down_proj
    here) splits its K blocks into planes: it equals the K-split fragment consumer's planes
    added in order."""
    from llmserve.kernels import load_int8_gemv

    f, lin = fo(), load_int8_gemv()
    H, I, N = 1024, 3072, 4096
    rng = np.random.default_rng(7 * T + awq)
    x0 = rng.standard_normal((T, H)).astype(F32)
    r = rng.standard_normal((T, H)).astype(F32)
    w = (1 + 0.1 * rng.standard_normal(H)).astype(F32)
    pk, inv = _int4_packed(N, H, 3, awq)
    xa, xb = cu.dev(x0), cu.dev(x0)
    h = f.add_rmsnorm_(xa, cu.dev(r), cu.dev(w), 1e-6)
    ref = lin.int4_linear_gemm_packed(h, pk, N, 128, inv)
    got = f.int4_linear_gemm_xfrag(f.add_rmsnorm_xfrag_(xb, cu.dev(r), cu.dev(w), inv, 1e-6),
                                   pk, T, N, H, 128)
    assert torch.equal(got, ref)
    pkd, invd = _int4_packed(1024, I, 4, awq)
    gu = cu.dev(rng.standard_normal((T, 2 * I)).astype(F32))
    ref = lin.int4_linear_gemm_packed(f.silu_mul(gu), pkd, 1024, 128, invd)
    P = int(cu.capi().llmserve_int4_packed_splits(T, 1024, I))
    assert P == 4
    planes = f.int4_linear_gemm_xfrag_split(f.silu_mul_xfrag(gu, invd), pkd, T, 1024, I, 128, P)
    got = planes[0].clone()
    for p in range(1, P):
        got = got + planes[p]
    assert torch.equal(got, ref)
