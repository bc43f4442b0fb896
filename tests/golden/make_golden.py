"""Writes the committed golden fixtures of this directory (run in the build container).

    python tests/golden/make_golden.py [quant | kernels | fused | attention_f32 ...]

quant_golden.npz — quantizer outputs computed with torch's CPU elementwise ops, the
arithmetic library the reference's quantizers run on (torch.round, IEEE division, amax/amin,
clamp; reference quant.py:41-43, :82-90, :103-114 and attention.py:153-157), on seeded
random weights plus hand-built rows that hit the edge cases: exact .5 ties for
round-half-to-even, all-zero and constant rows/groups (the 1e-8 clamps), subnormal and
very large values, a single outlier, and the AWQ fold with an outlier-driven scale. The
AWQ grid search is evaluated with the same torch CPU ops to record its alpha and scale.

kernels_golden.npz — outputs of the reference's own compiled CPU kernels (int8_linear,
int4_linear, paged_attention_decode_int8 built from the reference sources into
oracle/_ref/ by oracle/build.py) on small seeded inputs, including odd shapes, several
group sizes, ragged contexts and forced partition sizes. Skipped when oracle/_ref is not
built.

fused_golden.npz — outputs of the reference's compiled fused decoder-layer ops (rmsnorm,
add_rmsnorm_, silu_mul, rope_qk_ from fused_ops.cpp) on small seeded inputs: odd and Qwen3
hidden sizes, q/k norms on and off, head dims 64 and 128, RoPE tables at arbitrary positions.
Skipped when oracle/_ref is not built.

attention_f32_golden.npz — outputs of the reference's compiled fp32-cache decode
(paged_attention_decode) on small seeded inputs (ragged contexts, GQA 1/2/4, forced
partition sizes). Skipped when oracle/_ref is not built.
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))


# ---- torch-CPU quantizers (the reference's arithmetic, stated with torch ops) -------------

def t_int8(w: torch.Tensor):
    amax = w.abs().amax(dim=1)
    scale = (amax / 127.0).clamp_min(1e-8)
    return torch.round(w / scale[:, None]).clamp(-127, 127).to(torch.int8), scale


def t_int4(w: torch.Tensor, group: int):
    n, k = w.shape
    g = w.reshape(n, k // group, group)
    lo, hi = g.amin(-1, keepdim=True), g.amax(-1, keepdim=True)
    scale = ((hi - lo) / 15.0).clamp_min(1e-8)
    q = torch.round((g - lo) / scale).clamp(0, 15).to(torch.int32).reshape(n, k)
    zero = lo + 8.0 * scale
    return q, scale.squeeze(-1), zero.squeeze(-1)


def t_pack(q: torch.Tensor):
    q8 = q.to(torch.uint8)
    return q8[:, 0::2] | (q8[:, 1::2] << 4)


def t_kv(x: torch.Tensor):
    s = x.abs().amax(-1).clamp_min(1e-8) / 127.0
    return (x / s[..., None]).round().clamp(-127, 127).to(torch.int8), s


def t_awq_search(w: torch.Tensor, x: torch.Tensor, group: int):
    act = x.abs().mean(0).clamp_min(1e-5)
    ref = x @ w.t()
    best, best_s, best_a = float("inf"), None, None
    for i in range(11):
        a = i / 10
        s = act.pow(a)
        s = s / (s.max() * s.min()).sqrt()
        q, sc, z = t_int4(w * s[None, :], group)
        deq = ((q.float().reshape(w.shape[0], -1, group) - 8) * sc[..., None] + z[..., None])
        deq = deq.reshape(w.shape) / s[None, :]
        err = (x @ deq.t() - ref).pow(2).mean().item()
        if err < best:
            best, best_s, best_a = err, s, a
    return best_s, best_a


def special_int8_rows(K: int) -> torch.Tensor:
    rows = torch.zeros(8, K)
    # ties at scale 1: amax 127 -> scale = 1, values k + 0.5 round half to even
    r = torch.arange(K, dtype=torch.float32) % 127 - 63 + 0.5
    rows[1] = r
    rows[1, 0] = 127.0
    # scale 0.5 (amax 63.5): values (n + 0.5) * 0.5 hit .5 after division
    rows[2] = (torch.arange(K, dtype=torch.float32) % 120 - 60 + 0.5) * 0.5
    rows[2, 1] = 63.5
    rows[3] = torch.linspace(-1e-7, 1e-7, K)  # scale clamps to 1e-8
    rows[4] = torch.linspace(-3e-40, 3e-40, K)  # subnormals
    rows[5] = torch.linspace(-1e30, 1e30, K)
    rows[6] = torch.randn(K, generator=torch.Generator().manual_seed(7)) * 0.01
    rows[6, 5] = 100.0  # one outlier
    rows[7] = -rows[1]
    return rows


def near_tie_rows(n: int, K: int, seed: int) -> torch.Tensor:
    """Rows whose values sit on or one float32 ulp next to (k + 1/2) * scale, where IEEE
    division and a reciprocal multiply round to different integers."""
    g = torch.Generator().manual_seed(seed)
    amax = torch.rand(n, 1, generator=g, dtype=torch.float64) * 1.5 + 0.5
    amax = amax.float()
    scale = (amax / 127.0).double()
    k = torch.randint(-126, 126, (n, K), generator=g).double()
    rows = ((k + 0.5) * scale).float()
    rows[:, 0] = amax[:, 0]
    return rows


def special_int4_rows(K: int, group: int) -> torch.Tensor:
    G = K // group
    rows = torch.randn(6, K, generator=torch.Generator().manual_seed(11)) * 0.02
    grp = rows.view(6, G, group)
    grp[0, 0] = 0.25  # constant group: scale clamps to 1e-8, q = 0
    grp[1, 0] = (torch.arange(group, dtype=torch.float32) % 15) + 0.5  # mn 0.5 .. ties
    grp[1, 0, 0] = 0.0
    grp[1, 0, 1] = 15.0  # range 15 -> scale 1, (w - 0) / 1 = k + 0.5
    grp[2, 0] = torch.linspace(-7.5, 7.5, group)
    grp[3, 0] = torch.linspace(0, 1e-7, group)  # tiny range -> scale clamp
    grp[4, 0] = torch.linspace(-3e-40, 3e-40, group)
    grp[5, 0] = 0.0
    grp[5, 0, 3] = -2.0  # one low outlier
    return rows


def quant_golden() -> dict[str, np.ndarray]:
    g = torch.Generator().manual_seed(1234)
    out: dict[str, np.ndarray] = {}
    # int8 rows
    K = 256
    w8 = torch.cat([torch.randn(24, K, generator=g) * 0.02, torch.randn(8, K, generator=g),
                    special_int8_rows(K), near_tie_rows(16, K, 5)])
    q8, s8 = t_int8(w8)
    out.update(int8_w=w8.numpy(), int8_q=q8.numpy(), int8_scale=s8.numpy())
    # int4 groups, with and without AWQ fold
    K4 = 256
    for group in (32, 64, 128):
        w4 = torch.cat([torch.randn(16, K4, generator=g) * 0.02, special_int4_rows(K4, group)])
        q4, s4, z4 = t_int4(w4, group)
        out[f"int4_g{group}_w"] = w4.numpy()
        out[f"int4_g{group}_nib"] = t_pack(q4).numpy()
        out[f"int4_g{group}_scale"] = s4.numpy()
        out[f"int4_g{group}_zero"] = z4.numpy()
    # AWQ fold with an outlier-driven scale, and the grid search
    N, Ka, R = 64, 256, 128
    wa = torch.randn(N, Ka, generator=g) * 0.02
    xa = torch.randn(R, Ka, generator=g)
    outl = torch.randperm(Ka, generator=g)[: max(1, Ka // 100)]
    xa[:, outl] *= 20.0
    s, alpha = t_awq_search(wa, xa, 64)
    qa, sa, za = t_int4(wa * s[None, :], 64)
    out.update(awq_w=wa.numpy(), awq_x=xa.numpy(), awq_s=s.numpy(), awq_alpha=np.float64(alpha),
               awq_inv=(1.0 / s).numpy(), awq_nib=t_pack(qa).numpy(), awq_scale=sa.numpy(),
               awq_zero=za.numpy(), awq_group=np.int64(64))
    # int8 KV rows, plain and smoothed
    x = torch.randn(40, 2, 32, generator=g)
    x[0] = 0.0
    x[1, 0] = torch.arange(32, dtype=torch.float32) - 15.5  # amax 16... ties after scaling
    x[1, 0, 0] = 127.0  # scale 1
    x[2, 1] = torch.linspace(-1e-9, 1e-9, 32)
    x[3, 0, 7] = 40.0
    x[8:24] = near_tie_rows(32, 32, 6).view(16, 2, 32)
    kq, ks = t_kv(x)
    sm = x.abs().amax(0).clamp_min(1e-5).sqrt()
    sm = sm / sm.mean(-1, keepdim=True)
    kqs, kss = t_kv(x / sm)
    out.update(kv_x=x.numpy(), kv_q=kq.numpy(), kv_s=ks.numpy(), kv_smooth=sm.numpy(),
               kv_q_smoothed=kqs.numpy(), kv_s_smoothed=kss.numpy())
    return out


def kernels_golden() -> dict[str, np.ndarray] | None:
    from oracle import cpu as ocpu

    if not ocpu.ref_available():
        return None
    gemv = ocpu.ref_module("llmserve_int8_gemv")
    pa = ocpu.ref_module("llmserve_paged_attention")
    g = torch.Generator().manual_seed(99)
    out: dict[str, np.ndarray] = {}
    for M, K, N in ((1, 200, 77), (3, 200, 77), (16, 200, 77), (4, 1024, 96)):
        x = torch.randn(M, K, generator=g)
        q, s = t_int8(torch.randn(N, K, generator=g) * 0.02)
        y = gemv.int8_linear(x, q, s)
        key = f"i8_M{M}_K{K}_N{N}"
        out.update({key + "_x": x.numpy(), key + "_q": q.numpy(), key + "_s": s.numpy(),
                    key + "_y": y.numpy()})
    for M, K, N, group in ((1, 256, 80, 64), (5, 256, 80, 64), (16, 256, 80, 64),
                           (4, 1024, 64, 128), (2, 512, 48, 32)):
        x = torch.randn(M, K, generator=g)
        q, s, z = t_int4(torch.randn(N, K, generator=g) * 0.02, group)
        nib = t_pack(q).contiguous()
        y = gemv.int4_linear(x, nib, s.contiguous(), z.contiguous(), group)
        key = f"i4_M{M}_K{K}_N{N}_g{group}"
        out.update({key + "_x": x.numpy(), key + "_nib": nib.numpy(), key + "_s": s.numpy(),
                    key + "_z": z.numpy(), key + "_y": y.numpy()})
    cases = [
        ("pa_small", 8, 2, 32, 4, [1, 7, 33, 120, 4], 128, [0, 4, 8, 10000]),
        ("pa_d128", 4, 2, 128, 16, [17, 100, 200, 5], 24, [0, 32, 64]),
        ("pa_g1", 4, 4, 64, 8, [9, 23, 64], 32, [0, 16]),
    ]
    for name, hq, hk, d, bs, ctx, nblocks, parts in cases:
        kc = torch.randn(nblocks * bs, hk, d, generator=g)
        kc[..., 3] *= 8.0
        vc = torch.randn(nblocks * bs, hk, d, generator=g)
        kq, ks = t_kv(kc)
        vq, vs = t_kv(vc)
        perm = torch.randperm(nblocks, generator=g).tolist()
        tables, used = [], 0
        for c in ctx:
            n = -(-c // bs)
            tables.append(perm[used: used + n])
            used += n
        width = max(len(t) for t in tables)
        bt = torch.tensor([t + [0] * (width - len(t)) for t in tables], dtype=torch.long)
        cl = torch.tensor(ctx, dtype=torch.long)
        q = torch.randn(len(ctx), hq, d, generator=g)
        sc = d ** -0.5
        out.update({f"{name}_q": q.numpy(), f"{name}_kq": kq.numpy(), f"{name}_ks": ks.numpy(),
                    f"{name}_vq": vq.numpy(), f"{name}_vs": vs.numpy(), f"{name}_bt": bt.numpy(),
                    f"{name}_cl": cl.numpy(), f"{name}_meta": np.array([bs, sc], np.float64)})
        for p in parts:
            o = pa.paged_attention_decode_int8(q, kq, vq, ks.contiguous(), vs.contiguous(), bt,
                                               cl, bs, sc, p)
            out[f"{name}_out_p{p}"] = o.numpy()
    return out


def fused_golden() -> dict[str, np.ndarray] | None:
    from oracle import cpu as ocpu
    from oracle import fused_ops as ofo

    if not ocpu.ref_available():
        return None
    fo = ocpu.ref_module("llmserve_fused_ops")
    g = torch.Generator().manual_seed(123)
    out: dict[str, np.ndarray] = {}
    for T, H in ((3, 1024), (2, 200), (1, 2048)):
        x = torch.randn(T, H, generator=g) * 3.0
        r = torch.randn(T, H, generator=g)
        w = torch.rand(H, generator=g) + 0.5
        key = f"norm_T{T}_H{H}"
        out.update({key + "_x": x.numpy().copy(), key + "_r": r.numpy(), key + "_w": w.numpy(),
                    key + "_out": fo.rmsnorm(x, w, 1e-6).numpy()})
        xa = x.clone()
        o = fo.add_rmsnorm_(xa, r, w, 1e-6)
        out.update({key + "_xadd": xa.numpy(), key + "_outadd": o.numpy()})
    for T, I in ((2, 300), (4, 3072)):
        gu = torch.randn(T, 2 * I, generator=g) * 4.0
        out.update({f"silu_T{T}_I{I}_gu": gu.numpy(), f"silu_T{T}_I{I}_out": fo.silu_mul(gu).numpy()})
    for name, T, nq, nk, D, norms in (("rope_d128", 3, 4, 2, 128, True), ("rope_d64", 2, 2, 1, 64, False)):
        row = (nq + 2 * nk) * D
        qkv = torch.randn(T, row, generator=g)
        pos = np.array([0, 17, 4095][:T], np.int64)
        c, s_ = ofo.rope_tables(pos, D, 1e6)
        qw = torch.rand(D, generator=g) + 0.5 if norms else None
        kw = torch.rand(D, generator=g) + 0.5 if norms else None
        res = qkv.clone()
        fo.rope_qk_(res, torch.from_numpy(c), torch.from_numpy(s_), nq, nk, D, qw, kw, 1e-6)
        out.update({f"{name}_qkv": qkv.numpy(), f"{name}_cos": c, f"{name}_sin": s_,
                    f"{name}_out": res.numpy(),
                    f"{name}_meta": np.array([nq, nk, D, int(norms)], np.int64)})
        if norms:
            out.update({f"{name}_qw": qw.numpy(), f"{name}_kw": kw.numpy()})
    return out


def attention_f32_golden() -> dict[str, np.ndarray] | None:
    """The reference's fp32-cache decode (paged_attention_decode, paged_attention.cpp:350-359)
    on small seeded inputs: ragged contexts, GQA 1 / 2 / 4, head dims 32 / 64 / 128, forced
    partition sizes."""
    from oracle import cpu as ocpu

    if not ocpu.ref_available():
        return None
    pa = ocpu.ref_module("llmserve_paged_attention")
    g = torch.Generator().manual_seed(4321)
    out: dict[str, np.ndarray] = {}
    cases = [
        ("f32_small", 8, 2, 32, 4, [1, 7, 33, 120, 4], 128, [0, 8, 10000]),
        ("f32_d128", 4, 2, 128, 16, [17, 100, 200, 5], 24, [0, 32]),
        ("f32_g1", 4, 4, 64, 8, [9, 23, 64], 32, [0, 16]),
    ]
    for name, hq, hk, d, bs, ctx, nblocks, parts in cases:
        kc = torch.randn(nblocks * bs, hk, d, generator=g)
        kc[..., 3] *= 8.0
        vc = torch.randn(nblocks * bs, hk, d, generator=g)
        perm = torch.randperm(nblocks, generator=g).tolist()
        tables, used = [], 0
        for c in ctx:
            n = -(-c // bs)
            tables.append(perm[used: used + n])
            used += n
        width = max(len(t) for t in tables)
        bt = torch.tensor([t + [0] * (width - len(t)) for t in tables], dtype=torch.long)
        cl = torch.tensor(ctx, dtype=torch.long)
        q = torch.randn(len(ctx), hq, d, generator=g)
        sc = d ** -0.5
        out.update({f"{name}_q": q.numpy(), f"{name}_k": kc.numpy(), f"{name}_v": vc.numpy(),
                    f"{name}_bt": bt.numpy(), f"{name}_cl": cl.numpy(),
                    f"{name}_meta": np.array([bs, sc], np.float64)})
        for p in parts:
            o = pa.paged_attention_decode(q, kc, vc, bt, cl, bs, sc, p)
            out[f"{name}_out_p{p}"] = o.numpy()
    return out


WRITERS = {
    "quant": ("quant_golden.npz", quant_golden),
    "kernels": ("kernels_golden.npz", kernels_golden),
    "fused": ("fused_golden.npz", fused_golden),
    "attention_f32": ("attention_f32_golden.npz", attention_f32_golden),
}


def main(which: list[str]) -> None:
    """Writes the fixtures named in ``which`` (all of them when empty)."""
    torch.set_num_threads(4)
    for key in which or list(WRITERS):
        fname, fn = WRITERS[key]
        data = fn()
        if data is None:
            print(f"oracle/_ref not built: {fname} left unchanged")
            continue
        np.savez_compressed(HERE / fname, **data)
        print("wrote", HERE / fname)


if __name__ == "__main__":
    main(sys.argv[1:])
