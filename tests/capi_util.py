"""Calls into the C ABI (include/llmserve_hip.h) through ctypes, with torch providing the
device memory and the current stream. Used by the GPU parity tests."""

from __future__ import annotations

import ctypes

import numpy as np
import torch

from llmserve._native import capi, check


def _p(t: torch.Tensor | None):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def dev(a: np.ndarray, device="cuda") -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a)).to(device)


def int8_quantize(w: torch.Tensor):
    N, K = w.shape
    q = torch.empty(N, K, dtype=torch.int8, device=w.device)
    s = torch.empty(N, dtype=torch.float32, device=w.device)
    check(capi().llmserve_int8_quantize(_p(w), _p(q), _p(s), N, K, _stream()))
    return q, s


def int4_quantize(w: torch.Tensor, group: int, act_scale: torch.Tensor | None = None):
    N, K = w.shape
    nib = torch.empty(N, K // 2, dtype=torch.uint8, device=w.device)
    gs = torch.empty(N, K // group, dtype=torch.float32, device=w.device)
    gz = torch.empty_like(gs)
    inv = torch.empty(K, dtype=torch.float32, device=w.device) if act_scale is not None else None
    check(capi().llmserve_int4_quantize(_p(w), _p(act_scale), _p(nib), _p(gs), _p(gz), _p(inv),
                                        N, K, group, _stream()))
    return nib, gs, gz, inv


def kv_quantize_write(x, slots, data, scale, smooth=None):
    T, Hk, D = x.shape
    check(capi().llmserve_kv_quantize_write(_p(x), _p(slots), _p(smooth), _p(data), _p(scale),
                                            T, Hk, D, data.shape[0], _stream()))


def int8_linear(x, q, s):
    M, K = x.shape
    N = q.shape[0]
    y = torch.empty(M, N, dtype=torch.float32, device=x.device)
    check(capi().llmserve_int8_linear(_p(x), _p(q), _p(s), _p(y), M, N, K, _stream()))
    return y


def int4_linear(x, nib, gs, gz, group, inv=None):
    M, K = x.shape
    N = nib.shape[0]
    y = torch.empty(M, N, dtype=torch.float32, device=x.device)
    check(capi().llmserve_int4_linear(_p(x), _p(inv), _p(nib), _p(gs), _p(gz), _p(y), M, N, K,
                                      group, _stream()))
    return y


def int4_linear_gemm(x, nib, gs, gz, group, inv=None):
    M, K = x.shape
    N = nib.shape[0]
    y = torch.empty(M, N, dtype=torch.float32, device=x.device)
    L = capi()
    nbytes = L.llmserve_int4_linear_gemm_workspace_bytes(M, K)
    ws = torch.empty(max(nbytes, 16) // 4 + 4, dtype=torch.float32, device=x.device)
    check(L.llmserve_int4_linear_gemm(_p(x), _p(inv), _p(nib), _p(gs), _p(gz), _p(y), M, N, K,
                                      group, _p(ws), nbytes, _stream()))
    return y


def int4_gemm_pack(nib, gs, gz, group):
    N, K = nib.shape[0], nib.shape[1] * 2
    L = capi()
    nbytes = L.llmserve_int4_gemm_pack_bytes(N, K, group)
    packed = torch.empty(max(nbytes, 16), dtype=torch.uint8, device=nib.device)
    check(L.llmserve_int4_gemm_pack(_p(nib), _p(gs), _p(gz), N, K, group, _p(packed), nbytes,
                                    _stream()))
    return packed[:nbytes]


def int4_linear_gemm_packed(x, packed, N, group, inv=None):
    M, K = x.shape
    y = torch.empty(M, N, dtype=torch.float32, device=x.device)
    L = capi()
    nbytes = L.llmserve_int4_linear_gemm_packed_workspace_bytes(M, K)
    ws = torch.empty(max(nbytes, 16) // 4 + 4, dtype=torch.float32, device=x.device)
    check(L.llmserve_int4_linear_gemm_packed(_p(x), _p(inv), _p(packed), _p(y), M, N, K, group,
                                             _p(ws), nbytes, _stream()))
    return y


def int8_linear_prefill(x, q, s):
    M, K = x.shape
    N = q.shape[0]
    y = torch.empty(M, N, dtype=torch.float32, device=x.device)
    L = capi()
    nbytes = L.llmserve_int8_linear_prefill_workspace_bytes(M, N, K)
    ws = torch.empty(max(nbytes, 16) // 4 + 4, dtype=torch.float32, device=x.device)
    check(L.llmserve_int8_linear_prefill(_p(x), _p(q), _p(s), _p(y), M, N, K, _p(ws), nbytes,
                                         _stream()))
    return y


def paged_decode_int8(q, kc, vc, ks, vs, bt, cl, block_size, scale, partition_size=0, q_mult=None):
    B, Hq, D = q.shape
    num_slots, Hk = kc.shape[0], kc.shape[1]
    max_blocks = bt.shape[1]
    out = torch.empty_like(q)
    L = capi()
    nbytes = L.llmserve_paged_attention_workspace_bytes(B, Hq, Hk, D, max_blocks, block_size,
                                                        partition_size)
    ws = torch.empty(max(nbytes, 4) // 4 + 4, dtype=torch.float32, device=q.device)
    check(L.llmserve_paged_attention_decode_int8(
        _p(q), _p(kc), _p(vc), _p(ks), _p(vs), _p(bt), _p(cl), _p(out), B, Hq, Hk, D, num_slots,
        max_blocks, block_size, float(scale), partition_size, _p(q_mult), _p(ws), nbytes,
        _stream()))
    return out


def paged_decode_int8_xfrag(q, kc, vc, ks, vs, bt, cl, block_size, scale, partition_size=0,
                            q_mult=None, act_inv=None):
    """The decode whose merge also writes the [B, Hq*D] output times act_inv as activation
    fragments: (out, fragment bytes)."""
    B, Hq, D = q.shape
    num_slots, Hk = kc.shape[0], kc.shape[1]
    max_blocks = bt.shape[1]
    out = torch.empty_like(q)
    L = capi()
    nbytes = L.llmserve_paged_attention_workspace_bytes(B, Hq, Hk, D, max_blocks, block_size,
                                                        partition_size)
    ws = torch.empty(max(nbytes, 4) // 4 + 4, dtype=torch.float32, device=q.device)
    nx = L.llmserve_int4_xfrag_bytes(B, Hq * D)
    xf = torch.empty(max(nx, 16), dtype=torch.uint8, device=q.device)
    check(L.llmserve_paged_attention_decode_int8_xfrag(
        _p(q), _p(kc), _p(vc), _p(ks), _p(vs), _p(bt), _p(cl), _p(out), _p(act_inv), _p(xf), B,
        Hq, Hk, D, num_slots, max_blocks, block_size, float(scale), partition_size, _p(q_mult),
        _p(ws), nbytes, _stream()))
    return out, xf[:nx]


def paged_decode_f32(q, kc, vc, bt, cl, block_size, scale, partition_size=0):
    """The fp32-cache decode (llmserve_paged_attention_decode)."""
    B, Hq, D = q.shape
    num_slots, Hk = kc.shape[0], kc.shape[1]
    max_blocks = bt.shape[1]
    out = torch.empty_like(q)
    L = capi()
    nbytes = L.llmserve_paged_attention_workspace_bytes(B, Hq, Hk, D, max_blocks, block_size,
                                                        partition_size)
    ws = torch.empty(max(nbytes, 4) // 4 + 4, dtype=torch.float32, device=q.device)
    check(L.llmserve_paged_attention_decode(
        _p(q), _p(kc), _p(vc), _p(bt), _p(cl), _p(out), B, Hq, Hk, D, num_slots, max_blocks,
        block_size, float(scale), partition_size, _p(ws), nbytes, _stream()))
    return out


def paged_rows(q, kc, vc, ks, vs, bt, row_table, row_context, block_size, scale, q_mult=None):
    """Attention of query rows over block-table rows (llmserve_paged_attention_rows_int8 when
    ks / vs are given, else _f32)."""
    R, Hq, D = q.shape
    num_slots, Hk = kc.shape[0], kc.shape[1]
    max_blocks = bt.shape[1]
    out = torch.empty_like(q)
    L = capi()
    nbytes = L.llmserve_paged_attention_workspace_bytes(R, Hq, Hk, D, max_blocks, block_size, 0)
    ws = torch.empty(max(nbytes, 4) // 4 + 4, dtype=torch.float32, device=q.device)
    if ks is not None:
        check(L.llmserve_paged_attention_rows_int8(
            _p(q), _p(kc), _p(vc), _p(ks), _p(vs), _p(bt), bt.shape[0], _p(row_table),
            _p(row_context), _p(out), R, Hq, Hk, D, num_slots, max_blocks, block_size,
            float(scale), _p(q_mult), _p(ws), nbytes, _stream()))
    else:
        check(L.llmserve_paged_attention_rows_f32(
            _p(q), _p(kc), _p(vc), _p(bt), bt.shape[0], _p(row_table), _p(row_context), _p(out),
            R, Hq, Hk, D, num_slots, max_blocks, block_size, float(scale), _p(q_mult), _p(ws),
            nbytes, _stream()))
    return out


def attention_metadata(seq_info, tables, block_size, T):
    """(slot_mapping, row_table, row_context) of a step (llmserve_attention_metadata)."""
    S, width = tables.shape
    dev = tables.device
    slots = torch.empty(T, dtype=torch.long, device=dev)
    rows = torch.empty(T, dtype=torch.long, device=dev)
    ctx = torch.empty(T, dtype=torch.long, device=dev)
    check(capi().llmserve_attention_metadata(_p(seq_info), _p(tables), S, width, block_size, T,
                                             _p(slots), _p(rows), _p(ctx), _stream()))
    return slots, rows, ctx


def split_fragments(x, inv=None):
    """The activation fragments of x * inv (llmserve_int4_xfrag_split: the split pass of
    llmserve_int4_linear_gemm_packed above 16 rows) as a uint8 tensor."""
    M, K = x.shape
    L = capi()
    nbytes = L.llmserve_int4_xfrag_bytes(M, K)
    ws = torch.zeros(max(nbytes, 16), dtype=torch.uint8, device=x.device)
    check(L.llmserve_int4_xfrag_split(_p(x), _p(inv), _p(ws), M, K, nbytes, _stream()))
    return ws[:nbytes]


def assert_rel_close(got, ref, tol: float, what: str = ""):
    """max|got - ref| <= tol * max|ref| and ||got - ref|| / ||ref|| <= tol."""
    g = np.asarray(got.detach().cpu() if isinstance(got, torch.Tensor) else got, np.float64)
    r = np.asarray(ref.detach().cpu() if isinstance(ref, torch.Tensor) else ref, np.float64)
    assert g.shape == r.shape, (g.shape, r.shape)
    scale = np.abs(r).max() if r.size else 0.0
    err = np.abs(g - r).max() if r.size else 0.0
    rel = np.linalg.norm(g - r) / max(np.linalg.norm(r), 1e-30)
    assert err <= tol * max(scale, 1e-30) and rel <= tol, (
        f"{what}: max-abs {err:.3e} vs {tol:.1e}*{scale:.3e}, rel-L2 {rel:.3e}")
