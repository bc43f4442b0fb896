"""Weight-only quantization on MI355X: int8 per-channel and AWQ-scaled int4 group-wise.

Drop-in for the reference's ``llmserve.quant`` (src/llmserve/quant.py). Quantization runs
on the GPU in HIP kernels that reproduce the reference's torch CPU arithmetic bit for bit
(IEEE division, round-half-even, no contraction); the decode-time linears call the
dequant-in-register HIP GEMVs. Tensors live on a ROCm device: a CPU ``nn.Linear`` is moved to
the current GPU when it is quantized.

Kernel switches (class attributes, as in the reference, quant.py:35-37 and :123-124):
  Int8Linear.kernel: "auto" | "gemv" | "prefill" | "dequant" | "aten" | "w8a8"
  Int4Linear.kernel: "auto" | "gemv" | "gemm" | "gemm_ref" | "aten"
"auto" runs the HIP GEMV up to ``gemv_max_rows`` activation rows and the bf16-MFMA prefill
GEMM above. "dequant"/"aten" multiply by the dequantized weight with torch (the reference's
exact large-M path, quant.py:71-72; there is no aten int8pack kernel for ROCm). "w8a8" keeps the
reference's per-token int8 activation path (quant.py:51-56) in torch ops.
"""

from __future__ import annotations

import torch
from torch import nn

from llmserve.kernels import load_int8_gemv, load_quant


def _gpu(device: torch.device | str | None) -> torch.device:
    """The ROCm device to quantize on: `device` if it is one, else the current GPU."""
    d = torch.device(device) if device is not None else None
    if d is not None and d.type == "cuda":
        return d
    if not torch.cuda.is_available():
        raise RuntimeError("llmserve quantized linears need a ROCm GPU (no device is visible)")
    return torch.device("cuda", torch.cuda.current_device())


def swap_linears(module: nn.Module, factory) -> int:
    """Replace every ``nn.Linear`` child (recursively) with ``factory(linear)``
    (reference: src/llmserve/models/layers.py:117-126)."""
    n = 0
    for name, child in module.named_children():
        if isinstance(child, nn.Linear):
            setattr(module, name, factory(child))
            n += 1
        else:
            n += swap_linears(child, factory)
    return n


class Int8Linear(nn.Module):
    """Int8 weights, one fp32 scale per output channel (reference quant.py:22-79).

    ``scale = max(amax|w| / 127, 1e-8)``, ``q = clamp(round(w / scale), -127, 127)``, computed
    by ``llmserve_int8_quantize`` (bit-exact with quant.py:41-43).
    """

    # GEMV up to this many rows. The reference switches to W8A8 above 4 rows on its CPU;
    # on MI355X the weight-streaming GEMV stays HBM-bound up to 16 rows.
    gemv_max_rows = 16
    kernel = "auto"

    def __init__(self, linear: nn.Linear, device: torch.device | str | None = None) -> None:
        super().__init__()
        dev = _gpu(linear.weight.device if device is None else device)
        w = linear.weight.detach().to(device=dev, dtype=torch.float32).contiguous()
        q, scale = load_quant().int8_quantize(w)
        self.register_buffer("qweight", q)
        self.register_buffer("scale", scale)
        bias = linear.bias
        self.bias = (
            None if bias is None else nn.Parameter(bias.detach().to(dev).clone(), False)
        )
        self.in_features, self.out_features = linear.in_features, linear.out_features
        self._qweight_t = None  # [in, out] int8 for the w8a8 path, built lazily

    def _w8a8(self, x2: torch.Tensor) -> torch.Tensor:
        if self._qweight_t is None:
            self._qweight_t = self.qweight.t().contiguous()
        xs = (x2.abs().amax(dim=1, keepdim=True) / 127.0).clamp_min(1e-8)
        xq = torch.round(x2 / xs).clamp(-127, 127).to(torch.int8)
        return torch._int_mm(xq, self._qweight_t).float() * xs * self.scale

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        shape = x.shape
        x2 = x.reshape(-1, shape[-1]).contiguous()
        path = self.kernel
        rows = x2.shape[0]
        if path == "auto":
            path = "gemv" if rows <= self.gemv_max_rows else "prefill"
        if path == "gemv" and rows > 64:
            path = "prefill"
        if path == "prefill" and self.in_features % 64 != 0:
            path = "dequant"  # the MFMA GEMM steps K by 64
        if path == "gemv":
            y = load_int8_gemv().int8_linear(x2, self.qweight, self.scale)
        elif path == "prefill":
            y = load_int8_gemv().int8_linear_prefill(x2, self.qweight, self.scale)
        elif path == "w8a8":
            y = self._w8a8(x2)
        elif path in ("dequant", "aten"):
            y = x2 @ self.dequantize().t()
        else:
            raise ValueError(f"unknown Int8Linear kernel {path!r}")
        y = y.reshape(*shape[:-1], self.out_features)
        return y if self.bias is None else y + self.bias

    def dequantize(self) -> torch.Tensor:
        return self.qweight.float() * self.scale[:, None]


def _unpack_nibbles(nibbles: torch.Tensor) -> torch.Tensor:
    """uint8 [N, K/2] -> int32 [N, K]; byte j holds channel 2j (low) and 2j+1 (high)."""
    lo = (nibbles & 0xF).to(torch.int32)
    hi = (nibbles >> 4).to(torch.int32)
    return torch.stack([lo, hi], dim=-1).reshape(nibbles.shape[0], -1)


def _int4_quantize(w: torch.Tensor, group_size: int):
    """Asymmetric 4-bit, one (scale, zero) per group (reference quant.py:82-90).

    Returns (q int32 [N, K], scale [N, G], zero [N, G]) with ``zero = mn + 8 * scale``,
    computed on the GPU by ``llmserve_int4_quantize``.
    """
    dev = _gpu(w.device)
    w = w.detach().to(device=dev, dtype=torch.float32).contiguous()
    if w.shape[1] % group_size:
        raise ValueError(f"in_features {w.shape[1]} not divisible by group {group_size}")
    nib, scale, zero, _ = load_quant().int4_quantize(w, group_size)
    return _unpack_nibbles(nib), scale, zero


class Int4Linear(nn.Module):
    """Group-wise asymmetric int4 with optional AWQ scaling (reference quant.py:93-151).

    With ``act_scale`` s, ``W * s`` is quantized and activations are multiplied by ``1 / s``
    at run time; the HIP GEMV applies that pre-scale while staging x, so the product is the
    same fp32 ``x * inv_act_scale`` the reference computes.
    """

    max_fused_rows = 16  # the reference's GEMV limit (quant.py:123): above it, the large-M path
    gemv_max_rows = 4  # the HIP GEMV's rows when the packed matrix-core kernel applies
    max_packed_rows = 256  # up to this: the decode-batch kernel on the packed weight
    # "auto": the HIP GEMV up to gemv_max_rows rows (its straight-line kernel; measured at the
    # Qwen3-0.6B shapes, the matrix-core kernel ties it from 6 rows and is ~2x faster from 12),
    # then the HIP matrix-core GEMM on the packed weight ("gemm", K and group multiples of 128)
    # up to max_packed_rows rows; without a packed weight the GEMV up to max_fused_rows rows;
    # beyond, the matrix-core GEMM on the reference layout ("gemm_ref", out also a multiple of
    # 16), else dequantize + GEMM ("aten", the reference's large-M algorithm). Each name
    # forces its kernel for every batch.
    kernel = "auto"

    def __init__(
        self,
        linear: nn.Linear,
        group_size: int = 64,
        act_scale: torch.Tensor | None = None,
        device: torch.device | str | None = None,
    ) -> None:
        super().__init__()
        self.in_features, self.out_features = linear.in_features, linear.out_features
        if self.in_features % group_size:
            raise ValueError(f"in_features {self.in_features} not divisible by group {group_size}")
        dev = _gpu(linear.weight.device if device is None else device)
        w = linear.weight.detach().to(device=dev, dtype=torch.float32).contiguous()
        s = None
        if act_scale is not None:
            s = act_scale.detach().to(device=dev, dtype=torch.float32).contiguous()
        nib, g_scale, g_zero, inv = load_quant().int4_quantize(w, group_size, s)
        self.group_size = group_size
        if s is not None:
            self.register_buffer("inv_act_scale", inv)
        else:
            self.inv_act_scale = None
        self.register_buffer("nibbles", nib)  # [out, in/2]
        self.register_buffer("g_scale", g_scale)  # [out, n_groups]
        self.register_buffer("g_zero", g_zero)
        # the same weight rearranged for the batched matrix-core kernel (not saved: it is a
        # function of the three buffers above)
        packed = None
        if self.in_features % 128 == 0 and group_size % 128 == 0:
            packed = load_int8_gemv().int4_gemm_pack(nib, g_scale, g_zero, group_size)
        self.register_buffer("gemm_packed", packed, persistent=False)
        self.bias = (
            None if linear.bias is None else nn.Parameter(linear.bias.detach().to(dev).clone(), False)
        )

    def dequantize(self) -> torch.Tensor:
        """fp32 weight [out, in] of the (scaled) quantized matrix."""
        lo = (self.nibbles & 0xF).float()
        hi = (self.nibbles >> 4).float()
        q = torch.stack([lo, hi], dim=-1).reshape(self.out_features, -1, self.group_size)
        w = (q - 8) * self.g_scale[..., None] + self.g_zero[..., None]
        return w.reshape(self.out_features, self.in_features)

    def packed_path(self, rows: int) -> bool:
        """``kernel="auto"`` runs the packed matrix-core kernel for ``rows`` activation rows."""
        return (self.kernel == "auto" and self.gemm_packed is not None
                and self.gemv_max_rows < rows <= self.max_packed_rows)

    def gemm_ok(self) -> bool:
        """Shapes the reference-layout matrix-core kernel (int4_linear_gemm) takes."""
        return (self.in_features % 128 == 0 and self.group_size % 128 == 0
                and self.out_features % 16 == 0)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        shape = x.shape
        x2 = x.reshape(-1, shape[-1])
        rows = x2.shape[0]
        if self.kernel == "auto":
            if self.packed_path(rows):
                path = "gemm"
            elif rows <= self.max_fused_rows:
                path = "gemv"
            elif self.gemm_packed is not None and not self.gemm_ok():
                path = "gemm"
            else:
                path = "gemm_ref" if self.gemm_ok() else "aten"
        elif self.kernel in ("gemv", "gemm", "gemm_ref", "aten"):
            path = self.kernel
        else:
            raise ValueError(f"unknown Int4Linear kernel {self.kernel!r}")
        if path == "gemm" and self.gemm_packed is None:
            raise ValueError("Int4Linear: the packed matrix-core kernel needs in_features and "
                             "group_size multiples of 128")
        if path == "aten":
            if self.inv_act_scale is not None:
                x2 = x2 * self.inv_act_scale
            y = x2 @ self.dequantize().t()
        elif path == "gemm":
            y = load_int8_gemv().int4_linear_gemm_packed(x2.contiguous(), self.gemm_packed,
                                                         self.out_features, self.group_size,
                                                         self.inv_act_scale)
        else:
            fn = load_int8_gemv().int4_linear if path == "gemv" else load_int8_gemv().int4_linear_gemm
            y = fn(x2.contiguous(), self.nibbles, self.g_scale, self.g_zero, self.group_size,
                   self.inv_act_scale)
        y = y.reshape(*shape[:-1], self.out_features)
        return y if self.bias is None else y + self.bias


def _search_awq_scale(w: torch.Tensor, x: torch.Tensor, group_size: int) -> torch.Tensor:
    """Pick s = mean|x|^alpha (alpha on a grid) minimizing ||x W^T - (x/s) Q(W s)^T||
    (reference quant.py:154-170). Same torch ops, on the GPU, with the HIP int4 quantizer.
    The chosen alpha can differ from a CPU run only where two grid points tie to within the
    fp32 GEMM rounding of the two devices."""
    dev = _gpu(w.device)
    w = w.detach().to(device=dev, dtype=torch.float32)
    x = x.detach().to(device=dev, dtype=torch.float32)
    act = x.abs().mean(0).clamp_min(1e-5)
    ref = x @ w.t()
    best, best_s = float("inf"), None
    for alpha in [i / 10 for i in range(11)]:
        s = act.pow(alpha)
        s = s / (s.max() * s.min()).sqrt()  # keep scales centered around 1
        q, scale, zero = _int4_quantize(w * s[None, :], group_size)
        deq = (q.float().reshape(w.shape[0], -1, group_size) - 8) * scale[..., None] + zero[
            ..., None
        ]
        deq = deq.reshape(w.shape) / s[None, :]
        err = (x @ deq.t() - ref).pow(2).mean().item()
        if err < best:
            best, best_s = err, s
    return best_s


def quantize_model(
    model: nn.Module,
    method: str,
    group_size: int = 64,
    quantize_lm_head: bool = False,
    calib_acts: dict[str, torch.Tensor] | None = None,
) -> nn.Module:
    """Swap linear layers for quantized ones in place. ``method``: int8 | int4 | int4-awq
    (reference quant.py:173-205)."""
    if method not in ("int8", "int4", "int4-awq"):
        raise ValueError(f"unknown quantization {method!r}")
    if method == "int4-awq" and not calib_acts:
        raise ValueError("int4-awq needs calibration activations (see collect_linear_inputs)")
    lm_head = model.lm_head if hasattr(model, "lm_head") else None
    names = {id(m): n for n, m in model.named_modules()}

    def factory(lin: nn.Linear) -> nn.Module:
        if lin is lm_head and not quantize_lm_head:
            return lin
        if method == "int8":
            return Int8Linear(lin)
        s = None
        if method == "int4-awq":
            x = calib_acts.get(names[id(lin)])
            if x is not None:
                s = _search_awq_scale(lin.weight.detach().float(), x, group_size)
        return Int4Linear(lin, group_size, s)

    swap_linears(model, factory)
    model.quantization = method
    return model


@torch.inference_mode()
def collect_linear_inputs(
    model: nn.Module, run_fn, max_rows: int = 2048
) -> dict[str, torch.Tensor]:
    """Record (a sample of) the inputs every ``nn.Linear`` sees while ``run_fn()`` runs
    (reference quant.py:208-233)."""
    acts: dict[str, list[torch.Tensor]] = {}
    hooks = []
    for name, mod in model.named_modules():
        if isinstance(mod, nn.Linear):

            def hook(m, inp, out, name=name):
                acts.setdefault(name, []).append(inp[0].reshape(-1, inp[0].shape[-1]).detach())

            hooks.append(mod.register_forward_hook(hook))
    try:
        run_fn()
    finally:
        for h in hooks:
            h.remove()
    out = {}
    for name, xs in acts.items():
        x = torch.cat(xs)
        if x.shape[0] > max_rows:
            perm = torch.randperm(x.shape[0], generator=torch.Generator().manual_seed(0))
            x = x[perm[:max_rows].to(x.device)]
        out[name] = x
    return out


def weight_bytes(model: nn.Module) -> int:
    """Bytes of parameters + buffers (tied tensors counted once), excluding RoPE tables
    (reference quant.py:236-248)."""
    seen, total = set(), 0
    for name, t in list(model.named_parameters()) + list(model.named_buffers()):
        try:
            key = t.data_ptr()
        except RuntimeError:
            key = id(t)
        if "rope" in name or key in seen:
            continue
        seen.add(key)
        total += t.numel() * t.element_size()
    return total
