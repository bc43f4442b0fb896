"""Weight-only quantization: int8 per output channel and AWQ-scaled int4 per group.

Drop-in for the reference's ``llmserve.quant`` (src/llmserve/quant.py): the same classes,
buffers and functions. On a ROCm device the quantizers are HIP kernels that reproduce the
reference's torch CPU arithmetic bit for bit (IEEE division, round half to even, no
contraction), and the linears run this package's HIP kernels: the dequant-in-register GEMV for
decode rows, the packed matrix-core kernel for decode batches, the bf16 matrix-core GEMM for
prefill-sized inputs. On the CPU, or when the native library is missing (``load_* is None``),
the same formulas run as torch ops, as the reference's fallbacks do. A module lives on the
device of the ``nn.Linear`` it replaces (or ``device=``).

Kernel switches (class attributes, as in the reference, quant.py:35-37 and :123-124):
  Int8Linear.kernel: "auto" | "gemv" | "prefill" | "dequant" | "aten" | "w8a8"
  Int4Linear.kernel: "auto" | "gemv" | "gemm" | "gemm_ref" | "aten"
"""

from __future__ import annotations

import itertools
from collections import defaultdict

import torch
from torch import nn

from .kernels import load_int8_gemv, load_quant

QUANT_METHODS = ("int8", "int4", "int4-awq")


def _target(linear: nn.Linear, device) -> torch.device:
    return torch.device(device) if device is not None else linear.weight.device


def _native(kind: str, dev: torch.device):
    """The native op namespace for tensors on ``dev`` (None on the CPU or without the
    library)."""
    if dev.type != "cuda":
        return None
    return load_quant() if kind == "quant" else load_int8_gemv()


def swap_linears(module: nn.Module, factory) -> int:
    """Replace every ``nn.Linear`` below ``module`` with ``factory(linear)``; returns how many
    (reference: src/llmserve/models/layers.py:117-126)."""
    swapped = 0
    for name, child in list(module.named_children()):
        if isinstance(child, nn.Linear):
            setattr(module, name, factory(child))
            swapped += 1
        else:
            swapped += swap_linears(child, factory)
    return swapped


# ---- int8 ----------------------------------------------------------------------------------------


def _absmax_int8(t: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-row symmetric int8 of a [rows, cols] tensor with torch ops: scale = max(max|row| /
    127, 1e-8) (divide, then clamp: quant.py:42 and :54), q = clamp(round_half_even(t / scale),
    +-127)."""
    scale = torch.clamp(t.abs().amax(dim=1) / 127.0, min=1e-8)
    q = torch.clamp(torch.round(t / scale.unsqueeze(1)), -127, 127).to(torch.int8)
    return q, scale


class Int8Linear(nn.Module):
    """int8 weights with one fp32 scale per output channel (reference quant.py:22-79)."""

    # GEMV up to this many activation rows. The reference switches to W8A8 above 4 rows on
    # its CPU; on MI355X the weight-streaming GEMV stays ahead up to 16.
    gemv_max_rows = 16
    kernel = "auto"

    def __init__(self, linear: nn.Linear, device: torch.device | str | None = None) -> None:
        super().__init__()
        dev = _target(linear, device)
        w = linear.weight.detach().to(device=dev, dtype=torch.float32).contiguous()
        ops = _native("quant", dev)
        q, scale = ops.int8_quantize(w) if ops is not None else _absmax_int8(w)
        self.register_buffer("qweight", q)
        self.register_buffer("scale", scale.contiguous())
        self.bias = None
        if linear.bias is not None:
            self.bias = nn.Parameter(linear.bias.detach().to(dev).clone(), requires_grad=False)
        self.in_features, self.out_features = linear.in_features, linear.out_features
        self._qweight_t = None  # [in, out] copy for the W8A8 path, made on first use

    def dequantize(self) -> torch.Tensor:
        return self.qweight.to(torch.float32) * self.scale.unsqueeze(1)

    def _w8a8(self, x2: torch.Tensor) -> torch.Tensor:
        """Per-token int8 activations times the int8 weight (reference quant.py:51-56)."""
        if self._qweight_t is None:
            self._qweight_t = self.qweight.t().contiguous()
        xq, xs = _absmax_int8(x2)
        return torch._int_mm(xq, self._qweight_t).float() * xs.unsqueeze(1) * self.scale

    def _path(self, rows: int, native) -> str:
        path = self.kernel
        if path not in ("auto", "gemv", "prefill", "dequant", "aten", "w8a8"):
            raise ValueError(f"unknown Int8Linear kernel {path!r}")
        if path == "auto":
            path = "gemv" if rows <= self.gemv_max_rows else "prefill"
        if native is None and path in ("gemv", "prefill"):
            return "aten"
        if path == "gemv" and rows > 64:  # the GEMV's row limit (int8_gemv.cpp:22)
            path = "prefill"
        if path == "prefill" and self.in_features % 64:
            path = "dequant"  # the matrix-core GEMM steps K by 64
        return path

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        lead = x.shape[:-1]
        x2 = x.reshape(-1, x.shape[-1]).contiguous()
        native = _native("gemv", x2.device)
        path = self._path(x2.shape[0], native)
        if path == "gemv":
            y = native.int8_linear(x2, self.qweight, self.scale)
        elif path == "prefill":
            y = native.int8_linear_prefill(x2, self.qweight, self.scale)
        elif path == "w8a8":
            y = self._w8a8(x2)
        elif path == "aten" and x2.device.type == "cpu":
            y = torch.ops.aten._weight_int8pack_mm(x2, self.qweight, self.scale)
        else:
            y = x2 @ self.dequantize().t()
        y = y.reshape(*lead, self.out_features)
        return y if self.bias is None else y + self.bias


# ---- int4 ----------------------------------------------------------------------------------------


def _unpack_nibbles(nibbles: torch.Tensor) -> torch.Tensor:
    """uint8 [N, K/2] -> int32 [N, K]; byte j holds channel 2j (low) and 2j+1 (high)."""
    pair = torch.stack((nibbles & 0xF, nibbles >> 4), dim=-1)
    return pair.reshape(nibbles.shape[0], -1).to(torch.int32)


def _pack_nibbles(q: torch.Tensor) -> torch.Tensor:
    """int [N, K] in [0, 15] -> uint8 [N, K/2], even channel in the low nibble (quant.py:113)."""
    q8 = q.to(torch.uint8)
    return ((q8[:, 1::2] << 4) | q8[:, 0::2]).contiguous()


def _dequant_groups(q: torch.Tensor, scale: torch.Tensor, zero: torch.Tensor,
                    group_size: int) -> torch.Tensor:
    """w = (q - 8) * scale + zero per group (the kernel convention of quant.py:89), float32."""
    n = q.shape[0]
    g = q.to(torch.float32).reshape(n, -1, group_size)
    return ((g - 8) * scale.unsqueeze(-1) + zero.unsqueeze(-1)).reshape(n, -1)


def _int4_groups_torch(w: torch.Tensor, group_size: int):
    """Asymmetric 4-bit per group with torch ops (reference quant.py:82-90): scale =
    max((max - min) / 15, 1e-8), q = clamp(round_half_even((w - min) / scale), 0, 15),
    zero = min + 8 * scale."""
    n, k = w.shape
    grp = w.reshape(n, k // group_size, group_size)
    lo, hi = grp.amin(dim=-1, keepdim=True), grp.amax(dim=-1, keepdim=True)
    scale = torch.clamp((hi - lo) / 15.0, min=1e-8)
    q = torch.clamp(torch.round((grp - lo) / scale), 0, 15).to(torch.int32).reshape(n, k)
    return q, scale.squeeze(-1), (lo + 8.0 * scale).squeeze(-1)


def _int4_quantize(w: torch.Tensor, group_size: int):
    """(q int32 [N, K], scale [N, G], zero [N, G]) of ``w`` on its device: the
    ``llmserve_int4_quantize`` HIP kernel on a ROCm device, torch ops elsewhere."""
    w = w.detach().to(torch.float32).contiguous()
    if w.shape[1] % group_size:
        raise ValueError(f"in_features {w.shape[1]} not divisible by group {group_size}")
    ops = _native("quant", w.device)
    if ops is None:
        return _int4_groups_torch(w, group_size)
    nib, scale, zero, _ = ops.int4_quantize(w, group_size)
    return _unpack_nibbles(nib), scale, zero


class Int4Linear(nn.Module):
    """Group-wise asymmetric int4 with optional AWQ scaling (reference quant.py:93-151).

    With ``act_scale`` s the layer quantizes ``W * s`` and multiplies activations by ``1 / s``
    at run time; the HIP kernels apply that pre-scale while loading x (the same float32
    product).
    """

    max_fused_rows = 16  # the reference's GEMV limit (quant.py:123)
    gemv_max_rows = 4  # the HIP GEMV's rows when the packed matrix-core kernel applies
    max_packed_rows = 256  # up to this: the decode-batch kernel on the packed weight
    # "auto": the HIP GEMV up to gemv_max_rows rows, the matrix-core kernel on the packed weight
    # ("gemm", K and group multiples of 128) up to max_packed_rows, the GEMV up to
    # max_fused_rows when there is no packed weight, then the matrix-core GEMM on the reference
    # layout ("gemm_ref") or dequantize + GEMM ("aten", the reference's large-M algorithm).
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
        self.group_size = group_size
        dev = _target(linear, device)
        w = linear.weight.detach().to(device=dev, dtype=torch.float32).contiguous()
        s = None if act_scale is None else act_scale.detach().to(dev, torch.float32).contiguous()
        ops = _native("quant", dev)
        if ops is not None:
            nib, g_scale, g_zero, inv = ops.int4_quantize(w, group_size, s)
        else:
            q, g_scale, g_zero = _int4_groups_torch(w * s[None, :] if s is not None else w,
                                                    group_size)
            nib, inv = _pack_nibbles(q), (1.0 / s if s is not None else None)
        if s is not None:
            self.register_buffer("inv_act_scale", inv.contiguous())
        else:
            self.inv_act_scale = None
        self.register_buffer("nibbles", nib)  # [out, in / 2]
        self.register_buffer("g_scale", g_scale.contiguous())  # [out, groups]
        self.register_buffer("g_zero", g_zero.contiguous())
        # The weight rearranged for the decode-batch matrix-core kernel (not saved: it is a
        # function of the three buffers above).
        packed = None
        gemv = _native("gemv", dev)
        if gemv is not None and self.in_features % 128 == 0 and group_size % 128 == 0:
            packed = gemv.int4_gemm_pack(nib, g_scale, g_zero, group_size)
        self.register_buffer("gemm_packed", packed, persistent=False)
        self.bias = None
        if linear.bias is not None:
            self.bias = nn.Parameter(linear.bias.detach().to(dev).clone(), requires_grad=False)

    def dequantize(self) -> torch.Tensor:
        """fp32 [out, in] weight of the (AWQ-scaled) quantized matrix."""
        return _dequant_groups(_unpack_nibbles(self.nibbles), self.g_scale, self.g_zero,
                               self.group_size)

    def packed_path(self, rows: int) -> bool:
        """``kernel="auto"`` runs the packed matrix-core kernel for ``rows`` activation rows."""
        return (self.kernel == "auto" and self.gemm_packed is not None
                and self.gemv_max_rows < rows <= self.max_packed_rows)

    def gemm_ok(self) -> bool:
        """Shapes the reference-layout matrix-core kernel (int4_linear_gemm) takes."""
        return (self.in_features % 128 == 0 and self.group_size % 128 == 0
                and self.out_features % 16 == 0)

    def _path(self, rows: int, native) -> str:
        if self.kernel not in ("auto", "gemv", "gemm", "gemm_ref", "aten"):
            raise ValueError(f"unknown Int4Linear kernel {self.kernel!r}")
        if native is None:
            return "aten"
        if self.kernel != "auto":
            if self.kernel == "gemm" and self.gemm_packed is None:
                raise ValueError("Int4Linear: the packed matrix-core kernel needs in_features and "
                                 "group_size multiples of 128")
            return self.kernel
        if self.packed_path(rows):
            return "gemm"
        if rows <= self.max_fused_rows:
            return "gemv"
        if self.gemm_packed is not None and not self.gemm_ok():
            return "gemm"
        return "gemm_ref" if self.gemm_ok() else "aten"

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        lead = x.shape[:-1]
        x2 = x.reshape(-1, x.shape[-1])
        native = _native("gemv", x2.device)
        path = self._path(x2.shape[0], native)
        if path == "aten":
            xs = x2 * self.inv_act_scale if self.inv_act_scale is not None else x2
            y = xs @ self.dequantize().t()
        elif path == "gemm":
            y = native.int4_linear_gemm_packed(x2.contiguous(), self.gemm_packed,
                                               self.out_features, self.group_size,
                                               self.inv_act_scale)
        else:
            fn = native.int4_linear if path == "gemv" else native.int4_linear_gemm
            y = fn(x2.contiguous(), self.nibbles, self.g_scale, self.g_zero, self.group_size,
                   self.inv_act_scale)
        y = y.reshape(*lead, self.out_features)
        return y if self.bias is None else y + self.bias


# ---- AWQ scale search, model conversion, calibration --------------------------------------------

_AWQ_ALPHAS = tuple(i / 10 for i in range(11))


def _awq_candidate(act: torch.Tensor, alpha: float) -> torch.Tensor:
    """s = act^alpha, divided by sqrt(max(s) * min(s)) so that the scales centre on 1."""
    s = act.pow(alpha)
    return s / (s.max() * s.min()).sqrt()


def _search_awq_scale(w: torch.Tensor, x: torch.Tensor, group_size: int) -> torch.Tensor:
    """Per-input-channel AWQ scale: the candidate ``mean|x|^alpha`` (alpha on a 0.1 grid) whose
    int4 quantization of ``W * s`` gives the least mean squared output error on the calibration
    rows ``x`` (reference quant.py:154-170; the first of equal minima). Runs on the device of
    ``w`` (the HIP quantizer on a ROCm device); alpha can differ from a CPU run only where two
    grid points tie to within the fp32 GEMM rounding of the two devices."""
    w = w.detach().to(torch.float32)
    x = x.detach().to(device=w.device, dtype=torch.float32)
    act = x.abs().mean(0).clamp_min(1e-5)
    target = x @ w.t()
    best_err, best_s = float("inf"), None
    for alpha in _AWQ_ALPHAS:
        s = _awq_candidate(act, alpha)
        q, scale, zero = _int4_quantize(w * s[None, :], group_size)
        approx = _dequant_groups(q, scale, zero, group_size) / s[None, :]
        err = (x @ approx.t() - target).pow(2).mean().item()
        if err < best_err:
            best_err, best_s = err, s
    return best_s


def quantize_model(
    model: nn.Module,
    method: str,
    group_size: int = 64,
    quantize_lm_head: bool = False,
    calib_acts: dict[str, torch.Tensor] | None = None,
) -> nn.Module:
    """Replaces the model's ``nn.Linear`` layers in place (reference quant.py:173-205):
    ``method`` int8 | int4 | int4-awq; ``calib_acts`` (int4-awq) maps a linear's qualified name
    to its calibration inputs; the ``lm_head`` stays fp32 unless ``quantize_lm_head``."""
    if method not in QUANT_METHODS:
        raise ValueError(f"unknown quantization {method!r}")
    if method == "int4-awq" and not calib_acts:
        raise ValueError("int4-awq needs calibration activations (see collect_linear_inputs)")
    skip = None if quantize_lm_head else getattr(model, "lm_head", None)
    qualified = {id(m): name for name, m in model.named_modules()}

    def replace(lin: nn.Linear) -> nn.Module:
        if lin is skip:
            return lin
        if method == "int8":
            return Int8Linear(lin)
        scale = None
        calib = calib_acts.get(qualified[id(lin)]) if method == "int4-awq" else None
        if calib is not None:
            scale = _search_awq_scale(lin.weight.detach().float(), calib, group_size)
        return Int4Linear(lin, group_size, scale)

    swap_linears(model, replace)
    model.quantization = method
    return model


class _LinearInputRecorder:
    """Forward hooks on every ``nn.Linear`` of a model that keep the rows each one sees."""

    def __init__(self, model: nn.Module) -> None:
        self.rows: dict[str, list[torch.Tensor]] = defaultdict(list)
        self._handles = [m.register_forward_hook(self._hook(name))
                         for name, m in model.named_modules() if isinstance(m, nn.Linear)]

    def _hook(self, name: str):
        def keep(_mod, inputs, _out):
            x = inputs[0].detach()
            self.rows[name].append(x.reshape(-1, x.shape[-1]))
        return keep

    def close(self) -> None:
        for h in self._handles:
            h.remove()
        self._handles = []


def _row_sample(x: torch.Tensor, max_rows: int) -> torch.Tensor:
    """At most ``max_rows`` rows of ``x``: the first ``max_rows`` of a seed-0 permutation (the
    reference's choice, quant.py:230-231)."""
    if x.shape[0] <= max_rows:
        return x
    order = torch.randperm(x.shape[0], generator=torch.Generator().manual_seed(0))
    return x.index_select(0, order[:max_rows].to(x.device))


@torch.inference_mode()
def collect_linear_inputs(
    model: nn.Module, run_fn, max_rows: int = 2048
) -> dict[str, torch.Tensor]:
    """The inputs every ``nn.Linear`` of ``model`` receives while ``run_fn()`` runs, at most
    ``max_rows`` rows each (reference quant.py:208-233)."""
    rec = _LinearInputRecorder(model)
    try:
        run_fn()
    finally:
        rec.close()
    return {name: _row_sample(torch.cat(parts), max_rows) for name, parts in rec.rows.items()}


def weight_bytes(model: nn.Module) -> int:
    """Bytes of the model's parameters and buffers, each storage counted once (tied weights),
    RoPE tables excluded (reference quant.py:236-248)."""
    sizes: dict[object, int] = {}
    for name, t in itertools.chain(model.named_parameters(), model.named_buffers()):
        if t is None or "rope" in name:
            continue
        try:
            key = (t.untyped_storage().data_ptr(), t.storage_offset())
        except RuntimeError:  # tensors without storage
            key = id(t)
        sizes.setdefault(key, t.numel() * t.element_size())
    return sum(sizes.values())
