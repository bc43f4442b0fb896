"""Physical KV cache (reference: src/llmserve/kv_cache.py:21-68).

The cache is split into ``num_blocks`` fixed-size blocks of ``block_size`` token slots; each
layer holds a K and a V tensor of shape ``[num_blocks * block_size, kv_heads, head_dim]``, or,
with ``kv_dtype="int8"``, a pair of ``QuantizedKV`` (int8 data + one fp32 scale per slot and
head). ``cfg`` is any object with ``num_hidden_layers``, ``num_key_value_heads`` and
``head_dim`` (the reference's ``ModelConfig``). The block allocator of the reference module is
host bookkeeping of the scheduler and is not part of this package.
"""

from __future__ import annotations

import torch

from llmserve.attention import QuantizedKV


def _kv_bytes_per_token(cfg, dtype_bytes: int) -> int:
    # reference config.py:81-83
    return 2 * cfg.num_hidden_layers * cfg.num_key_value_heads * cfg.head_dim * dtype_bytes


class KVCache:
    """Per-layer K and V tensors of shape ``[num_blocks * block_size, kv_heads, head_dim]``."""

    def __init__(
        self,
        cfg,
        num_blocks: int,
        block_size: int,
        dtype: torch.dtype = torch.float32,
        device: str | torch.device = "cpu",
        kv_dtype: str = "auto",
    ) -> None:
        self.num_blocks = num_blocks
        self.block_size = block_size
        self.kv_dtype = kv_dtype
        shape = (num_blocks * block_size, cfg.num_key_value_heads, cfg.head_dim)
        if kv_dtype == "int8":
            self.layers = [
                (QuantizedKV(*shape, device), QuantizedKV(*shape, device))
                for _ in range(cfg.num_hidden_layers)
            ]
            return
        if kv_dtype != "auto":
            raise ValueError(f"kv_dtype must be 'auto' or 'int8', got {kv_dtype!r}")
        self.layers = [
            (
                torch.zeros(shape, dtype=dtype, device=device),
                torch.zeros(shape, dtype=dtype, device=device),
            )
            for _ in range(cfg.num_hidden_layers)
        ]

    @staticmethod
    def blocks_for_memory(
        cfg, mem_bytes: int, block_size: int, dtype_bytes: int = 4, kv_dtype="auto"
    ) -> int:
        per_token = _kv_bytes_per_token(cfg, dtype_bytes)
        if kv_dtype == "int8":  # 1 byte per element + one fp32 scale per (layer, head, K/V)
            per_token = 2 * cfg.num_hidden_layers * cfg.num_key_value_heads * (cfg.head_dim + 4)
        return max(1, mem_bytes // (per_token * block_size))

    def set_k_smoothing(self, factors: list[torch.Tensor], num_q_heads: int) -> None:
        """Install per-layer key smoothing factors (int8 KV only)."""
        assert self.kv_dtype == "int8" and len(factors) == len(self.layers)
        for (k, _), s in zip(self.layers, factors, strict=True):
            k.set_smoothing(s, num_q_heads)

    def nbytes(self) -> int:
        if self.kv_dtype == "int8":
            return sum(k.nbytes() + v.nbytes() for k, v in self.layers)
        return sum(k.numel() * k.element_size() * 2 for k, _ in self.layers)
