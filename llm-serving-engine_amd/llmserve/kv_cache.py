"""Physical KV cache (reference: src/llmserve/kv_cache.py:18-68).

``num_blocks`` blocks of ``block_size`` token slots; every layer holds a (K, V) pair of flat
``[num_blocks * block_size, kv_heads, head_dim]`` caches: float tensors of ``dtype``
(``kv_dtype="auto"``) or ``QuantizedKV`` pairs (``kv_dtype="int8"``: int8 rows plus one fp32
scale per slot and head). ``cfg`` is any object with ``num_hidden_layers``,
``num_key_value_heads`` and ``head_dim`` (the reference's ``ModelConfig``). The block allocator
of the reference module is scheduler bookkeeping and is not part of this package.
"""

from __future__ import annotations

import torch

from .attention import QuantizedKV

KV_DTYPES = ("auto", "int8")


def kv_bytes_per_token(cfg, dtype_bytes: int = 4, kv_dtype: str = "auto") -> int:
    """Cache bytes one token occupies over all layers, K and V: ``dtype_bytes`` per element,
    or for int8 one byte per element plus a 4-byte scale per kv head (reference
    config.py:81-83 and kv_cache.py:54-56)."""
    per_head = cfg.head_dim + 4 if kv_dtype == "int8" else cfg.head_dim * dtype_bytes
    return 2 * cfg.num_hidden_layers * cfg.num_key_value_heads * per_head


class KVCache:
    """Per-layer K and V caches of ``num_blocks * block_size`` slots each."""

    def __init__(
        self,
        cfg,
        num_blocks: int,
        block_size: int,
        dtype: torch.dtype = torch.float32,
        device: str | torch.device = "cpu",
        kv_dtype: str = "auto",
    ) -> None:
        if kv_dtype not in KV_DTYPES:
            raise ValueError(f"kv_dtype must be 'auto' or 'int8', got {kv_dtype!r}")
        self.num_blocks = num_blocks
        self.block_size = block_size
        self.kv_dtype = kv_dtype
        geometry = (num_blocks * block_size, cfg.num_key_value_heads, cfg.head_dim)

        def one_cache():
            if kv_dtype == "int8":
                return QuantizedKV(*geometry, device)
            return torch.zeros(geometry, dtype=dtype, device=device)

        self.layers = [(one_cache(), one_cache()) for _ in range(cfg.num_hidden_layers)]

    @staticmethod
    def blocks_for_memory(
        cfg, mem_bytes: int, block_size: int, dtype_bytes: int = 4, kv_dtype="auto"
    ) -> int:
        """How many blocks fit in ``mem_bytes`` (at least one)."""
        block_bytes = kv_bytes_per_token(cfg, dtype_bytes, kv_dtype) * block_size
        return max(1, mem_bytes // block_bytes)

    def set_k_smoothing(self, factors: list[torch.Tensor], num_q_heads: int) -> None:
        """Installs one key-smoothing factor tensor [kv_heads, head_dim] per layer (int8 only)."""
        assert self.kv_dtype == "int8", "key smoothing needs the int8 cache"
        assert len(factors) == len(self.layers), "one smoothing factor tensor per layer"
        for (k_cache, _), s in zip(self.layers, factors):
            k_cache.set_smoothing(s, num_q_heads)

    def nbytes(self) -> int:
        total = 0
        for pair in self.layers:
            for c in pair:
                total += c.nbytes() if isinstance(c, QuantizedKV) else c.numel() * c.element_size()
        return total
