"""llmserve quantized decode path on MI355X (gfx950).

Drop-in for the reference's ``llmserve.quant``, ``llmserve.attention``, ``llmserve.kv_cache``
and ``llmserve.kernels`` modules (Buland-Choudhary/llm-serving-engine, src/llmserve/): the
same classes and functions, running hand-written HIP kernels on ROCm tensors.
"""

__all__ = ["attention", "kernels", "kv_cache", "quant"]
