"""MI355X-native fused quantized SDPA decode (drop-in for mlx_qsdpa).

Public API (mlx_qsdpa/__init__.py:71-78): ``quantized_sdpa``,
``cache_sdpa`` and the four quantized caches, on PyTorch-ROCm tensors.
The kernels are hand-written HIP for gfx950 behind the C ABI of
include/qsdpa.h (``libqsdpa_hip.so``).
"""

from __future__ import annotations

from .cache import (
    BatchQuantizedRotatingSDPACache,
    BatchQuantizedSDPACache,
    QuantizedRotatingSDPACache,
    QuantizedSDPACache,
)
from .dispatch import fallback_sdpa, quantized_sdpa
from .kernels import dequantize, quantize

# Decode length below which cache_sdpa dequantizes and runs plain attention.
# The reference uses 16384, measured on an M2 Ultra (mlx_qsdpa/__init__.py:19,
# 38-39); on MI355X the fused kernel is not slower at any measured length.
DEFAULT_CROSSOVER = 0


def cache_sdpa(q, k_quant, v_quant, cache, scale=None, mask=None, crossover=None, *,
               kv_start=None):
    """Attention over a quantized cache with length-based dispatch.

    mlx_qsdpa/__init__.py:12-68: N < crossover goes through dequantize +
    attention; otherwise the fused quantized kernel.  Prefill (qL > 1),
    which the reference always dequantizes, runs fused where the
    matrix-core kernel takes the shape.
    ``crossover=None`` uses DEFAULT_CROSSOVER.  ``kv_start`` (extension) is
    forwarded to quantized_sdpa (or folded into the mask on the fallback).
    """
    D = q.shape[-1]
    qL = q.shape[2]
    N = k_quant[0].shape[2]
    if scale is None:
        scale = D ** -0.5
    if crossover is None:
        crossover = DEFAULT_CROSSOVER
    if qL == 1 and N < crossover:
        return fallback_sdpa(q, k_quant, v_quant, bits=cache.bits, group_size=cache.group_size,
                             scale=scale, mask=mask, kv_start=kv_start)
    # qL > 1: the fused kernel where it takes the shape, else the reference's
    # dequantize + attention (quantized_sdpa decides).
    return quantized_sdpa(q, k_quant[0], v_quant[0], k_quant[1], v_quant[1], k_quant[2],
                          v_quant[2], scale=scale, mask=mask, bits=cache.bits,
                          group_size=cache.group_size, kv_start=kv_start)


# The model side (needs cache_sdpa above): the router keyed on
# _use_fused_sdpa, an attention layer calling it, cache save / load.
from .attention import Attention, KVCache, scaled_dot_product_attention  # noqa: E402
from .cache_io import load_cache, save_cache  # noqa: E402

__all__ = [
    "quantized_sdpa",
    "QuantizedSDPACache",
    "BatchQuantizedSDPACache",
    "QuantizedRotatingSDPACache",
    "BatchQuantizedRotatingSDPACache",
    "cache_sdpa",
    "quantize",
    "dequantize",
    "scaled_dot_product_attention",
    "Attention",
    "KVCache",
    "save_cache",
    "load_cache",
]
