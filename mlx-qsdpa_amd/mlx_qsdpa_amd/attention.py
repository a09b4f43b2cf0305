"""The model side: an attention layer that routes on ``_use_fused_sdpa``.

The reference's caches carry ``_use_fused_sdpa = True`` so that the runtime
calling them can tell their ``update_and_fetch`` result -- quantized
``(packed, scales, biases)`` tuples -- from a plain cache's tensors and send
it to the fused kernel (mlx_qsdpa/cache.py:57-71, 241-242; README.md:274-278:
the router itself lives downstream).  Here that router is
``scaled_dot_product_attention``, and ``Attention`` is a grouped-query
attention layer (rotary positions at the cache's offsets) that calls it the
way a model's layer calls its runtime's attention hook:

    k, v = cache.update_and_fetch(k, v)
    out = scaled_dot_product_attention(q, k, v, cache=cache, scale=..., mask=...)

A quantized cache goes to ``cache_sdpa`` (the HIP kernels); anything else
(``KVCache`` below, or no cache) goes to a plain float32 attention.
"""

from __future__ import annotations

import math

import torch
from torch import nn

from . import cache_sdpa, kernels
from .dispatch import attention_fp32


def scaled_dot_product_attention(queries, keys, values, cache=None, scale=None, mask=None, *,
                                 kv_start=None):
    """Attention over what ``cache.update_and_fetch`` returned.

    A cache marked ``_use_fused_sdpa`` returned quantized tuples: they go
    to ``cache_sdpa`` (fused HIP decode / prefill).  Any other cache, or
    none, returned plain [B, H_kv, N, D] tensors: plain attention.
    """
    if scale is None:
        scale = queries.shape[-1] ** -0.5
    if getattr(cache, "_use_fused_sdpa", False):
        return cache_sdpa(queries, keys, values, cache, scale=scale, mask=mask, kv_start=kv_start)
    if isinstance(keys, tuple):
        raise TypeError("quantized keys need a cache marked _use_fused_sdpa")
    return attention_fp32(queries, keys, values, scale, mask, kv_start)


class KVCache:
    """A plain (unquantized) growing cache: the non-fused side of the
    router.  update_and_fetch returns [B, H_kv, offset, D] views."""

    step = 256

    def __init__(self):
        self.keys = None
        self.values = None
        self.offset = 0

    def update_and_fetch(self, keys, values):
        S = keys.shape[2]
        if self.keys is None or self.offset + S > self.keys.shape[2]:
            n = ((self.offset + S + self.step - 1) // self.step) * self.step
            nk = keys.new_zeros((*keys.shape[:2], n, keys.shape[3]))
            nv = values.new_zeros((*values.shape[:2], n, values.shape[3]))
            if self.keys is not None:
                nk[:, :, :self.offset] = self.keys[:, :, :self.offset]
                nv[:, :, :self.offset] = self.values[:, :, :self.offset]
            self.keys, self.values = nk, nv
        self.keys[:, :, self.offset:self.offset + S] = keys
        self.values[:, :, self.offset:self.offset + S] = values
        self.offset += S
        return self.keys[:, :, :self.offset], self.values[:, :, :self.offset]

    def make_mask(self, N, return_array=False, window_size=None):
        return None if N == 1 else "causal"


def _rope(x, positions, theta):
    """Rotary embedding (half-split layout) at integer positions [B, L]."""
    D = x.shape[-1]
    inv = theta ** (-torch.arange(0, D, 2, device=x.device, dtype=torch.float32) / D)
    if x.device.type == "cuda":
        positions = kernels.to_device(positions, x.device)
    ang = positions.float()[:, None, :, None] * inv
    cos, sin = torch.cos(ang), torch.sin(ang)
    x1, x2 = x.float()[..., : D // 2], x.float()[..., D // 2:]
    return torch.cat([x1 * cos - x2 * sin, x2 * cos + x1 * sin], dim=-1).to(x.dtype)


class Attention(nn.Module):
    """Grouped-query attention with rotary positions, calling the router.

    forward(x [B, L, dim], mask=None, cache=None) -> [B, L, dim].  Without
    a mask the layer takes ``cache.make_mask(L)``; a one-token step on a
    batch cache with ``kv_start`` skips the left padding by index instead.
    """

    def __init__(self, dim, n_heads, n_kv_heads, head_dim=None, rope_theta=10000.0, bias=False,
                 dtype=torch.float16, device=None):
        super().__init__()
        if n_heads % n_kv_heads:
            raise ValueError("n_heads must be a multiple of n_kv_heads")
        self.n_heads, self.n_kv_heads = n_heads, n_kv_heads
        self.head_dim = head_dim or dim // n_heads
        self.scale = self.head_dim ** -0.5
        self.rope_theta = rope_theta
        kw = dict(bias=bias, dtype=dtype, device=device)
        self.q_proj = nn.Linear(dim, n_heads * self.head_dim, **kw)
        self.k_proj = nn.Linear(dim, n_kv_heads * self.head_dim, **kw)
        self.v_proj = nn.Linear(dim, n_kv_heads * self.head_dim, **kw)
        self.o_proj = nn.Linear(n_heads * self.head_dim, dim, **kw)

    def forward(self, x, mask=None, cache=None):
        B, L, _ = x.shape
        q = self.q_proj(x).reshape(B, L, self.n_heads, self.head_dim).transpose(1, 2)
        k = self.k_proj(x).reshape(B, L, self.n_kv_heads, self.head_dim).transpose(1, 2)
        v = self.v_proj(x).reshape(B, L, self.n_kv_heads, self.head_dim).transpose(1, 2)
        off = 0 if cache is None else cache.offset
        off = torch.as_tensor(off, dtype=torch.int64).reshape(-1, 1).expand(B, 1)
        pos = off + torch.arange(L)[None, :]
        q, k = _rope(q, pos, self.rope_theta), _rope(k, pos, self.rope_theta)
        kv_start = None
        if cache is not None and mask is None:
            if L == 1 and hasattr(cache, "kv_start"):
                kv_start = cache.kv_start(x.device)
            else:
                mask = cache.make_mask(L)
        elif cache is None and mask is None and L > 1:
            mask = "causal"
        if cache is not None:
            k, v = cache.update_and_fetch(k.contiguous(), v.contiguous())
        out = scaled_dot_product_attention(q.contiguous(), k, v, cache=cache, scale=self.scale, mask=mask,
                                           kv_start=kv_start)
        return self.o_proj(out.transpose(1, 2).reshape(B, L, -1))

    def reset_parameters(self, generator=None):
        """Random weights (std 1/sqrt(fan_in)) for synthetic runs."""
        with torch.no_grad():
            for lin in (self.q_proj, self.k_proj, self.v_proj, self.o_proj):
                w = torch.randn(lin.weight.shape, generator=generator) / math.sqrt(lin.weight.shape[1])
                lin.weight.copy_(w.to(lin.weight.dtype))
                if lin.bias is not None:
                    lin.bias.zero_()
