"""The oracle's dequantize + float64 SDPA, restated with torch on the GPU.

TEST INFRASTRUCTURE, for checks at BASELINE sizes (C2 at 128K keys, C3 at
1M, the C5 window every step) where the numpy oracle would take minutes.
It computes exactly what oracle/attention.py:quantized_sdpa_reference
computes -- value = T(float32(scale * code + bias)) with the product and sum
in float64 (oracle/affine.py:dequantize), then softmax attention in float64
with the MLX mask conventions (oracle/attention.py:sdpa) -- and
tests/test_gpu_parity_full.py pins it to the numpy oracle on small inputs
(dequantized values bit-exact, outputs equal to 1e-12).  No product code is
used.
"""

from __future__ import annotations

import torch


def dequantize(packed, scales, biases, group_size: int, bits: int, dtype: torch.dtype):
    """[..., N, W] uint32 codes + [..., N, D/gs] scales / biases -> [..., N, D] in `dtype`."""
    per = 32 // bits
    shifts = torch.arange(per, device=packed.device, dtype=torch.int64) * bits
    words = packed.view(torch.int32).to(torch.int64) & 0xFFFFFFFF
    codes = (words[..., None] >> shifts) & ((1 << bits) - 1)
    codes = codes.reshape(*packed.shape[:-1], -1).double()
    s = scales.double().repeat_interleave(group_size, dim=-1)
    b = torch.zeros_like(s) if biases is None else biases.double().repeat_interleave(group_size, dim=-1)
    return (s * codes + b).float().to(dtype)


def sdpa(q, k, v, scale: float, mask=None):
    """float64 attention.  q [B, Hq, L, D], k / v [B, Hkv, N, D] (head h uses
    kv head h // (Hq / Hkv)); mask None, "causal" (lower-right aligned), a
    bool keep-mask or an additive mask broadcastable to [B, Hq, L, N].
    Query rows with every key masked return zeros.  Returns float64."""
    B, Hq, L, D = q.shape
    Hkv, N = k.shape[1], k.shape[2]
    G = Hq // Hkv
    qd = q.double().reshape(B, Hkv, G * L, D)
    kt = k.double().transpose(-1, -2).contiguous()
    s = torch.matmul(qd, kt).reshape(B, Hq, L, N) * float(scale)
    if isinstance(mask, str):
        if mask != "causal":
            raise ValueError(mask)
        qi = torch.arange(L, device=q.device)[:, None] + (N - L)
        s = s.masked_fill(qi < torch.arange(N, device=q.device)[None, :], float("-inf"))
    elif mask is not None:
        m = mask.to(q.device)
        if m.dtype == torch.bool:
            s = s.masked_fill(~m, float("-inf"))
        else:
            s = s + m.double()
    mx = s.amax(dim=-1, keepdim=True)
    safe = torch.where(torch.isfinite(mx), mx, torch.zeros_like(mx))
    e = torch.exp(s - safe)
    den = e.sum(dim=-1, keepdim=True)
    p = torch.where(den > 0, e / torch.where(den > 0, den, torch.ones_like(den)), torch.zeros_like(e))
    o = torch.matmul(p.reshape(B, Hkv, G * L, N), v.double().contiguous())
    return o.reshape(B, Hq, L, D)


def quantized_sdpa(q, kq, vq, *, bits: int, group_size: int, scale=None, mask=None):
    """oracle.attention.quantized_sdpa_reference on torch tensors (kq / vq:
    (packed, scales, biases) with biases possibly None)."""
    D = q.shape[-1]
    if scale is None:
        scale = D ** -0.5
    k = dequantize(*kq, group_size, bits, q.dtype)
    v = dequantize(*vq, group_size, bits, q.dtype)
    return sdpa(q, k, v, scale, mask)
