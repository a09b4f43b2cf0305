"""quantized_sdpa: validation and routing onto the HIP decode kernels.

Mirrors mlx_qsdpa/dispatch.py:8-111 (same signature, same ValueError set,
same defaults for ``scale`` and for missing biases), with four MI355X
choices:

* Masked decode runs in-kernel (bool keep-mask or additive mask), where the
  reference falls back to dequantize + SDPA (dispatch.py:68-83).
* ``threshold`` keeps its meaning when given (N <= threshold: single pass,
  else split-K); the default ``None`` lets the library pick the split count
  for 256 CUs.
* ``kv_start`` (extension) skips keys before a per-sequence start index, the
  left padding of a batched cache, without reading them.

* Several query positions (qL > 1: speculative or chunked decoding,
  prefill) run on the fused matrix-core kernel, including mask="causal"
  (aligned to the last key), where the reference dequantizes and runs SDPA.
  Shapes that kernel does not take (D = 64, unaligned views) keep the
  reference's path: HIP dequantize, then float32 attention with torch on
  the GPU (dispatch.py:68-83).

Head dims the library does not compile (any other multiple of 32, e.g. 32
or 512, which the reference's validation accepts: dispatch.py:48-49) take
that same dequantize + attention path at every qL.
"""

from __future__ import annotations

import torch

from . import _lib, kernels


def _validate(q, packed_k, packed_v, bits, group_size):
    """dispatch.py:42-65."""
    if q.dim() != 4:
        raise ValueError(f"q must be 4D (B, H_q, qL, D), got ndim={q.dim()}")
    B, H_q, qL, D = q.shape
    if bits not in (4, 8):
        raise ValueError(f"bits must be 4 or 8, got {bits}")
    if D % 32 != 0:
        raise ValueError(f"D must be multiple of 32, got {D}")
    elems_per_int = 32 // bits
    pack_D = D // elems_per_int
    if packed_k.dim() != 4 or packed_v.dim() != 4:
        raise ValueError("packed_k and packed_v must be 4D (B, H_kv, N, pack_D)")
    _, H_kv, N, actual_pack_D = packed_k.shape
    if actual_pack_D != pack_D:
        raise ValueError(
            f"packed_k last dim {actual_pack_D} != expected pack_D={pack_D} "
            f"for bits={bits}, D={D}")
    if H_q % H_kv != 0:
        raise ValueError(f"H_q ({H_q}) must be divisible by H_kv ({H_kv})")
    return B, H_q, qL, D, H_kv, N


def attention_fp32(q, k, v, scale, mask=None, kv_start=None):
    """float32 SDPA on the GPU with MLX mask conventions.

    q [B,Hq,L,D], k/v [B,Hkv,N,D] (dequantized T), grouped-query heads.
    Bool masks keep True, float masks are added, "causal" is lower-right
    aligned; keys before kv_start[b] are skipped; rows with every key masked
    return 0.  Output has q's dtype.
    """
    B, Hq, L, D = q.shape
    Hkv, N = k.shape[1], k.shape[2]
    G = Hq // Hkv
    qf = q.float().reshape(B, Hkv, G * L, D)
    kt = k.float().transpose(-1, -2).contiguous()
    s = torch.matmul(qf, kt).reshape(B, Hq, L, N) * float(scale)
    cols = torch.arange(N, device=q.device)
    if isinstance(mask, str):
        if mask != "causal":
            raise ValueError(f"unknown mask {mask!r}")
        rows = torch.arange(L, device=q.device)[:, None] + (N - L)
        s = s.masked_fill(cols[None, :] > rows, float("-inf"))
    elif mask is not None:
        m = mask.to(q.device)
        s = s.masked_fill(~m, float("-inf")) if m.dtype == torch.bool else s + m.float()
    if kv_start is not None:
        ks = kv_start.to(q.device, torch.int64)
        s = s.masked_fill(cols[None, None, None, :] < ks[:, None, None, None], float("-inf"))
    p = torch.nan_to_num(torch.softmax(s, dim=-1), nan=0.0)
    o = torch.matmul(p.reshape(B, Hkv, G * L, N), v.float().contiguous())
    return o.reshape(B, Hq, L, D).to(q.dtype)


def dequantize_attention(q, k_quant, v_quant, *, bits, group_size, scale, mask, kv_start=None):
    """The reference's dequantize + SDPA path (dispatch.py:68-83)."""
    k = kernels.dequantize(*k_quant, group_size=group_size, bits=bits)
    v = kernels.dequantize(*v_quant, group_size=group_size, bits=bits)
    return attention_fp32(q, k, v, scale, mask, kv_start)


def fallback_sdpa(q, k_quant, v_quant, *, bits, group_size, scale, mask=None, kv_start=None):
    """Dequantize (HIP) + float32 attention: the path of dispatch.py:68-83.

    Missing biases are zeros (dispatch.py:71, 76); keys before kv_start[b]
    are masked.
    """
    kb = k_quant[2] if k_quant[2] is not None else torch.zeros_like(k_quant[1])
    vb = v_quant[2] if v_quant[2] is not None else torch.zeros_like(v_quant[1])
    return dequantize_attention(q, (k_quant[0], k_quant[1], kb), (v_quant[0], v_quant[1], vb),
                                bits=bits, group_size=group_size, scale=scale, mask=mask,
                                kv_start=kv_start)


def quantized_sdpa(
    q,
    packed_k,
    packed_v,
    k_scales,
    v_scales,
    k_biases=None,
    v_biases=None,
    scale=None,
    mask=None,
    bits=4,
    group_size=32,
    threshold=None,
    *,
    kv_start=None,
    num_splits=None,
):
    """Quantized scaled dot-product attention for decode (qL = 1).

    Args (as mlx_qsdpa.quantized_sdpa, dispatch.py:22-40):
        q:          (B, H_q, qL, D) float16/bfloat16
        packed_k/v: (B, H_kv, N, D*bits/32) uint32
        k/v_scales: (B, H_kv, N, D/group_size) q.dtype
        k/v_biases: same shape, or None for the symmetric format
        scale:      softmax scale (default D**-0.5)
        mask:       None, bool keep-mask or additive mask broadcastable to
                    (B, H_q, 1, N); "causal" (no-op for qL = 1)
        bits:       4 or 8;  group_size: 32, 64 or 128
        threshold:  N <= threshold -> single pass, else split-K;
                    None -> choose for the GPU
        kv_start:   optional (B,) int tensor: keys before it are ignored
        num_splits: optional explicit split count (overrides threshold)
    Returns (B, H_q, qL, D) in q's dtype.
    """
    # A decode step that repeats an earlier call's geometry relaunches that
    # call's argument block (the checks below held for it; its shapes and
    # strides are the block's key).
    if mask is None and kv_start is None and threshold is None and num_splits is None and q.dim() == 4 \
            and q.shape[2] == 1 and q.shape[3] in kernels.HEAD_DIMS and bits in (4, 8):
        both = k_biases is not None and v_biases is not None
        out = kernels.decode_repeat(q, packed_k, packed_v, k_scales, v_scales, k_biases if both else None,
                                    v_biases if both else None,
                                    scale=q.shape[3] ** -0.5 if scale is None else scale, bits=bits,
                                    group_size=group_size)
        if out is not None:
            return out
    B, H_q, qL, D, H_kv, N = _validate(q, packed_k, packed_v, bits, group_size)
    if scale is None:
        scale = D ** -0.5                                          # dispatch.py:86-87
    # The kernels read packed rows in 16-byte pieces; a view whose rows are
    # not 16-byte aligned is copied first, as the reference's kernel builder
    # copies every input (ensure_row_contiguous, kernels.py:190).
    packed_k, packed_v = _row_aligned(packed_k), _row_aligned(packed_v)
    # A mask made on the host (as a cache's make_mask may make it) goes to
    # the device in stream order, without waiting.
    if isinstance(mask, torch.Tensor) and q.device.type == "cuda":
        mask = kernels.to_device(mask, q.device)
    if isinstance(kv_start, torch.Tensor) and q.device.type == "cuda":
        kv_start = kernels.to_device(kv_start, q.device)

    if D not in kernels.HEAD_DIMS or (qL > 1 and not _fused_takes(
            q, packed_k, packed_v, k_scales, v_scales, k_biases, v_biases, scale, bits, group_size)):
        return fallback_sdpa(q, (packed_k, k_scales, k_biases),    # dispatch.py:68-83
                             (packed_v, v_scales, v_biases), bits=bits, group_size=group_size,
                             scale=scale, mask=mask, kv_start=kv_start)

    has_biases = k_biases is not None and v_biases is not None     # dispatch.py:89-94
    if not has_biases:
        k_biases = v_biases = None
    causal = False
    if isinstance(mask, str):
        if mask != "causal":
            raise ValueError(f"unknown mask {mask!r}")
        causal = qL > 1                                            # qL == 1: sees every key
        mask = None

    if num_splits is None:
        if threshold is None:
            num_splits = 0
        elif N <= threshold:                                       # dispatch.py:98
            num_splits = 1
        else:
            auto, _ = kernels.decode_plan(q, packed_k, packed_v, k_scales, v_scales, k_biases,
                                          v_biases, scale=scale, bits=bits,
                                          group_size=group_size)
            num_splits = max(2, auto)
    return kernels.decode(q, packed_k, packed_v, k_scales, v_scales, k_biases, v_biases,
                          scale=scale, bits=bits, group_size=group_size, mask=mask,
                          kv_start=kv_start, num_splits=num_splits, causal=causal)


def _row_aligned(t):
    """`t` itself if its rows start on 16-byte boundaries, else a contiguous copy."""
    if t.data_ptr() % 16 == 0 and all(st % 4 == 0 for st in t.stride()[:3]) and t.stride(-1) == 1:
        return t
    return t.contiguous()


def _fused_takes(q, packed_k, packed_v, k_scales, v_scales, k_biases, v_biases, scale, bits,
                 group_size):
    """Whether the fused kernel takes several query positions for these
    inputs (the matrix-core path: D 128 or 256, aligned views).  Extension:
    the reference sends every qL > 1 call to dequantize + attention."""
    if k_biases is None or v_biases is None:
        k_biases = v_biases = None
    try:
        kernels.decode_plan(q, packed_k, packed_v, k_scales, v_scales, k_biases, v_biases,
                            scale=scale, bits=bits, group_size=group_size)
    except _lib.QsdpaError as e:
        if e.code == _lib.QSDPA_ERR_UNSUPPORTED:
            return False
        raise
    return True
