"""Reference attention over dequantized K/V -- TEST INFRASTRUCTURE.

The reference's own parity oracle is its fallback path: dequantize K/V to T,
then ``mx.fast.scaled_dot_product_attention`` (mlx_qsdpa/dispatch.py:68-83,
mlx_qsdpa/__init__.py:49-60, tests/conftest.py:79-83).  Here the dequantize
is ``affine.dequantize`` (T-rounded) and the attention is computed in
float64, so the only rounding left to compare against is the kernel's own.

Mask conventions (MLX SDPA): a bool mask keeps keys where True; a float mask
is added to the scaled scores; the string "causal" is the lower-right aligned
causal mask (query i sees key j iff j <= i + kL - qL).  A query row whose keys
are all masked produces zeros; this is the ``global_sum == 0`` guard of the
reference's fused kernels (mlx_qsdpa/kernels.py:152, 408).

Pinning: closed forms in tests (N = 1 returns the value row, identical keys
return mean(V), a constant added to every V bias shifts the output by that
constant, permutation invariance over keys), plus brute-force loops on tiny
inputs in tests/test_oracle_attention.py.
"""

from __future__ import annotations

import numpy as np

from . import affine


def create_causal_mask(N, offset, window_size=None, left_padding=None):
    """numpy restatement of mlx_qsdpa/cache.py:15-43 (_create_causal_mask).

    ``offset`` is an int or an int array [B]; the batched form returns a
    bool array [B, 1, N, max(offset) + N].
    """
    if isinstance(offset, np.ndarray) and offset.ndim > 0:
        max_off = int(offset.max())                                # cache.py:26
        total = max_off + N
        q_pos = np.arange(N)[None, :] + offset[:, None]            # (B, N)
        k_pos = np.arange(total)[None, :]                          # (1, total)
        mask = q_pos[:, :, None] >= k_pos[:, None, :]              # cache.py:30
        if left_padding is not None:
            mask = mask & (k_pos[:, None, :] >= np.asarray(left_padding)[:, None, None])
        if window_size is not None:
            mask = mask & (q_pos[:, :, None] - k_pos[:, None, :] < window_size)
        return mask[:, None, :, :]
    q_idx = np.arange(offset, offset + N)                          # cache.py:37
    k_idx = np.arange(offset + N)
    mask = q_idx[:, None] >= k_idx[None]
    if window_size is not None:
        mask = mask & (q_idx[:, None] - k_idx[None] < window_size)
    return mask


def sdpa(q, k, v, scale, mask=None):
    """float64 SDPA.  q [B,Hq,L,D], k/v [B,Hkv,N,D] (GQA: head h uses h//G).

    Returns float64 [B, Hq, L, D].
    """
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    B, Hq, L, D = q.shape
    Hkv, N = k.shape[1], k.shape[2]
    G = Hq // Hkv
    qg = q.reshape(B, Hkv, G, L, D)
    s = np.einsum("bkgld,bknd->bkgln", qg, k) * float(scale)       # [B,Hkv,G,L,N]
    s = s.reshape(B, Hq, L, N)
    if isinstance(mask, str):
        if mask != "causal":
            raise ValueError(f"unknown mask string {mask!r}")
        qi = np.arange(L)[:, None] + (N - L)
        kj = np.arange(N)[None, :]
        s = np.where(qi >= kj, s, -np.inf)
    elif mask is not None:
        m = np.asarray(mask)
        if m.dtype == np.bool_:
            s = np.where(np.broadcast_to(m, s.shape), s, -np.inf)
        else:
            s = s + m.astype(np.float64)
    mx_ = s.max(axis=-1, keepdims=True)
    safe = np.where(np.isfinite(mx_), mx_, 0.0)
    e = np.exp(s - safe)
    den = e.sum(axis=-1, keepdims=True)
    p = np.where(den > 0, e / np.where(den > 0, den, 1.0), 0.0)
    pg = p.reshape(B, Hkv, G, L, N)
    o = np.einsum("bkgln,bknd->bkgld", pg, v)
    return o.reshape(B, Hq, L, D)


def quantized_sdpa_reference(q, k_packed, v_packed, k_scales, v_scales,
                             k_biases, v_biases, *, bits, group_size, dtype,
                             scale=None, mask=None):
    """The reference's fallback path (dispatch.py:68-83) in float64.

    All tensor arguments are numpy (T-valued float32 for q / scales / biases,
    uint32 for packed).  ``k_biases``/``v_biases`` None = zero biases
    (dispatch.py:71, 76).  Returns float64 [B, Hq, L, D].
    """
    D = q.shape[-1]
    if scale is None:
        scale = D ** -0.5                                           # dispatch.py:79-80
    k = affine.dequantize(k_packed, k_scales, k_biases, group_size, bits, dtype)
    v = affine.dequantize(v_packed, v_scales, v_biases, group_size, bits, dtype)
    return sdpa(q, k, v, scale, mask)


def decode_fp32(q, k_packed, v_packed, k_scales, v_scales, k_biases, v_biases,
                *, bits, group_size, scale=None):
    """float32 dequantize + SDPA decode (qL = 1) without T rounding.

    The CPU baseline of bench.py: the reference's CPU-capable path
    (dispatch.py:68-83) as a straightforward numpy float32 program.
    """
    B, Hq, L, D = q.shape
    Hkv = k_packed.shape[1]
    G = Hq // Hkv
    if scale is None:
        scale = D ** -0.5
    per = 32 // bits

    def deq(p, s, b):
        codes = affine.unpack(p, bits).astype(np.float32)
        s32 = np.repeat(np.asarray(s, np.float32), group_size, axis=-1)
        out = codes * s32
        if b is not None:
            out += np.repeat(np.asarray(b, np.float32), group_size, axis=-1)
        return out

    del per
    k = deq(k_packed, k_scales, k_biases)
    v = deq(v_packed, v_scales, v_biases)
    qg = np.asarray(q, np.float32).reshape(B, Hkv, G, D) * np.float32(scale)
    s = np.matmul(qg, np.swapaxes(k, -1, -2))                      # [B,Hkv,G,N]
    s -= s.max(axis=-1, keepdims=True)
    np.exp(s, out=s)
    s /= s.sum(axis=-1, keepdims=True)
    o = np.matmul(s, v)                                             # [B,Hkv,G,D]
    return o.reshape(B, Hq, 1, D)


def decode_fp32_threads(q, k_packed, v_packed, k_scales, v_scales, k_biases, v_biases,
                        *, bits, group_size, threads, scale=None):
    """decode_fp32 on `threads` host threads: the keys are cut into `threads`
    contiguous ranges, each thread dequantizes its range and computes its
    partial softmax (row max m, sum l, unnormalised output a), and the
    partials are merged as  o = sum_i exp(m_i - M) a_i / sum_i exp(m_i - M) l_i
    (M = max_i m_i).  numpy releases the GIL inside its array operations,
    so the ranges run in parallel; each thread's BLAS calls are limited to
    one thread.  The CPU baseline of bench.py on all host cores; pinned to
    decode_fp32 by tests/test_oracle_attention.py."""
    from concurrent.futures import ThreadPoolExecutor

    from threadpoolctl import threadpool_limits

    B, Hq, L, D = q.shape
    Hkv, N = k_packed.shape[1], k_packed.shape[2]
    G = Hq // Hkv
    if scale is None:
        scale = D ** -0.5
    threads = max(1, min(int(threads), N))
    cuts = np.linspace(0, N, threads + 1).astype(int)
    qg = np.asarray(q, np.float32).reshape(B, Hkv, G, D) * np.float32(scale)

    def deq(p, s, b, lo, hi):
        codes = affine.unpack(p[:, :, lo:hi], bits).astype(np.float32)
        out = codes * np.repeat(np.asarray(s[:, :, lo:hi], np.float32), group_size, axis=-1)
        if b is not None:
            out += np.repeat(np.asarray(b[:, :, lo:hi], np.float32), group_size, axis=-1)
        return out

    def part(i):
        lo, hi = cuts[i], cuts[i + 1]
        k = deq(k_packed, k_scales, k_biases, lo, hi)
        v = deq(v_packed, v_scales, v_biases, lo, hi)
        s = np.matmul(qg, np.swapaxes(k, -1, -2))                  # [B,Hkv,G,n]
        m = s.max(axis=-1, keepdims=True)
        np.exp(s - m, out=s)
        return m, s.sum(axis=-1, keepdims=True), np.matmul(s, v)

    with threadpool_limits(limits=1), ThreadPoolExecutor(max_workers=threads) as ex:
        parts = list(ex.map(part, range(threads)))
    M = np.max(np.stack([p[0] for p in parts]), axis=0)
    num = sum(np.exp(p[0] - M) * p[2] for p in parts)
    den = sum(np.exp(p[0] - M) * p[1] for p in parts)
    return (num / den).reshape(B, Hq, 1, D)
