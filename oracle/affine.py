"""MLX affine quantization format, restated in numpy -- TEST INFRASTRUCTURE.

Representation
--------------
A "T-valued" array is a float32 numpy array whose every element is exactly
representable in the storage dtype T ("f16" or "bf16").  ``to_T`` rounds
float32/float64 to such values with round-to-nearest-even.  Packed words are
numpy uint32.

Format (reference: mlx_qsdpa/kernels.py:101-105, 125-129)
------------------------------------------------------------
``packed[..., w]`` holds ``32 // bits`` consecutive elements; element ``j``
sits in bits ``[j*bits, (j+1)*bits)``.  The value of element ``d`` is
``scale[d // gs] * q[d] + bias[d // gs]``.

Quantizer contract (mx.quantize; called at mlx_qsdpa/cache.py:186-187,
314-315, 576-577, 610-611, 798-799, 830-831)
----------------------------------------------------------------------
MLX itself (``mlx>=0.21.0``, pyproject.toml:10, no lock file) is absent from
this container, so the per-group rule below is a restatement of the published
MLX ``affine_quantize`` (its ``mlx/ops.cpp`` formulation), all in float32:

    w_min, w_max = min, max of the group          (exact: T -> f32)
    scale = max((w_max - w_min) / (2^bits - 1), 1e-7)
    side  = |w_min| > |w_max|
    scale = side ? scale : -scale
    edge  = side ? w_min : w_max
    q0    = rint(edge / scale)
    scale = (q0 != 0) ? edge / q0 : scale          # zero is exactly on the grid
    bias  = (q0 != 0) ? edge : 0
    q     = clip(rint((w - bias) / scale), 0, 2^bits - 1)
    stored scale, bias = to_T(scale), to_T(bias)

``rint`` rounds half to even.  Recorded deviations from MLX's Metal kernel:
MLX's GPU kernel rounds half away from zero and starts its running max at 0;
both only matter for exact ties or for an all-negative group.

Dequantize contract (mx.dequantize; mlx_qsdpa/dispatch.py:69-78)
---------------------------------------------------------------
    value = to_T(fmaf(float(scale), float(q), float(bias)))
i.e. one float32 fused multiply-add then one rounding to T.

Pinning
-------
* ``pack``/``unpack``/element order: the reference kernel's shift rule
  (kernels.py:103-105) and known-answer words in tests/golden.
* ``quantize``: hand-derived known-answer groups (tests/golden/
  affine_known_answers.json) that separate every branch above, the rounding
  mode, and the scale sign; plus MLX's published error bound
  |w - dequant(quantize(w))| <= |scale|/2 (+ T rounding) on random data.
* ``dequantize``: exact-arithmetic identity on integer grids and the fma
  known answers in the same file.
"""

from __future__ import annotations

import numpy as np

DTYPES = ("f16", "bf16")


# ---------------------------------------------------------------------------
# T rounding
# ---------------------------------------------------------------------------
def f32_to_bf16_bits(x) -> np.ndarray:
    """Round float32 values to bfloat16 (nearest-even); returns uint16 bits.

    uint32 arithmetic: u + 0x7FFF + lsb stays below 2^32 for every non-NaN
    pattern (at most 0xFF800000 + 0x8000); NaN patterns, where it may wrap,
    are replaced by the quiet-NaN branch.
    """
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    is_nan = (u & np.uint32(0x7FFFFFFF)) > np.uint32(0x7F800000)
    lsb = (u >> np.uint32(16)) & np.uint32(1)
    with np.errstate(over="ignore"):
        r = ((u + np.uint32(0x7FFF) + lsb) >> np.uint32(16)).astype(np.uint16)
    return np.where(is_nan, ((u >> np.uint32(16)) | np.uint32(0x40)).astype(np.uint16), r).astype(np.uint16)


def bf16_bits_to_f32(b) -> np.ndarray:
    """bfloat16 bits (uint16) -> float32 values."""
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def to_T(x, dtype: str) -> np.ndarray:
    """Round to the nearest T value (ties to even); returns float32.

    float64 input is first rounded to float32 (a single rounding when the
    float64 value is exact, which holds for every use in this package).
    """
    x32 = np.asarray(x).astype(np.float32)
    if dtype == "f16":
        return x32.astype(np.float16).astype(np.float32)
    if dtype == "bf16":
        return bf16_bits_to_f32(f32_to_bf16_bits(x32))
    raise ValueError(f"unknown dtype {dtype!r}")


def T_bits(x, dtype: str) -> np.ndarray:
    """Bit pattern (uint16) of T-valued float32 data, for exact comparisons."""
    x32 = np.asarray(x, dtype=np.float32)
    if dtype == "f16":
        return x32.astype(np.float16).view(np.uint16)
    return f32_to_bf16_bits(x32)


# ---------------------------------------------------------------------------
# packing
# ---------------------------------------------------------------------------
def pack(q: np.ndarray, bits: int) -> np.ndarray:
    """Pack integer codes [..., D] into uint32 words [..., D*bits/32]."""
    per = 32 // bits
    q = np.asarray(q, dtype=np.uint64)
    D = q.shape[-1]
    if D % per:
        raise ValueError("D must be a multiple of 32/bits")
    qr = q.reshape(*q.shape[:-1], D // per, per)
    shifts = (np.arange(per, dtype=np.uint64) * bits)
    return (qr << shifts).sum(axis=-1).astype(np.uint32)


def unpack(packed: np.ndarray, bits: int) -> np.ndarray:
    """Unpack uint32 words [..., W] into codes [..., W*32/bits] (uint32)."""
    per = 32 // bits
    p = np.asarray(packed, dtype=np.uint32)[..., None]
    shifts = (np.arange(per, dtype=np.uint32) * bits)
    mask = np.uint32((1 << bits) - 1)
    q = (p >> shifts) & mask
    return q.reshape(*p.shape[:-2], p.shape[-2] * per)


# ---------------------------------------------------------------------------
# quantize / dequantize
# ---------------------------------------------------------------------------
def group_params(wg: np.ndarray, bits: int):
    """Per-group float32 (scale, bias) for groups along the last axis."""
    wg = np.asarray(wg, dtype=np.float32)
    n_bins = np.float32((1 << bits) - 1)
    eps = np.float32(1e-7)
    w_max = wg.max(axis=-1)
    w_min = wg.min(axis=-1)
    scale = np.maximum((w_max - w_min) / n_bins, eps).astype(np.float32)
    side = np.abs(w_min) > np.abs(w_max)
    scale = np.where(side, scale, -scale).astype(np.float32)
    edge = np.where(side, w_min, w_max).astype(np.float32)
    with np.errstate(divide="ignore", invalid="ignore"):
        q0 = np.rint(edge / scale).astype(np.float32)
        snapped = (edge / q0).astype(np.float32)
    nz = q0 != 0
    scale = np.where(nz, snapped, scale).astype(np.float32)
    bias = np.where(nz, edge, np.float32(0)).astype(np.float32)
    return scale, bias


def quantize(w: np.ndarray, group_size: int, bits: int, dtype: str):
    """mx.quantize restated: T-valued w [..., D] -> (packed, scales, biases).

    scales/biases are returned T-valued (float32 holding T values).
    """
    w = np.asarray(w, dtype=np.float32)
    D = w.shape[-1]
    if D % group_size:
        raise ValueError("D must be a multiple of group_size")
    wg = w.reshape(*w.shape[:-1], D // group_size, group_size)
    scale, bias = group_params(wg, bits)
    n_bins = np.float32((1 << bits) - 1)
    with np.errstate(divide="ignore", invalid="ignore"):
        qf = np.rint((wg - bias[..., None]) / scale[..., None]).astype(np.float32)
    q = np.clip(qf, np.float32(0), n_bins).astype(np.uint32)
    q = q.reshape(*w.shape[:-1], D)
    return pack(q, bits), to_T(scale, dtype), to_T(bias, dtype)


def dequantize(packed, scales, biases, group_size: int, bits: int, dtype: str):
    """mx.dequantize restated: value = to_T(fmaf(scale, q, bias)).

    ``biases`` may be None (symmetric format, zero biases).  The float64
    expression s*q + b is exact for every fp16 input (the operand span is at
    most 47 bits) and, for bf16, rounds to the float32 fma result whenever it
    is not exact, so one float64->float32 rounding reproduces fmaf.
    """
    q = unpack(packed, bits).astype(np.float64)
    D = q.shape[-1]
    s = np.asarray(scales, dtype=np.float64)
    b = np.zeros_like(s) if biases is None else np.asarray(biases, dtype=np.float64)
    s = np.repeat(s, group_size, axis=-1)[..., :D]
    b = np.repeat(b, group_size, axis=-1)[..., :D]
    return to_T(s * q + b, dtype)


def random_T(rng: np.random.Generator, shape, dtype: str, outlier_frac=0.0,
             outlier_gain=8.0) -> np.ndarray:
    """~N(0,1) T-valued data; a seeded `outlier_frac` of last-axis channels x gain."""
    x = rng.standard_normal(size=shape).astype(np.float32)
    if outlier_frac > 0:
        D = shape[-1]
        n_out = max(1, int(round(outlier_frac * D)))
        ch = rng.choice(D, size=n_out, replace=False)
        x[..., ch] *= np.float32(outlier_gain)
    return to_T(x, dtype)
