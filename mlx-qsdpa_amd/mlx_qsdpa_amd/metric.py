"""Algorithmic byte count of one decode (the metric's roofline numerator).

Same formula as mlx_qsdpa/bench_comparison.py:81-118: q + packed K/V +
scales + biases read, out written, 2-byte q/out.  ``valid_tokens`` lets a
left-padded batch count only the keys the kernel reads.
"""

from __future__ import annotations

HBM_PEAK_BYTES_PER_S = 8.0e12  # MI355X HBM3E


def kv_bytes_per_token(H_kv, D, bits, group_size, has_bias=True):
    """Bytes of K + V per token of one sequence (all KV heads)."""
    pack_bytes = D * bits // 8
    meta = (D // group_size) * 2 * (2 if has_bias else 1)
    return 2 * H_kv * (pack_bytes + meta)


def compute_bytes(B, H_q, H_kv, N, D, qL, path, bits=4, group_size=32):
    """(bytes_read, bytes_written) -- bench_comparison.py:81-108."""
    bytes_written = B * H_q * qL * D * 2
    q_bytes = B * H_q * qL * D * 2
    if path == "fp16":
        return q_bytes + B * H_kv * N * D * 2 * 2, bytes_written
    elems_per_int = 32 // bits
    pack_D = D // elems_per_int
    num_groups = D // group_size
    per_kv = B * H_kv * N * (pack_D * 4 + num_groups * 2 + num_groups * 2)
    return q_bytes + per_kv * 2, bytes_written


def compute_bandwidth_gbps(total_bytes, median_us):
    """bench_comparison.py:111-118."""
    return total_bytes / (median_us * 1e-6) / 1e9


def decode_bytes(B, H_q, H_kv, D, bits, group_size, valid_tokens):
    """Algorithmic bytes of one decode over `valid_tokens` keys in total
    (summed over the batch): q + out + K/V/scales/biases of those keys."""
    qo = 2 * B * H_q * D * 2
    return qo + valid_tokens * kv_bytes_per_token(H_kv, D, bits, group_size)
