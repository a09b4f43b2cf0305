"""Byte and bandwidth formulas of mlx_qsdpa/bench_comparison.py:81-118.

TEST INFRASTRUCTURE: the checker for the library's own
``mlx_qsdpa_amd.metric`` module.  Pinned by the known answers of
tests/test_bench_comparison.py:113-160 (transcribed into
tests/golden/reference_fixtures.json).
"""


def compute_bytes(B, H_q, H_kv, N, D, qL, path, bits=4, group_size=32):
    """(bytes_read, bytes_written) of one attention call (fp16 q/out)."""
    bytes_written = B * H_q * qL * D * 2
    q_bytes = B * H_q * qL * D * 2
    if path == "fp16":
        return q_bytes + B * H_kv * N * D * 2 * 2, bytes_written
    pack_D = D // (32 // bits)
    num_groups = D // group_size
    per_kv = B * H_kv * N * (pack_D * 4 + num_groups * 2 + num_groups * 2)
    return q_bytes + per_kv * 2, bytes_written


def compute_bandwidth_gbps(total_bytes, median_us):
    return total_bytes / (median_us * 1e-6) / 1e9
