"""CPU oracle for the quantized SDPA decode path -- TEST INFRASTRUCTURE ONLY.

This package restates, in numpy, the reference algorithms the MI355X library
must reproduce.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import it, and only as the checker.
The shipped library (``mlx-qsdpa_amd/``) never imports, links or calls it.

Modules
-------
affine     MLX affine quantize / dequantize / pack / unpack
           (the mx.quantize contract; see the module docstring).
attention  float64 scaled-dot-product attention over dequantized K/V (the
           reference's own fallback and parity oracle) and the causal-mask
           helper of mlx_qsdpa/cache.py:15-43.
caches     the four quantized cache state machines of mlx_qsdpa/cache.py.
metric     the byte / bandwidth formulas of mlx_qsdpa/bench_comparison.py.

Pinning status of every function is recorded in each module's docstring.
"""
