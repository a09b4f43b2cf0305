"""Scripted cache sequences run against both the product caches (torch) and
the oracle caches (numpy); the final buffers, counters and fetched views
must match bit-exactly.  Used by the CPU host-logic tests (with the kernel
wrappers patched to the oracle) and by the GPU tests (real HIP kernels).
"""

from __future__ import annotations

import numpy as np
import torch

from conftest import from_np, to_np, torch_dtype
from oracle import affine
from oracle import caches as oc

import mlx_qsdpa_amd.cache as pc

# (name, class kind, ctor kwargs, list of chunk lengths S per update)
SCENARIOS = [
    ("single_growth", "single", dict(bits=4, group_size=32, step=64), [60, 10, 1, 1, 70]),
    ("single_decode", "single", dict(bits=8, group_size=64, step=16), [1] * 20),
    ("batch_decode", "batch", dict(left_padding=[0, 3, 1], bits=4, group_size=64), [5, 1, 1, 300]),
    ("rot_fill_wrap", "rot", dict(max_size=8, bits=4, group_size=32), [1] * 21),
    ("rot_prefill_wrap", "rot", dict(max_size=8, bits=4, group_size=32), [6, 1, 1, 1, 1, 5, 1, 1, 12]),
    ("rot_keep_sinks", "rot", dict(max_size=8, keep=2, bits=8, group_size=32), [3, 1, 1, 1, 1, 1, 1, 1, 1, 4, 1, 1]),
    ("brot_decode_wrap", "brot", dict(left_padding=[0, 2], max_size=8, bits=4, group_size=32), [1] * 19),
    ("brot_prefill_after_wrap", "brot", dict(left_padding=[1, 0], max_size=16, bits=8, group_size=128), [5] + [1] * 20 + [7, 1, 1]),
    ("brot_keep_sinks", "brot", dict(left_padding=[0, 0], max_size=12, keep=4, bits=8, group_size=64), [6] + [1] * 15 + [5, 1]),
]

_DIMS = {"single": 256, "single_decode": 128, "batch": 128, "rot": 64, "brot": 128}


def _dims(name, kind):
    D = 128 if name in ("single_decode",) else _DIMS[kind]
    if name == "brot_prefill_after_wrap":
        D = 128
    return D


def _product(kind, kw):
    if kind == "single":
        return pc.QuantizedSDPACache(**kw)
    if kind == "batch":
        return pc.BatchQuantizedSDPACache(**kw)
    if kind == "rot":
        return pc.QuantizedRotatingSDPACache(**kw)
    return pc.BatchQuantizedRotatingSDPACache(**kw)


def _oracle(kind, kw, dtype):
    kw = dict(kw, dtype=dtype)
    if kind == "single":
        return oc.QuantizedSDPACache(**kw)
    if kind == "batch":
        return oc.BatchQuantizedSDPACache(**kw)
    if kind == "rot":
        return oc.QuantizedRotatingSDPACache(**kw)
    return oc.BatchQuantizedRotatingSDPACache(**kw)


def _batch(kind, kw):
    return len(kw["left_padding"]) if kind in ("batch", "brot") else 1


def run_scenario(name, kind, kw, chunks, dtype, device=None, seed=0):
    """Run both implementations step by step; compare after every update."""
    rng = np.random.default_rng(seed)
    B = _batch(kind, kw)
    H = 2
    D = _dims(name, kind)
    tdt = torch_dtype(dtype)
    prod = _product(kind, kw)
    orc = _oracle(kind, kw, dtype)
    for step, S in enumerate(chunks):
        k = affine.random_T(rng, (B, H, S, D), dtype, outlier_frac=0.02)
        v = affine.random_T(rng, (B, H, S, D), dtype)
        pk, pv = prod.update_and_fetch(from_np(k, tdt, device), from_np(v, tdt, device))
        ok, ov = orc.update_and_fetch(k, v)
        ctx = f"{name} step {step} (S={S})"
        for got, want in ((pk, ok), (pv, ov)):
            for i in range(3):
                g = to_np(got[i])
                assert g.shape == want[i].shape, f"{ctx}: shape {g.shape} vs {want[i].shape}"
                if i == 0:
                    assert np.array_equal(g, want[i]), f"{ctx}: packed words differ"
                else:
                    assert np.array_equal(affine.T_bits(g, dtype), affine.T_bits(want[i], dtype)), \
                        f"{ctx}: scales/biases differ"
        assert prod._idx == orc._idx if hasattr(orc, "_idx") else True, ctx
        if kind in ("batch", "brot"):
            assert np.array_equal(prod.offset.numpy(), orc.offset), ctx
        else:
            assert prod.offset == orc.offset, ctx
        assert prod.size() == orc.size(), ctx
    return prod, orc
