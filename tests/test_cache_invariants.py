"""Invariants of the rotating caches that the reference leaves undefined.

The reference asserts ``keep == 0`` (mlx_qsdpa/cache.py:512, 732) and its
mask width after the ring wraps disagrees with the keys it returns
(cache.py:636-644 vs 588-591).  Both caches here (the shipped torch caches
and the oracle's numpy caches) define those rules; these tests pin them
without reusing either implementation's index arithmetic:

* every update is replayed on ``window_model.WindowModel``, which keeps the
  window's tokens in temporal order and knows nothing about ring pointers;
  after every update the cache's ``state`` (temporal order) must equal the
  model row for row, and the keys it returns (ring order) must hold the
  sinks in slots [0, keep) and the model's other rows in some order;
* as long as only single tokens were appended, the sink rows are
  bit-exactly quantize(first keep tokens);
* with keep = 0 the same model is the reference's rotating window, and the
  reference's own index sequences are pinned by the fixtures in
  tests/golden/reference_fixtures.json (tests/test_host_logic.py);
* a mask made before an update (as a model's forward pass makes it) is
  lower-right causal over exactly the keys that update returns.

The shipped caches run here on CPU with the two kernel wrappers replaced by
the oracle quantizer (conftest.cpu_kernels); tests/test_gpu_cache.py runs
the same sequences on the GPU kernels.
"""

import numpy as np
import pytest
import torch

from conftest import from_np, to_np, torch_dtype
from oracle import affine
from oracle import caches as oc
from window_model import WindowModel, assert_same_multiset, assert_same_rows, random_chunks

import mlx_qsdpa_amd.cache as pc

B, H, D = 2, 2, 64


def _np3(t):
    return tuple(to_np(x) if isinstance(x, torch.Tensor) else np.asarray(x) for x in t)


def _sl(t, a, b):
    return tuple(x[:, :, a:b] for x in t)


def _make(kind, impl, max_size, keep, bits, gs, dtype):
    if impl == "product":
        if kind == "single":
            return pc.QuantizedRotatingSDPACache(max_size, keep=keep, bits=bits, group_size=gs)
        return pc.BatchQuantizedRotatingSDPACache([0] * B, max_size, keep=keep, bits=bits, group_size=gs)
    if kind == "single":
        return oc.QuantizedRotatingSDPACache(max_size, keep=keep, bits=bits, group_size=gs, dtype=dtype)
    return oc.BatchQuantizedRotatingSDPACache([0] * B, max_size, keep=keep, bits=bits, group_size=gs,
                                              dtype=dtype)


def _temporal_state(cache, kind):
    """The cache's tokens in temporal order: `state` of a single cache, the
    per-sequence `extract` of a batch cache (stacked over the batch)."""
    if kind == "single":
        return _np3(cache.state[0]), _np3(cache.state[1])
    parts_k, parts_v = [], []
    for i in range(B):
        single = cache.extract(i)
        k, v = single.state
        parts_k.append(_np3(k))
        parts_v.append(_np3(v))
    cat = lambda ps: tuple(np.concatenate([p[j] for p in ps], axis=0) for j in range(3))  # noqa: E731
    return cat(parts_k), cat(parts_v)


def run_window_invariants(kind, impl, max_size, keep, bits, gs, dtype, seed, device=None, chunks=None):
    """Replay a random decode / prefill sequence on a cache and on the window
    model; check the invariants after every update.  Returns the cache."""
    rng = np.random.default_rng(seed)
    tdt = torch_dtype(dtype)
    cache = _make(kind, impl, max_size, keep, bits, gs, dtype)
    model = WindowModel(max_size, keep, bits, gs, dtype)
    if chunks is None:
        chunks = random_chunks(rng, max_size, 4 * max_size)
    decode_only = True
    for step, S in enumerate(chunks):
        k = affine.random_T(rng, (B, H, S, D), dtype, outlier_frac=0.02)
        v = affine.random_T(rng, (B, H, S, D), dtype)
        if impl == "product":
            kq, vq = cache.update_and_fetch(from_np(k, tdt, device), from_np(v, tdt, device))
        else:
            kq, vq = cache.update_and_fetch(k, v)
        model.update(k, v)
        decode_only = decode_only and S == 1
        ctx = f"{kind}/{impl} keep={keep} step {step} (S={S}, {len(model)} in window)"
        kq, vq = _np3(kq), _np3(vq)
        n = len(model)
        assert kq[0].shape[2] == n, f"{ctx}: {kq[0].shape[2]} keys returned"
        sinks = min(keep, n)
        for got, want in ((kq, model.k), (vq, model.v)):
            assert_same_rows(_sl(got, 0, sinks), _sl(want, 0, sinks), dtype, ctx + " sinks")
            assert_same_multiset(got, want, dtype, ctx + " window")
        if decode_only and sinks:
            first = affine.quantize(model.raw_first[:, :, :sinks], gs, bits, dtype)
            assert_same_rows(_sl(kq, 0, sinks), first, dtype, ctx + " sinks = quantize(first tokens)")
        sk, sv = _temporal_state(cache, kind)
        assert_same_rows(sk, model.k, dtype, ctx + " state (temporal order)")
        assert_same_rows(sv, model.v, dtype, ctx + " state (temporal order)")
    return cache


CASES = [  # (max_size, keep, bits, gs, dtype, seed)
    (8, 0, 4, 32, "f16", 1),
    (8, 1, 4, 32, "f16", 2),
    (8, 4, 8, 64, "bf16", 3),
    (12, 4, 4, 64, "f16", 4),
    (12, 11, 8, 32, "bf16", 5),  # one ring slot after the sinks
    (16, 3, 4, 32, "bf16", 6),
]


@pytest.mark.parametrize("impl", ["product", "oracle"])
@pytest.mark.parametrize("kind", ["single", "batch"])
@pytest.mark.parametrize("case", CASES, ids=lambda c: "W{}_keep{}_b{}_g{}_{}".format(*c[:5]))
def test_rotating_window_matches_model(cpu_kernels, kind, impl, case):
    max_size, keep, bits, gs, dtype, seed = case
    run_window_invariants(kind, impl, max_size, keep, bits, gs, dtype, seed)


@pytest.mark.parametrize("impl", ["product", "oracle"])
def test_first_wrap_onto_the_sinks(cpu_kernels, impl):
    """Decodes only, across the first wrap and two more: the slot after the
    last is the first slot after the sinks, never a sink."""
    run_window_invariants("single", impl, 8, 3, 4, 32, "f16", 11, chunks=[1] * 30)
    run_window_invariants("batch", impl, 8, 3, 4, 32, "f16", 12, chunks=[1] * 30)


@pytest.mark.parametrize("impl", ["product", "oracle"])
def test_prefill_longer_than_the_window(cpu_kernels, impl):
    """A first chunk longer than the window keeps its first `keep` and last
    max_size - keep tokens; later chunks requantize the dequantized window."""
    run_window_invariants("single", impl, 8, 2, 8, 32, "bf16", 13, chunks=[20, 1, 1, 9, 1, 3])
    run_window_invariants("batch", impl, 8, 2, 8, 32, "bf16", 14, chunks=[20, 1, 1, 9, 1, 3])


def _lower_right(N, n):
    return np.arange(n)[None, :] <= (n - N) + np.arange(N)[:, None]


@pytest.mark.parametrize("impl", ["product", "oracle"])
@pytest.mark.parametrize("keep", [0, 2])
def test_mask_is_causal_over_returned_keys(cpu_kernels, impl, keep):
    """make_mask(N) taken before an update (as a forward pass takes it) is
    the lower-right causal mask over exactly the keys the update returns,
    before and after the window wraps.  Chunks stay within the window's
    non-sink part, so every query's own key is among the returned keys."""
    max_size, bits, gs, dtype = 16, 4, 32, "f16"
    rng = np.random.default_rng(21 + keep)
    tdt = torch_dtype(dtype)
    for kind in ("single", "batch"):
        cache = _make(kind, impl, max_size, keep, bits, gs, dtype)
        for step, S in enumerate([3, 1, 5, 1, 1, 7, 2, 1, 9, 4, 1, 1, 6, 3, 8]):
            mask = cache.make_mask(S, return_array=True) if S > 1 else None
            k = affine.random_T(rng, (B, H, S, D), dtype)
            v = affine.random_T(rng, (B, H, S, D), dtype)
            if impl == "product":
                kq, _ = cache.update_and_fetch(from_np(k, tdt), from_np(v, tdt))
            else:
                kq, _ = cache.update_and_fetch(k, v)
            if mask is None:
                continue
            n = kq[0].shape[2]
            m = to_np(mask) if isinstance(mask, torch.Tensor) else np.asarray(mask)
            want = _lower_right(S, n)
            ctx = f"{kind}/{impl} keep={keep} step {step}: S={S}, {n} keys"
            if kind == "single":
                assert m.shape == (S, n), f"{ctx}: mask shape {m.shape}"
                assert np.array_equal(m.astype(bool), want), ctx
            else:
                assert m.shape == (B, 1, S, n), f"{ctx}: mask shape {m.shape}"
                for bi in range(B):
                    assert np.array_equal(m[bi, 0].astype(bool), want), f"{ctx} (b={bi})"
