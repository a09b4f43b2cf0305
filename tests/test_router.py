"""The model side on CPU: the router's dispatch on ``_use_fused_sdpa``, its
plain branch against the oracle's float64 attention, the Attention layer's
rotary offsets, and save / load of all four caches (kernel wrappers
replaced by conftest.cpu_kernels; tests/test_gpu_router.py runs the fused
branch and a save / load in the middle of a decode on the GPU)."""

import numpy as np
import pytest
import torch

from conftest import from_np, to_np, torch_dtype
from oracle import affine
from oracle import attention as oa
from window_model import assert_same_rows

import mlx_qsdpa_amd as mq
import mlx_qsdpa_amd.attention as att
import mlx_qsdpa_amd.cache as pc


def _np3(t):
    return tuple(to_np(x) for x in t)


@pytest.mark.parametrize("mask", [None, "causal", "bool", "additive", "kv_start"])
def test_plain_branch_matches_oracle(mask):
    rng = np.random.default_rng(1)
    B, Hq, Hkv, L, N, D = 2, 8, 2, 3, 40, 64
    q = rng.standard_normal((B, Hq, L, D)).astype(np.float32)
    k = rng.standard_normal((B, Hkv, N, D)).astype(np.float32)
    v = rng.standard_normal((B, Hkv, N, D)).astype(np.float32)
    kw, m_np = {}, None
    if mask == "causal":
        m_np = m_t = "causal"
    elif mask == "bool":
        m_np = rng.random((B, 1, L, N)) < 0.7
        m_t = torch.from_numpy(m_np)
    elif mask == "additive":
        m_np = (rng.standard_normal((1, Hq, L, N)) * 2).astype(np.float32)
        m_t = torch.from_numpy(m_np)
    elif mask == "kv_start":
        ks = np.array([5, 31])
        kw["kv_start"] = torch.from_numpy(ks)
        m_np = np.arange(N)[None, None, None, :] >= ks[:, None, None, None]
        m_t = None
    else:
        m_t = None
    cache = mq.KVCache()
    kf, vf = cache.update_and_fetch(torch.from_numpy(k), torch.from_numpy(v))
    got = mq.scaled_dot_product_attention(torch.from_numpy(q), kf, vf, cache=cache, scale=0.11, mask=m_t, **kw)
    # oracle.attention.sdpa expects repeated kv heads
    want = oa.sdpa(q, np.repeat(k, Hq // Hkv, axis=1), np.repeat(v, Hq // Hkv, axis=1), 0.11, m_np)
    np.testing.assert_allclose(got.numpy(), want, rtol=1e-5, atol=1e-5)


def test_router_dispatches_on_the_marker(monkeypatch):
    calls = []
    monkeypatch.setattr(att, "cache_sdpa", lambda *a, **k: calls.append(type(a[3]).__name__) or "fused")
    q = torch.zeros(1, 2, 1, 64)
    for c in (pc.QuantizedSDPACache(), pc.BatchQuantizedSDPACache([0]), pc.QuantizedRotatingSDPACache(8),
              pc.BatchQuantizedRotatingSDPACache([0], 8)):
        assert mq.scaled_dot_product_attention(q, ("k",), ("v",), cache=c) == "fused"
    assert calls == ["QuantizedSDPACache", "BatchQuantizedSDPACache", "QuantizedRotatingSDPACache",
                     "BatchQuantizedRotatingSDPACache"]

    class Marked:
        _use_fused_sdpa = False

    with pytest.raises(TypeError):  # quantized tuples with a cache that does not take them
        mq.scaled_dot_product_attention(q, (torch.zeros(1),), (torch.zeros(1),), cache=Marked())
    out = mq.scaled_dot_product_attention(q, torch.ones(1, 2, 4, 64), torch.ones(1, 2, 4, 64), cache=Marked())
    assert torch.allclose(out, torch.ones_like(out))
    assert calls == ["QuantizedSDPACache", "BatchQuantizedSDPACache", "QuantizedRotatingSDPACache",
                     "BatchQuantizedRotatingSDPACache"]


def test_attention_layer_incremental_equals_full():
    """Rotary positions at the cache offset: a prefill + one-token steps
    through a KVCache give the full causal pass's outputs."""
    torch.manual_seed(0)
    layer = mq.Attention(256, 8, 2, head_dim=32, dtype=torch.float32)
    layer.reset_parameters(torch.Generator().manual_seed(1))
    x = torch.randn(2, 11, 256)
    with torch.no_grad():
        full = layer(x)
        cache = mq.KVCache()
        parts = [layer(x[:, :6], cache=cache)] + [layer(x[:, t:t + 1], cache=cache) for t in range(6, 11)]
    torch.testing.assert_close(torch.cat(parts, dim=1), full, rtol=1e-4, atol=1e-4)


def _fill(cache, rng, steps, B, dtype="f16"):
    tdt = torch_dtype(dtype)
    for S in steps:
        k = affine.random_T(rng, (B, 2, S, 64), dtype)
        v = affine.random_T(rng, (B, 2, S, 64), dtype)
        cache.update_and_fetch(from_np(k, tdt), from_np(v, tdt))


def _caches(rng):
    a = pc.QuantizedSDPACache(bits=4, group_size=32)
    _fill(a, rng, [30, 1, 1], 1)
    singles = []
    for n in (5, 9):
        s = pc.QuantizedSDPACache(bits=4, group_size=32)
        _fill(s, rng, [n], 1)
        singles.append(s)
    b = pc.BatchQuantizedSDPACache.merge(singles)
    _fill(b, rng, [1], 2)
    r = pc.QuantizedRotatingSDPACache(8, keep=2, bits=8, group_size=64)
    _fill(r, rng, [3] + [1] * 9, 1)
    rb = pc.BatchQuantizedRotatingSDPACache([0, 1], 8, keep=0, bits=4, group_size=32)
    _fill(rb, rng, [4] + [1] * 7, 2)
    return [a, b, r, rb, pc.QuantizedSDPACache()]


def test_save_load_roundtrip(cpu_kernels, tmp_path, rng):
    caches = _caches(rng)
    path = tmp_path / "caches.safetensors"
    mq.save_cache(path, caches, metadata={"model": "synthetic"})
    loaded, meta = mq.load_cache(path, return_metadata=True)
    assert meta["model"] == "synthetic"
    for i, (c, l) in enumerate(zip(caches, loaded)):
        assert type(c) is type(l) and c.meta_state == l.meta_state, i
        sc, sl = c.state, l.state
        for j in range(2):
            if sc[j] is None:
                assert sl[j] is None
            else:
                assert_same_rows(_np3(sl[j]), _np3(sc[j]), "f16", f"cache {i} state {j}")
        if len(sc) == 4:
            assert sc[2].tolist() == sl[2].tolist() and sc[3].tolist() == sl[3].tolist()
    # Both go on updating with the same tokens and keep equal (temporal) states.
    for i, (c, l) in enumerate(zip(caches[:4], loaded[:4])):
        B = c.state[0][0].shape[0]
        for step, S in enumerate([1, 1, 3, 1]):
            seed = 100 * i + step
            _fill(c, np.random.default_rng(seed), [S], B)
            _fill(l, np.random.default_rng(seed), [S], B)
            for j in range(2):
                assert_same_rows(_np3(l.state[j]), _np3(c.state[j]), "f16", f"cache {i} step {step}")
            assert np.array_equal(np.asarray(c.offset), np.asarray(l.offset))
