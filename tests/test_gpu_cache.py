"""Caches on the GPU: every update runs the HIP quantize / dequantize kernels;
buffers, counters and fetched views must equal the oracle caches bit-exactly.
Plus the cache -> kernel pipeline (cache_sdpa) against the oracle.
"""

import numpy as np
import pytest
import torch

from cache_scenarios import SCENARIOS, run_scenario
from conftest import from_np, to_np
from oracle import affine, attention
from oracle import caches as oc

import mlx_qsdpa_amd as mq

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-3, 1e-2


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
@pytest.mark.parametrize("sc", SCENARIOS, ids=lambda s: s[0])
def test_scenarios_bit_exact(device, sc, dtype):
    run_scenario(*sc, dtype=dtype, device=device)


def _close(got, want, ctx):
    err = np.abs(got - want)
    assert np.all(err <= ATOL + RTOL * np.abs(want)), f"{ctx}: max err {err.max():.3e}"


@pytest.mark.parametrize("crossover", [0, 10 ** 9])
def test_cache_sdpa_paths(device, crossover):
    """__init__.py:12-68: both dispatch branches agree with the oracle."""
    rng = np.random.default_rng(21)
    B, Hq, Hkv, N, D = 1, 32, 2, 1000, 256
    c = mq.QuantizedSDPACache(bits=4, group_size=32)
    oc_ = oc.QuantizedSDPACache(bits=4, group_size=32)
    k = affine.random_T(rng, (B, Hkv, N, D), "f16")
    v = affine.random_T(rng, (B, Hkv, N, D), "f16")
    kq, vq = c.update_and_fetch(from_np(k, torch.float16, device), from_np(v, torch.float16, device))
    okq, ovq = oc_.update_and_fetch(k, v)
    q = affine.random_T(rng, (B, Hq, 1, D), "f16")
    out = mq.cache_sdpa(from_np(q, torch.float16, device), kq, vq, c, crossover=crossover)
    want = attention.quantized_sdpa_reference(q, *okq[:1], ovq[0], okq[1], ovq[1], okq[2], ovq[2],
                                              bits=4, group_size=32, dtype="f16")
    _close(to_np(out), want, f"crossover={crossover}")


def test_cache_sdpa_prefill_and_mask(device):
    rng = np.random.default_rng(22)
    B, Hq, Hkv, N, D = 1, 4, 2, 64, 256
    c = mq.QuantizedSDPACache(bits=8, group_size=32)
    k = affine.random_T(rng, (B, Hkv, N, D), "f16")
    v = affine.random_T(rng, (B, Hkv, N, D), "f16")
    kq, vq = c.update_and_fetch(from_np(k, torch.float16, device), from_np(v, torch.float16, device))
    okq, ovq = oc.QuantizedSDPACache(bits=8, group_size=32).update_and_fetch(k, v)
    ref_args = (okq[0], ovq[0], okq[1], ovq[1], okq[2], ovq[2])
    q8 = affine.random_T(rng, (B, Hq, 8, D), "f16")
    out = mq.cache_sdpa(from_np(q8, torch.float16, device), kq, vq, c, mask="causal")
    want = attention.quantized_sdpa_reference(q8, *ref_args, bits=8, group_size=32, dtype="f16",
                                              mask="causal")
    _close(to_np(out), want, "prefill")
    q1 = affine.random_T(rng, (B, Hq, 1, D), "f16")
    keep = (np.arange(N) >= N - 8)[None, None, None, :]
    out = mq.cache_sdpa(from_np(q1, torch.float16, device), kq, vq, c, crossover=0,
                        mask=torch.from_numpy(keep).to(device))
    want = attention.quantized_sdpa_reference(q1, *ref_args, bits=8, group_size=32, dtype="f16",
                                              mask=keep)
    _close(to_np(out), want, "masked decode")


def test_batched_decode_pipeline(device):
    """C4 shape: left-padded batch cache, append one token per sequence, decode
    with kv_start = left padding; compare with the oracle (additive -inf mask)."""
    rng = np.random.default_rng(23)
    B, Hq, Hkv, D, bits, gs = 4, 32, 8, 128, 4, 64
    lengths = [700, 1200, 65, 1024]
    singles, osingles = [], []
    for n in lengths:
        k = affine.random_T(rng, (1, Hkv, n, D), "f16")
        v = affine.random_T(rng, (1, Hkv, n, D), "f16")
        s = mq.QuantizedSDPACache(bits=bits, group_size=gs)
        s.update_and_fetch(from_np(k, torch.float16, device), from_np(v, torch.float16, device))
        o = oc.QuantizedSDPACache(bits=bits, group_size=gs, dtype="f16")
        o.update_and_fetch(k, v)
        singles.append(s)
        osingles.append(o)
    batch = mq.BatchQuantizedSDPACache.merge(singles)
    obatch = oc.BatchQuantizedSDPACache.merge(osingles)
    for step in range(3):
        k = affine.random_T(rng, (B, Hkv, 1, D), "f16")
        v = affine.random_T(rng, (B, Hkv, 1, D), "f16")
        kq, vq = batch.update_and_fetch(from_np(k, torch.float16, device),
                                        from_np(v, torch.float16, device))
        okq, ovq = obatch.update_and_fetch(k, v)
        assert np.array_equal(to_np(kq[0]), okq[0])
        q = affine.random_T(rng, (B, Hq, 1, D), "f16")
        N = okq[0].shape[2]
        lp = obatch.left_padding
        add = np.where(np.arange(N)[None, :] >= lp[:, None], 0.0, -np.inf)[:, None, None, :]
        want = attention.quantized_sdpa_reference(q, okq[0], ovq[0], okq[1], ovq[1], okq[2], ovq[2],
                                                  bits=bits, group_size=gs, dtype="f16", mask=add)
        out = mq.cache_sdpa(from_np(q, torch.float16, device), kq, vq, batch,
                            kv_start=batch.kv_start(device))
        _close(to_np(out), want, f"batched step {step}")


def test_rotating_window_pipeline(device):
    """C5 shape (small): rotating batch cache with sinks; prefill chunk after the
    ring wrapped (causal, through the fallback), then decode steps (fused)."""
    rng = np.random.default_rng(24)
    B, Hq, Hkv, D, bits, gs, W, keep = 2, 16, 4, 128, 8, 128, 64, 4
    T = torch.bfloat16
    c = mq.BatchQuantizedRotatingSDPACache([0, 0], max_size=W, keep=keep, bits=bits, group_size=gs)
    o = oc.BatchQuantizedRotatingSDPACache([0, 0], max_size=W, keep=keep, bits=bits,
                                           group_size=gs, dtype="bf16")

    def step(S, qL):
        k = affine.random_T(rng, (B, Hkv, S, D), "bf16", outlier_frac=0.01)
        v = affine.random_T(rng, (B, Hkv, S, D), "bf16")
        kq, vq = c.update_and_fetch(from_np(k, T, device), from_np(v, T, device))
        okq, ovq = o.update_and_fetch(k, v)
        for i in range(3):
            g = to_np(kq[i])
            assert np.array_equal(g if i == 0 else affine.T_bits(g, "bf16"),
                                  okq[i] if i == 0 else affine.T_bits(okq[i], "bf16"))
        q = affine.random_T(rng, (B, Hq, qL, D), "bf16")
        mask = "causal" if qL > 1 else None
        out = mq.cache_sdpa(from_np(q, T, device), kq, vq, c, mask=mask)
        want = attention.quantized_sdpa_reference(q, okq[0], ovq[0], okq[1], ovq[1], okq[2],
                                                  ovq[2], bits=bits, group_size=gs, dtype="bf16",
                                                  mask=mask)
        _close(to_np(out), want, f"S={S} qL={qL} idx={c._idx}")

    step(40, 40)
    for _ in range(60):
        step(1, 1)
    step(20, 20)
    for _ in range(5):
        step(1, 1)
