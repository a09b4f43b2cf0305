"""GPU parity at the BASELINE configurations' full sizes, and the decode-loop
patterns that smaller cases do not exercise.

* C3 (GQA-16, D=256, 4-bit gs32, fp16) at N = 32K, 64K, 128K and 1M keys;
  C2 (H_q = H_kv = 2, D=256, 8-bit gs64, bf16, 1% outlier channels x8) at
  N = 64K and 128K: the fused kernel (through the C ABI) against the float64
  oracle (tests/torch_oracle.py, pinned here to oracle/attention.py).
* C4 at full shape through BatchQuantizedSDPACache.update_and_fetch and
  cache_sdpa (left padding as kv_start and as an additive mask).
* C5 end to end through BatchQuantizedRotatingSDPACache (B=4, H_q=16,
  H_kv=4, D=128, 8-bit gs128, bf16, window 4096, keep=4): advanced past the
  wrap, a qL=512 causal chunk, then 64 decode steps; every step's cache
  views are bit-exact against the oracle caches and every attention output
  is within tolerance of the float64 oracle (reference anchor:
  tests/test_rotating_sdpa_integration.py:6-65 of mlx-qsdpa).
* One DecodePlan reused back to back on the same stream with its inputs
  overwritten in place between calls (no host synchronisation): each output
  matches the oracle for its own inputs.
* The rotating-window invariants of tests/test_cache_invariants.py on the
  HIP quantize / dequantize kernels.
* qL > 1 calls the fused kernel does not take (D = 64, a K view whose rows
  are not 16-byte aligned) through the dequantize + attention path.
* Head dims the library does not compile (D = 32, 512) at qL = 1 and > 1
  through the same path.

Tolerance (north star): |out - ref| <= 2e-3 + 1e-2 |ref|.
"""

import numpy as np
import pytest
import torch

import torch_oracle
from conftest import from_np, to_np, torch_dtype
from oracle import affine, attention
from oracle import caches as oc
from test_cache_invariants import CASES as WINDOW_CASES, run_window_invariants

import mlx_qsdpa_amd as mq
from mlx_qsdpa_amd import kernels

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-3, 1e-2


def assert_close(got, want, ctx):
    got, want = got.double(), want.double()
    err = (got - want).abs()
    bad = err > ATOL + RTOL * want.abs()
    assert bool(torch.isfinite(got).all()), f"{ctx}: non-finite output"
    assert not bool(bad.any()), (f"{ctx}: {int(bad.sum())} of {bad.numel()} outside tolerance, "
                                 f"max abs err {err.max().item():.3e}")


# ---------------------------------------------------------------------------
# the GPU restatement of the oracle, pinned to the numpy oracle
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("case", [
    (2, 8, 2, 77, 128, 4, 32, "f16", None),
    (1, 4, 4, 300, 256, 8, 64, "bf16", "causal"),
    (3, 6, 3, 64, 64, 4, 64, "bf16", "bool"),
    (1, 16, 2, 129, 128, 8, 128, "f16", "additive"),
], ids=["f16-4b", "bf16-8b-causal", "bf16-bool", "f16-additive"])
def test_torch_oracle_matches_numpy_oracle(device, case):
    B, Hq, Hkv, N, D, bits, gs, dt, mk = case
    rng = np.random.default_rng(5)
    L = 5 if mk == "causal" else 1
    q = affine.random_T(rng, (B, Hq, L, D), dt)
    kq = affine.quantize(affine.random_T(rng, (B, Hkv, N, D), dt, outlier_frac=0.02), gs, bits, dt)
    vq = affine.quantize(affine.random_T(rng, (B, Hkv, N, D), dt), gs, bits, dt)
    m_np = m_t = None
    if mk == "causal":
        m_np = m_t = "causal"
    elif mk == "bool":
        m_np = rng.random((B, 1, L, N)) > 0.3
        m_t = torch.from_numpy(m_np).to(device)
    elif mk == "additive":
        m_np = np.where(rng.random((1, Hq, L, N)) > 0.2, rng.standard_normal((1, Hq, L, N)), -np.inf)
        m_t = torch.from_numpy(m_np).to(device)
    T = torch_dtype(dt)
    dev = lambda t: from_np(t, T, device)  # noqa: E731
    k_t = torch_oracle.dequantize(dev(kq[0]), dev(kq[1]), dev(kq[2]), gs, bits, T)
    k_np = affine.dequantize(*kq, gs, bits, dt)
    assert np.array_equal(affine.T_bits(to_np(k_t), dt), affine.T_bits(k_np, dt))
    got = torch_oracle.quantized_sdpa(dev(q), tuple(map(dev, kq)), tuple(map(dev, vq)), bits=bits,
                                      group_size=gs, mask=m_t).cpu().numpy()
    want = attention.quantized_sdpa_reference(q, kq[0], vq[0], kq[1], vq[1], kq[2], vq[2], bits=bits,
                                              group_size=gs, dtype=dt, mask=m_np)
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12)


# ---------------------------------------------------------------------------
# C3 and C2 at full N
# ---------------------------------------------------------------------------
def _synthetic_kv(device, B, Hkv, N, D, bits, gs, T, outliers=0.0, seed=0):
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    out = []
    for _ in range(2):
        w = torch.randn((B, Hkv, N, D), generator=g, device=device)
        if outliers:
            n_out = max(1, round(outliers * D))
            for h in range(Hkv):  # a seeded choice of channels per head, x8
                ch = torch.randperm(D, generator=g, device=device)[:n_out]
                w[:, h, :, ch] *= 8.0
        out.append(kernels.quantize(w.to(T), gs, bits))
        del w
    return out


@pytest.mark.parametrize("N", [32768, 65536, 131072, 1048576])
def test_c3_full_size(device, N):
    B, Hq, Hkv, D, bits, gs, T = 1, 32, 2, 256, 4, 32, torch.float16
    kq, vq = _synthetic_kv(device, B, Hkv, N, D, bits, gs, T, seed=N)
    g = torch.Generator(device=device)
    g.manual_seed(1)
    q = torch.randn((B, Hq, 1, D), generator=g, device=device).to(T)
    want = torch_oracle.quantized_sdpa(q, kq, vq, bits=bits, group_size=gs)
    for splits in (None, 1):
        got = mq.quantized_sdpa(q, kq[0], vq[0], kq[1], vq[1], kq[2], vq[2], bits=bits, group_size=gs,
                                num_splits=splits)
        assert_close(got, want, f"C3 N={N} splits={splits}")


@pytest.mark.parametrize("N", [65536, 131072])
def test_c2_full_size(device, N):
    B, Hq, Hkv, D, bits, gs, T = 1, 2, 2, 256, 8, 64, torch.bfloat16
    kq, vq = _synthetic_kv(device, B, Hkv, N, D, bits, gs, T, outliers=0.01, seed=N + 1)
    g = torch.Generator(device=device)
    g.manual_seed(2)
    q = torch.randn((B, Hq, 1, D), generator=g, device=device).to(T)
    want = torch_oracle.quantized_sdpa(q, kq, vq, bits=bits, group_size=gs)
    for splits in (None, 1):
        got = mq.quantized_sdpa(q, kq[0], vq[0], kq[1], vq[1], kq[2], vq[2], bits=bits, group_size=gs,
                                num_splits=splits)
        assert_close(got, want, f"C2 N={N} splits={splits}")


# ---------------------------------------------------------------------------
# C5 end to end
# ---------------------------------------------------------------------------
def test_c5_rotating_pipeline(device):
    B, Hq, Hkv, D, bits, gs, W, keep = 4, 16, 4, 128, 8, 128, 4096, 4
    dt, T = "bf16", torch.bfloat16
    rng = np.random.default_rng(55)
    cache = mq.BatchQuantizedRotatingSDPACache([0] * B, max_size=W, keep=keep, bits=bits, group_size=gs)
    ocache = oc.BatchQuantizedRotatingSDPACache([0] * B, max_size=W, keep=keep, bits=bits, group_size=gs,
                                                dtype=dt)

    def step(S, qL, ctx):
        k = affine.random_T(rng, (B, Hkv, S, D), dt, outlier_frac=0.01)
        v = affine.random_T(rng, (B, Hkv, S, D), dt)
        kq, vq = cache.update_and_fetch(from_np(k, T, device), from_np(v, T, device))
        okq, ovq = ocache.update_and_fetch(k, v)
        for got, want in ((kq, okq), (vq, ovq)):
            assert np.array_equal(to_np(got[0]), want[0]), f"{ctx}: packed words differ"
            for i in (1, 2):
                assert np.array_equal(affine.T_bits(to_np(got[i]), dt), affine.T_bits(want[i], dt)), \
                    f"{ctx}: scales / biases differ"
        if qL == 0:
            return
        q = from_np(affine.random_T(rng, (B, Hq, qL, D), dt), T, device)
        mask = "causal" if qL > 1 else None
        out = mq.cache_sdpa(q, kq, vq, cache, mask=mask)
        want = torch_oracle.quantized_sdpa(q, tuple(from_np(x, T, device) for x in okq),
                                           tuple(from_np(x, T, device) for x in ovq),
                                           bits=bits, group_size=gs, mask=mask)
        assert_close(out, want, ctx)

    # Advance every sequence past the wrap: a long prompt (the window keeps
    # the 4 sinks and the newest 4092 tokens), then decodes that cycle the
    # ring over [keep, 4096).
    step(10000, 0, "prompt of 10000 tokens")
    for i in range(150):
        step(1, 0, f"advance {i}")
    assert cache._idx > W
    step(512, 512, "qL=512 causal chunk after the wrap")
    for i in range(64):
        step(1, 1, f"decode {i}")


# ---------------------------------------------------------------------------
# C4 at full shape through the batch cache
# ---------------------------------------------------------------------------
def test_c4_batch_cache_full_shape(device):
    """C4 (B=16, H_q=32, H_kv=8, D=128, 4-bit gs64, f16, lengths U[1K, 32K]
    left-padded) through the API: BatchQuantizedSDPACache.update_and_fetch
    (a left-padded prompt, then one appended token per sequence and step)
    and cache_sdpa, with the padding as kv_start and as an additive -inf
    mask (reference anchor: tests/test_cache_sdpa.py:177-344 of mlx-qsdpa).

    Cache state: a seeded sample of 4096 prompt rows and every appended
    column are bit-exact against the numpy quantizer; the prompt part is
    unchanged by each append (also across the growth by 256 slots); offsets,
    left padding and the key count follow the oracle cache (run on
    one-head D=32 stand-ins of the same token counts, which is all they
    depend on).  Attention: within tolerance of the float64 oracle over the
    cache's contents with the padding masked."""
    B, Hq, Hkv, D, bits, gs, dt, T = 16, 32, 8, 128, 4, 64, "f16", torch.float16
    gen = torch.Generator(device="cpu")
    gen.manual_seed(4)
    lengths = torch.randint(1024, 32769, (B,), generator=gen).numpy()
    lmax = int(lengths.max())
    lp = (lmax - lengths).tolist()
    cache = mq.BatchQuantizedSDPACache(lp, bits=bits, group_size=gs)
    meta = oc.BatchQuantizedSDPACache(lp, bits=bits, group_size=32, dtype=dt)
    g = torch.Generator(device=device)
    g.manual_seed(4)
    k = torch.randn((B, Hkv, lmax, D), generator=g, device=device).to(T)
    v = torch.randn((B, Hkv, lmax, D), generator=g, device=device).to(T)
    kq, vq = cache.update_and_fetch(k, v)
    meta.update_and_fetch(np.zeros((B, 1, lmax, 32), np.float32), np.zeros((B, 1, lmax, 32), np.float32))
    rng = np.random.default_rng(4)
    bs, hs, ts = rng.integers(0, B, 4096), rng.integers(0, Hkv, 4096), rng.integers(0, lmax, 4096)
    for src, got in ((k, kq), (v, vq)):
        want = affine.quantize(to_np(src[bs, hs, ts]), gs, bits, dt)
        assert np.array_equal(got[0].view(torch.int32)[bs, hs, ts].cpu().numpy().view(np.uint32), want[0]), \
            "prompt rows: packed words differ"
        for i in (1, 2):
            assert np.array_equal(affine.T_bits(to_np(got[i][bs, hs, ts]), dt), affine.T_bits(want[i], dt)), \
                "prompt rows: scales / biases differ"
    del k, v
    for step in range(4):
        prev = tuple(t.clone() for t in kq + vq)
        kn = affine.random_T(rng, (B, Hkv, 1, D), dt)
        vn = affine.random_T(rng, (B, Hkv, 1, D), dt)
        kq, vq = cache.update_and_fetch(from_np(kn, T, device), from_np(vn, T, device))
        meta.update_and_fetch(np.zeros((B, 1, 1, 32), np.float32), np.zeros((B, 1, 1, 32), np.float32))
        N = lmax + step + 1
        assert cache.size() == meta.size() == N and kq[0].shape[2] == N
        assert np.array_equal(cache.offset.numpy(), meta.offset)
        assert np.array_equal(cache.left_padding.numpy(), meta.left_padding)
        for old, new in zip(prev, kq + vq):
            assert torch.equal(new[:, :, :N - 1].view(torch.int32) if new.dtype == torch.uint32 else new[:, :, :N - 1],
                               old.view(torch.int32) if old.dtype == torch.uint32 else old), \
                f"step {step}: an append changed earlier columns"
        for src, got in ((kn, kq), (vn, vq)):
            want = affine.quantize(src, gs, bits, dt)
            assert np.array_equal(to_np(got[0][:, :, N - 1:]), want[0]), f"step {step}: appended words differ"
            for i in (1, 2):
                assert np.array_equal(affine.T_bits(to_np(got[i][:, :, N - 1:]), dt), affine.T_bits(want[i], dt)), \
                    f"step {step}: appended scales / biases differ"
        q = from_np(affine.random_T(rng, (B, Hq, 1, D), dt), T, device)
        keep = torch.arange(N, device=device)[None, :] >= torch.tensor(lp, device=device)[:, None]
        want = torch_oracle.quantized_sdpa(q, kq, vq, bits=bits, group_size=gs, mask=keep[:, None, None, :])
        out = mq.cache_sdpa(q, kq, vq, cache, kv_start=cache.kv_start(device))
        assert_close(out, want, f"C4 step {step} kv_start")
        add = torch.zeros((B, 1, 1, N), dtype=T, device=device).masked_fill(~keep[:, None, None, :], float("-inf"))
        out = mq.cache_sdpa(q, kq, vq, cache, mask=add)
        assert_close(out, want, f"C4 step {step} additive mask")


# ---------------------------------------------------------------------------
# one DecodePlan, inputs overwritten in place between calls
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("case", [(1, 32, 2, 8192, 256, 4, 32, "f16"), (3, 16, 4, 3000, 128, 8, 64, "bf16")],
                         ids=["C3-like", "B3-G4-bf16"])
def test_decode_plan_back_to_back(device, case):
    """Four calls of one split-K plan on one stream, each preceded by an
    in-place copy of new inputs into the plan's buffers; no host sync until
    the end.  The reused partials / schedule must not leak between calls."""
    B, Hq, Hkv, N, D, bits, gs, dt = case
    T = torch_dtype(dt)
    rng = np.random.default_rng(88)
    sets = []
    for _ in range(4):
        q = affine.random_T(rng, (B, Hq, 1, D), dt)
        kq = affine.quantize(affine.random_T(rng, (B, Hkv, N, D), dt), gs, bits, dt)
        vq = affine.quantize(affine.random_T(rng, (B, Hkv, N, D), dt), gs, bits, dt)
        sets.append((q, kq, vq))

    def dev(x):
        return from_np(x, T, device)  # uint32 arrays keep their type

    host = [(dev(q), tuple(map(dev, kq)), tuple(map(dev, vq))) for q, kq, vq in sets]
    bufs = [host[0][0].clone(), *[t.clone() for t in host[0][1]], *[t.clone() for t in host[0][2]]]
    plan = kernels.DecodePlan(bufs[0], bufs[1], bufs[4], bufs[2], bufs[5], bufs[3], bufs[6], scale=D ** -0.5,
                              bits=bits, group_size=gs, num_splits=0)
    assert plan.num_splits > 1
    outs = []
    order = [1, 2, 3, 0, 2]
    for i in order:
        src = [host[i][0], *host[i][1], *host[i][2]]
        for dst, s in zip(bufs, src):
            dst.copy_(s, non_blocking=True)
        outs.append(plan().clone())
    torch.cuda.synchronize()
    for i, out in zip(order, outs):
        q, kq, vq = sets[i]
        want = attention.quantized_sdpa_reference(q, kq[0], vq[0], kq[1], vq[1], kq[2], vq[2], bits=bits,
                                                  group_size=gs, dtype=dt)
        assert_close(out, torch.from_numpy(want).to(device), f"{case} inputs {i}")
    assert torch.equal(outs[1], outs[4]), "the same inputs gave different outputs"


# ---------------------------------------------------------------------------
# rotating-window invariants on the HIP kernels
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("kind", ["single", "batch"])
@pytest.mark.parametrize("case", WINDOW_CASES, ids=lambda c: "W{}_keep{}_b{}_g{}_{}".format(*c[:5]))
def test_rotating_window_invariants_on_gpu(device, kind, case):
    max_size, keep, bits, gs, dtype, seed = case
    run_window_invariants(kind, "product", max_size, keep, bits, gs, dtype, seed, device=device)


# ---------------------------------------------------------------------------
# qL > 1 through dequantize + attention
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("layout", ["D64", "scales-2B-aligned"])
def test_multi_query_fallback_path(device, monkeypatch, layout):
    """Shapes the fused kernel does not take for qL > 1 run the reference's
    path (dispatch.py:68-83): HIP dequantize, float32 attention.  The fused
    kernel is made to fail, so passing proves the fallback ran; causal, a
    bool mask and kv_start (folded into the mask) are covered.  Layouts: D =
    64, and K scale / bias rows only 2-byte aligned where the matrix-core
    kernel reads a quarter row's two groups as one 32-bit word (D = 256,
    group_size = 32)."""
    B, Hq, Hkv, N, L = 2, 8, 2, 200, 6
    D, bits, gs, dt = (64, 4, 32, "f16") if layout == "D64" else (256, 4, 32, "bf16")
    T = torch_dtype(dt)
    rng = np.random.default_rng(66)
    q = affine.random_T(rng, (B, Hq, L, D), dt)
    kq = affine.quantize(affine.random_T(rng, (B, Hkv, N, D), dt), gs, bits, dt)
    vq = affine.quantize(affine.random_T(rng, (B, Hkv, N, D), dt), gs, bits, dt)

    def dev(x):
        return from_np(x, T, device)  # uint32 arrays keep their type

    dk, dv = tuple(map(dev, kq)), tuple(map(dev, vq))
    if layout == "scales-2B-aligned":
        # K scale and bias rows one element (2 bytes) off a 4-byte boundary:
        # views into wider buffers.
        G = kq[1].shape[-1]
        views = []
        for t in (dk[1], dk[2]):
            wide = torch.zeros((B, Hkv, N, G + 1), dtype=T, device=device)
            wide[..., 1:] = t
            views.append(wide[..., 1:])
        dk = (dk[0], views[0], views[1])

    def no_fused(*a, **k):
        raise AssertionError("the fused kernel ran")

    monkeypatch.setattr(kernels, "decode", no_fused)
    starts = np.array([0, 37])
    for mask in ("causal", "bool", None):
        m_t = m_np = None
        if mask == "causal":
            m_t = m_np = "causal"
        elif mask == "bool":
            m_np = rng.random((B, 1, L, N)) > 0.4
            m_np[..., -1] = True
            m_t = torch.from_numpy(m_np).to(device)
        got = mq.quantized_sdpa(dev(q), dk[0], dv[0], dk[1], dv[1], dk[2], dv[2], bits=bits, group_size=gs,
                                mask=m_t, kv_start=torch.tensor(starts, dtype=torch.int32, device=device))
        keep = np.arange(N)[None, None, None, :] >= starts[:, None, None, None]
        if mask == "causal":
            qi = np.arange(L)[:, None] + (N - L)
            full = keep & (qi >= np.arange(N)[None, :])[None, None]
        elif mask == "bool":
            full = keep & m_np
        else:
            full = np.broadcast_to(keep, (B, 1, L, N))
        want = attention.quantized_sdpa_reference(q, kq[0], vq[0], kq[1], vq[1], kq[2], vq[2], bits=bits,
                                                  group_size=gs, dtype=dt, mask=full)
        assert_close(got, torch.from_numpy(want).to(device), f"{layout} mask={mask}")


@pytest.mark.parametrize("D,bits,gs,dt", [(32, 4, 32, "f16"), (512, 8, 64, "bf16"), (512, 4, 128, "f16")],
                         ids=["D32-4b", "D512-8b", "D512-4b-gs128"])
def test_uncompiled_head_dims(device, monkeypatch, D, bits, gs, dt):
    """Head dims the library does not compile (the reference's validation
    accepts any D % 32 == 0: dispatch.py:48-49, kernels templated on D:
    kernels.py:44-50) return the attention through dequantize + attention,
    for one query position and for several, unmasked, bool-masked, additive
    and causal, with and without kv_start.  The fused kernel is made to
    fail, so passing proves the fallback ran."""
    B, Hq, Hkv, N = 2, 8, 2, 150
    T = torch_dtype(dt)
    rng = np.random.default_rng(D + bits)
    kq = affine.quantize(affine.random_T(rng, (B, Hkv, N, D), dt), gs, bits, dt)
    vq = affine.quantize(affine.random_T(rng, (B, Hkv, N, D), dt), gs, bits, dt)
    dk = tuple(from_np(x, T, device) for x in kq)
    dv = tuple(from_np(x, T, device) for x in vq)

    def no_fused(*a, **k):
        raise AssertionError("the fused kernel ran")

    monkeypatch.setattr(kernels, "decode", no_fused)
    monkeypatch.setattr(kernels, "decode_repeat", no_fused)
    for L in (1, 3):
        q = affine.random_T(rng, (B, Hq, L, D), dt)
        for mask in (None, "bool", "additive", "causal"):
            for starts in (None, np.array([0, 41])):
                m_t = m_np = None
                if mask == "causal":
                    m_t = m_np = "causal"
                elif mask == "bool":
                    m_np = rng.random((B, 1, L, N)) > 0.4
                    m_np[..., -1] = True
                    m_t = torch.from_numpy(m_np).to(device)
                elif mask == "additive":
                    m_np = affine.random_T(rng, (B, 1, L, N), dt)
                    m_np[rng.random((B, 1, L, N)) < 0.3] = -np.inf
                    m_np[..., -1] = 0.0
                    m_t = from_np(m_np, T, device)
                ks = None if starts is None else torch.tensor(starts, dtype=torch.int32, device=device)
                got = mq.quantized_sdpa(from_np(q, T, device), dk[0], dv[0], dk[1], dv[1], dk[2], dv[2],
                                        bits=bits, group_size=gs, mask=m_t, kv_start=ks)
                full = m_np
                if starts is not None:
                    keep = np.arange(N)[None, None, None, :] >= starts[:, None, None, None]
                    if mask is None:
                        full = np.broadcast_to(keep, (B, 1, L, N))
                    elif mask == "causal":
                        qi = np.arange(L)[:, None] + (N - L)
                        full = keep & (qi >= np.arange(N)[None, :])[None, None]
                    elif mask == "bool":
                        full = keep & m_np
                    else:
                        full = np.where(keep, m_np, -np.inf).astype(np.float32)
                want = attention.quantized_sdpa_reference(q, kq[0], vq[0], kq[1], vq[1], kq[2], vq[2],
                                                          bits=bits, group_size=gs, dtype=dt, mask=full)
                assert got.shape == (B, Hq, L, D) and got.dtype == T
                assert_close(got, torch.from_numpy(want).to(device),
                             f"D={D} L={L} mask={mask} kv_start={starts is not None}")


def test_misaligned_packed_rows_are_copied(device):
    """Packed K / V views whose rows are not 16-byte aligned (one word into a
    wider buffer) decode correctly, through a copy (the reference copies
    every input, kernels.py:190), for one query position and for several."""
    B, Hq, Hkv, N, D, bits, gs, dt = 2, 16, 2, 300, 128, 4, 32, "f16"
    T = torch_dtype(dt)
    rng = np.random.default_rng(67)
    kq = affine.quantize(affine.random_T(rng, (B, Hkv, N, D), dt), gs, bits, dt)
    vq = affine.quantize(affine.random_T(rng, (B, Hkv, N, D), dt), gs, bits, dt)
    W = kq[0].shape[-1]
    packed = []
    for p in (kq[0], vq[0]):
        wide = torch.zeros((B, Hkv, N, W + 1), dtype=torch.uint32, device=device)
        wide[..., 1:] = from_np(p, T, device)
        packed.append(wide[..., 1:])
        assert packed[-1].data_ptr() % 16 != 0
    for L, mask in ((1, None), (5, "causal")):
        q = affine.random_T(rng, (B, Hq, L, D), dt)
        got = mq.quantized_sdpa(from_np(q, T, device), packed[0], packed[1], from_np(kq[1], T, device),
                                from_np(vq[1], T, device), from_np(kq[2], T, device), from_np(vq[2], T, device),
                                bits=bits, group_size=gs, mask=mask)
        want = attention.quantized_sdpa_reference(q, kq[0], vq[0], kq[1], vq[1], kq[2], vq[2], bits=bits,
                                                  group_size=gs, dtype=dt, mask=mask)
        assert_close(got, torch.from_numpy(want).to(device), f"misaligned packed rows, qL={L}")
