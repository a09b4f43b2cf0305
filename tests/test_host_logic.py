"""Host logic of the shipped package, on CPU.

The cache classes run with their two kernel wrappers (quantize_into,
dequantize) replaced by the oracle, so every index / mask / growth /
state-machine rule is exercised against the reference's own expectations
(tests/golden/reference_fixtures.json) and against the oracle caches.
"""

import json

import numpy as np
import pytest
import torch

from cache_scenarios import SCENARIOS, run_scenario
from conftest import GOLDEN, from_np, to_np
from oracle import affine, metric as ometric
from oracle import caches as oc

import mlx_qsdpa_amd as mq
from mlx_qsdpa_amd import cache as pc, metric

REF = json.loads((GOLDEN / "reference_fixtures.json").read_text())


def _kv(rng, B, H, S, D, dtype=torch.float16):
    name = "f16" if dtype == torch.float16 else "bf16"
    return (from_np(affine.random_T(rng, (B, H, S, D), name), dtype),
            from_np(affine.random_T(rng, (B, H, S, D), name), dtype))


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
@pytest.mark.parametrize("sc", SCENARIOS, ids=lambda s: s[0])
def test_scenarios_match_oracle(cpu_kernels, sc, dtype):
    run_scenario(*sc, dtype=dtype)


# ---- reference expectations (rotating) -----------------------------------
def _decode_n(c, rng, n, B=1, H=1, D=64):
    out = None
    for _ in range(n):
        out = c.update_and_fetch(*_kv(rng, B, H, 1, D))
    return out


def test_rotating_fill_and_wrap(cpu_kernels, rng):
    for key in ("rotating_fill", "rotating_wrap"):
        g = REF[key]
        c = pc.QuantizedRotatingSDPACache(max_size=g["max_size"], bits=4, group_size=32)
        k, _ = _decode_n(c, rng, g["decodes"])
        assert (c.offset, c._idx, c.size(), k[0].shape[2]) == (g["offset"], g["idx"], g["size"],
                                                                g["k_len"])


def test_rotating_single_step(cpu_kernels, rng):
    g = REF["rotating_single_step"]
    c = pc.QuantizedRotatingSDPACache(max_size=g["max_size"], bits=4, group_size=32)
    k, v = c.update_and_fetch(*_kv(rng, 1, 2, 1, 256))
    assert len(k) == 3 and len(v) == 3
    assert (c.offset, c._idx, k[0].shape[2]) == (g["offset"], g["idx"], g["k_len"])


def test_rotating_nbytes_fixed(cpu_kernels, rng):
    g = REF["rotating_nbytes_fixed"]
    c = pc.QuantizedRotatingSDPACache(max_size=g["max_size"], bits=4, group_size=32)
    assert c.nbytes == 0
    _decode_n(c, rng, 1)
    n0 = c.nbytes
    _decode_n(c, rng, g["decodes_after_first"])
    assert c.nbytes == n0 > 0


def test_rotating_mask_and_trim(cpu_kernels, rng):
    g = REF["rotating_mask_before_rotation"]
    c = pc.QuantizedRotatingSDPACache(max_size=g["max_size"], bits=4, group_size=32)
    _decode_n(c, rng, g["decodes"], H=2)
    assert c.make_mask(1, return_array=True) is None
    assert list(c.make_mask(g["N"], return_array=True).shape[-2:]) == g["mask_shape_last2"]
    assert pc.QuantizedRotatingSDPACache(max_size=16).make_mask(1) is None
    g = REF["rotating_trim"]
    c = pc.QuantizedRotatingSDPACache(max_size=g["max_size"], bits=4, group_size=32)
    _decode_n(c, rng, g["decodes"], H=2)
    assert c.is_trimmable()
    assert c.trim(g["trim"]) == g["trimmed"]
    assert (c.offset, c._idx) == (g["offset"], g["idx"])
    g = REF["rotating_not_trimmable"]
    c = pc.QuantizedRotatingSDPACache(max_size=g["max_size"], bits=4, group_size=32)
    _decode_n(c, rng, g["decodes"], H=2)
    assert c.is_trimmable() is g["trimmable"]


def test_rotating_prefill_paths(cpu_kernels, rng):
    g = REF["rotating_prefill"]
    c = pc.QuantizedRotatingSDPACache(max_size=g["max_size"], bits=4, group_size=32)
    k, _ = c.update_and_fetch(*_kv(rng, 1, 2, g["S"], 64))
    assert (c.offset, k[0].shape[2]) == (g["offset"], g["k_len"])
    g = REF["rotating_prefill_exceeds"]
    c = pc.QuantizedRotatingSDPACache(max_size=g["max_size"], bits=4, group_size=32)
    k, _ = c.update_and_fetch(*_kv(rng, 1, 2, g["S"], 64))
    assert (c.offset, c.size(), k[0].shape[2]) == (g["offset"], g["size"], g["k_len"])
    g = REF["rotating_prefill_then_decode"]
    c = pc.QuantizedRotatingSDPACache(max_size=g["max_size"], bits=4, group_size=32)
    c.update_and_fetch(*_kv(rng, 1, 2, g["S"], 64))
    assert (c.offset, c._idx) == (g["after_prefill"]["offset"], g["after_prefill"]["idx"])
    k, _ = _decode_n(c, rng, g["decodes"], H=2)
    a = g["after_decode"]
    assert (c.offset, c._idx, c.size(), k[0].shape[2]) == (a["offset"], a["idx"], a["size"],
                                                            a["k_len"])


def test_rotating_state_roundtrip(cpu_kernels, rng):
    """tests/test_rotating_cache.py:189-210: restored cache writes identically."""
    c = pc.QuantizedRotatingSDPACache(max_size=16, bits=4, group_size=32)
    _decode_n(c, rng, 5, H=2)
    c2 = pc.QuantizedRotatingSDPACache(max_size=16, bits=4, group_size=32)
    c2.state = c.state
    c2.offset, c2._idx = c.offset, c._idx
    k, v = _kv(rng, 1, 2, 1, 64)
    k1, v1 = c.update_and_fetch(k, v)
    k2, v2 = c2.update_and_fetch(k, v)
    assert torch.equal(k1[0], k2[0]) and torch.equal(v1[0], v2[0])


def test_rotating_keep_validation():
    with pytest.raises(ValueError):
        pc.QuantizedRotatingSDPACache(max_size=8, keep=8)
    with pytest.raises(ValueError):
        pc.QuantizedRotatingSDPACache(max_size=8, bits=3)
    c = pc.QuantizedRotatingSDPACache(max_size=8, keep=4)
    assert c.keep == 4


# ---- reference expectations (batch rotating) ------------------------------
def test_batch_rotating_reference_cases(cpu_kernels, rng):
    g = REF["batch_rotating_decode_wrap"]
    c = pc.BatchQuantizedRotatingSDPACache([0] * g["B"], max_size=g["max_size"], bits=4,
                                           group_size=32)
    k, _ = _decode_n(c, rng, g["decodes"], B=g["B"], H=2)
    assert (c.size(), k[0].shape[2], k[0].shape[0]) == (g["size"], g["k_len"], g["B"])
    g = REF["batch_rotating_multi_token"]
    c = pc.BatchQuantizedRotatingSDPACache([0] * g["B"], max_size=g["max_size"], bits=4,
                                           group_size=32)
    for S in g["chunks"]:
        k, _ = c.update_and_fetch(*_kv(rng, g["B"], g["H_kv"], S, g["D"]))
    assert c.size() == g["size"] and list(k[0].shape) == g["k_shape"]
    g = REF["batch_rotating_filter"]
    c = pc.BatchQuantizedRotatingSDPACache([0, 0], max_size=g["max_size"], bits=4, group_size=32)
    _decode_n(c, rng, g["decodes"], B=2, H=2)
    c.filter(torch.tensor(g["keep_index"]))
    assert c._keys[0].shape[0] == g["B_after"] and c.offset.shape[0] == g["B_after"]
    g = REF["batch_rotating_extract"]
    c = pc.BatchQuantizedRotatingSDPACache([0, 0], max_size=g["max_size"], bits=4, group_size=32)
    _decode_n(c, rng, g["decodes"], B=2, H=2)
    e = c.extract(0)
    assert isinstance(e, pc.QuantizedRotatingSDPACache)
    assert e.offset == g["offset"] and e.max_size == g["max_size"]


def test_batch_rotating_extract_after_wrap(cpu_kernels, rng):
    """tests/test_batch_rotating_cache.py:160-181: extract == quantize(last 4 keys)."""
    g = REF["batch_rotating_extract_after_wrap"]
    c = pc.BatchQuantizedRotatingSDPACache([0], max_size=g["max_size"], bits=4, group_size=32)
    keys = []
    for _ in range(g["decodes"]):
        k, v = _kv(rng, 1, 1, 1, 64)
        keys.append(k)
        c.update_and_fetch(k, v)
    e = c.extract(0)
    want = affine.quantize(to_np(torch.cat(keys[-g["last"]:], dim=2)), 32, 4, "f16")[0]
    assert e.offset == g["offset"]
    assert np.array_equal(to_np(e.state[0][0]), want)


def test_batch_rotating_merge_singles(cpu_kernels, rng):
    caches = []
    for n in (3, 5):
        c = pc.QuantizedRotatingSDPACache(max_size=16, bits=4, group_size=32)
        _decode_n(c, rng, n, H=2)
        caches.append(c)
    b = pc.BatchQuantizedRotatingSDPACache.merge(caches)
    assert isinstance(b, pc.BatchQuantizedRotatingSDPACache)
    assert b._keys[0].shape[0] == 2 and b.max_size == 16


@pytest.mark.parametrize("key,cls", [("batch_mask_left_padding", "single"),
                                     ("batch_rotating_mask_left_padding", "rot")])
def test_mask_goldens(cpu_kernels, rng, key, cls):
    g = REF[key]
    cs = []
    for n in g["lengths"]:
        if cls == "single":
            c = pc.QuantizedSDPACache(bits=4, group_size=32)
            c.update_and_fetch(*_kv(rng, 1, 2, n, 256))
        else:
            c = pc.QuantizedRotatingSDPACache(max_size=g["max_size"], bits=4, group_size=32)
            _decode_n(c, rng, n, H=2)
        cs.append(c)
    batch = (pc.QuantizedSDPACache.merge(cs) if cls == "single"
             else pc.BatchQuantizedRotatingSDPACache.merge(cs))
    mask = batch.make_mask(g["N"])
    assert list(mask.shape) == g["shape"]
    assert torch.equal(mask.cpu(), torch.tensor(g["expected"]))


# ---- reference expectations (single / batch) -------------------------------
def test_cache_defaults_and_protocol(cpu_kernels, rng):
    c = mq.QuantizedSDPACache()
    assert (c.bits, c.group_size, c.offset) == (4, 32, 0)
    assert c.empty() and c.nbytes == 0 and c.is_trimmable()
    assert c.make_mask(N=1) is None and c.make_mask(N=8) == "causal"
    c2 = mq.QuantizedSDPACache(bits=8, group_size=64, step=512)
    assert (c2.bits, c2.group_size) == (8, 64)
    with pytest.raises(ValueError):
        mq.QuantizedSDPACache(bits=5)
    k, v = c.update_and_fetch(*_kv(rng, 1, 2, 1, 256))
    assert k[0].shape == (1, 2, 1, 32) and k[0].dtype == torch.uint32
    assert k[1].shape == (1, 2, 1, 8) and k[1].dtype == torch.float16
    assert c.nbytes > 0


def test_cache_growth_and_trim(cpu_kernels, rng):
    g = REF["cache_growth"]
    c = pc.QuantizedSDPACache(bits=4, group_size=32, step=g["step"])
    for S in g["chunks"]:
        k, _ = c.update_and_fetch(*_kv(rng, 1, 2, S, 256))
    assert c.offset == g["offset"] and k[0].shape[2] == g["k_len"]
    for case in REF["cache_trim"]["cases"]:
        c = pc.QuantizedSDPACache(bits=4, group_size=32)
        c.update_and_fetch(*_kv(rng, 1, 2, case["fill"], 256))
        assert c.trim(case["trim"]) == case["trimmed"] and c.offset == case["offset"]


def test_cache_state_roundtrip(cpu_kernels, rng):
    c = pc.QuantizedSDPACache(bits=4, group_size=32)
    kq, _ = c.update_and_fetch(*_kv(rng, 1, 2, 20, 256))
    c2 = pc.QuantizedSDPACache.from_state(c.state, c.meta_state)
    assert (c2.offset, c2.bits, c2.group_size) == (20, 4, 32)
    assert torch.equal(kq[0], c2.state[0][0])


def test_merge_and_extract(cpu_kernels, rng):
    g = REF["cache_merge_extract"]
    cs = []
    for n in g["lengths"]:
        c = pc.QuantizedSDPACache(bits=4, group_size=32)
        c.update_and_fetch(*_kv(rng, 1, 2, n, 256))
        cs.append(c)
    b = pc.QuantizedSDPACache.merge(cs)
    assert isinstance(b, pc.BatchQuantizedSDPACache)
    st = b.state
    assert st[2].shape[0] == g["state_batch"] and st[3].shape[0] == g["state_batch"]
    assert [b.extract(i).offset for i in range(2)] == g["extract_offsets"]
    # extracted tokens are the original ones
    for i, c in enumerate(cs):
        e = b.extract(i)
        assert torch.equal(e._keys[0], c.state[0][0])


def test_batch_prepare_finalize_matches_oracle(cpu_kernels, rng):
    """prepare(right_padding) + finalize roll (cache.py:324-348, 46-51)."""
    p = pc.BatchQuantizedSDPACache([0, 0, 0], bits=4, group_size=32)
    o = oc.BatchQuantizedSDPACache([0, 0, 0], bits=4, group_size=32)
    p.prepare(right_padding=[2, 0, 1])
    o.prepare(right_padding=[2, 0, 1])
    k = affine.random_T(rng, (3, 2, 7, 64), "f16")
    v = affine.random_T(rng, (3, 2, 7, 64), "f16")
    p.update_and_fetch(from_np(k, torch.float16), from_np(v, torch.float16))
    o.update_and_fetch(k, v)
    p.finalize()
    o.finalize()
    for i in range(3):
        assert np.array_equal(affine.T_bits(to_np(p._keys[i]), "f16") if i else to_np(p._keys[i]),
                              affine.T_bits(o._keys[i], "f16") if i else o._keys[i])
    assert p.left_padding.tolist() == o.left_padding.tolist()
    assert p.offset.tolist() == o.offset.tolist()
    with pytest.raises(ValueError):
        p.prepare(left_padding=[1, 1, 1])


def test_batch_filter_extend(cpu_kernels, rng):
    a = pc.BatchQuantizedSDPACache([0, 2], bits=4, group_size=32)
    a.update_and_fetch(*_kv(rng, 2, 2, 5, 64))
    b = pc.BatchQuantizedSDPACache([1], bits=4, group_size=32)
    b.update_and_fetch(*_kv(rng, 1, 2, 3, 64))
    a.extend(b)
    assert a._keys[0].shape[0] == 3 and a._idx == 5
    assert a.left_padding.tolist() == [0, 2, 3]
    a.filter([1, 2])
    assert a.left_padding.tolist() == [0, 1] and a._idx == 3


# ---- dispatch / API ----------------------------------------------------------
@pytest.mark.parametrize("case", REF["validation_errors"]["cases"], ids=lambda c: c["match"])
def test_quantized_sdpa_validation(case):
    q = torch.zeros(case["q_shape"], dtype=torch.float16)
    D = case["q_shape"][-1]
    bits = case["bits"]
    H_kv = case.get("H_kv", 1)
    per = 32 // bits if bits in (4, 8) else 8
    last = case.get("packed_last", D // per)
    pk = torch.zeros((1, H_kv, 4, last), dtype=torch.uint32)
    s = torch.zeros((1, H_kv, 4, 1), dtype=torch.float16)
    with pytest.raises(ValueError, match=case["match"]):
        mq.quantized_sdpa(q, pk, pk, s, s, s, s, bits=bits, group_size=32)


def test_kernels_refuse_cpu_tensors():
    q = torch.zeros((1, 2, 1, 128), dtype=torch.float16)
    pk = torch.zeros((1, 2, 4, 16), dtype=torch.uint32)
    s = torch.zeros((1, 2, 4, 4), dtype=torch.float16)
    with pytest.raises(RuntimeError, match="ROCm GPU only"):
        mq.quantized_sdpa(q, pk, pk, s, s, s, s, bits=4, group_size=32)


def test_metric_known_answers():
    for key in ("bytes_fp16", "bytes_quantized"):
        g = REF[key]
        assert metric.compute_bytes(**g["args"]) == (g["read"], g["write"])
        assert ometric.compute_bytes(**g["args"]) == (g["read"], g["write"])
    g = REF["bandwidth"]
    assert abs(metric.compute_bandwidth_gbps(g["total_bytes"], g["median_us"]) - g["gbps"]) < 0.01
    # headline config: GQA-16, D=256, 4-bit gs=32, N=128K
    r, w = metric.compute_bytes(1, 32, 2, 131072, 256, 1, "quantized", 4, 32)
    assert r + w == 83_918_848
    assert metric.decode_bytes(1, 32, 2, 256, 4, 32, 131072) == 83_918_848


# ---- stream-K schedule of a left-padded batch (device code in csrc/common.h) ----
def _streamk_segments(T, U):
    """Integer rules of the schedule (streamk_total / streamk_find /
    streamk_write_sched and the kernel's segment loop): unit u owns global
    tiles [u*C, (u+1)*C) of the sequences laid end to end; its part in
    sequence b is a segment at partial column u + b."""
    total = sum(T)
    C = max(1, -(-total // U))
    P = np.concatenate([[0], np.cumsum(T)[:-1]]).astype(int)
    segs = []
    for u in range(U):
        g, g_end = u * C, min((u + 1) * C, total)
        for b, (p, t) in enumerate(zip(P, T)):
            lo, hi = max(g, p), min(g_end, p + t)
            if hi > lo:
                segs.append((u, b, lo - p, hi - p, u + b))
    sched = [((p // C) + b, (p + t - 1) // C - p // C + 1) if t > 0 else (0, 0)
             for b, (p, t) in enumerate(zip(P, T))]
    return C, segs, sched


@pytest.mark.parametrize("seed", range(20))
def test_streamk_schedule_invariants(seed):
    r = np.random.default_rng(seed)
    B = int(r.integers(2, 80))
    T = [int(x) for x in r.integers(0, 300, size=B)]
    T[int(r.integers(B))] = 0                       # an empty sequence
    U = B * int(r.integers(1, 5))
    C, segs, sched = _streamk_segments(T, U)
    cols = [s[4] for s in segs]
    assert len(cols) == len(set(cols))              # one partial slot per segment
    assert max(cols, default=0) < U + B             # within the U + B columns of a row
    per_unit = {}
    for u, b, lo, hi, _ in segs:
        per_unit[u] = per_unit.get(u, 0) + hi - lo
    assert max(per_unit.values(), default=0) <= C   # equal work: at most C tiles a unit
    for b, t in enumerate(T):                       # every tile exactly once, columns consecutive
        mine = sorted((lo, hi, col) for u, bb, lo, hi, col in segs if bb == b)
        assert sum(hi - lo for lo, hi, _ in mine) == t
        assert all(mine[i][1] == mine[i + 1][0] for i in range(len(mine) - 1))
        first, count = sched[b]
        assert [c for _, _, c in mine] == list(range(first, first + count))


# ---- DecodePlan: how far set_keys may move N --------------------------------
def test_plan_capacity_checks():
    """A plan's capacity may not exceed any buffer's storage (set_keys would
    send the kernel past it) nor go with a mask sized for fewer keys (the
    kernel would read the mask past its end).  Checked before any device use."""
    from mlx_qsdpa_amd import kernels

    B, Hkv, cap, n0, D, bits, gs = 2, 2, 64, 40, 128, 4, 32
    W, G = D * bits // 32, D // gs
    full = [torch.zeros((B, Hkv, cap, w), dtype=dt) for w, dt in
            ((W, torch.uint32), (W, torch.uint32), (G, torch.float16), (G, torch.float16),
             (G, torch.float16), (G, torch.float16))]
    views = [t[:, :, :n0] for t in full]
    assert [kernels._rows_in_storage(v) for v in views] == [cap] * 6
    # the last head's rows end where the storage ends
    assert kernels._rows_in_storage(full[0][:, 1:, :n0]) == cap
    q = torch.zeros((B, 8, 1, D), dtype=torch.float16)
    args = dict(scale=1.0, bits=bits, group_size=gs)
    with pytest.raises(ValueError, match="storage holds 64 rows"):
        kernels.DecodePlan(q, *views[:2], views[2], views[3], views[4], views[5], capacity=cap + 1, **args)
    with pytest.raises(ValueError, match="mask"):
        kernels.DecodePlan(q, *views[:2], views[2], views[3], views[4], views[5], capacity=cap,
                           mask=torch.ones((B, 1, 1, n0), dtype=torch.bool), **args)
    with pytest.raises(ValueError, match="below"):
        kernels.DecodePlan(q, *views[:2], views[2], views[3], views[4], views[5], capacity=n0 - 1, **args)
    # within capacity the plan reaches the device check (these are CPU tensors)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        kernels.DecodePlan(q, *views[:2], views[2], views[3], views[4], views[5], capacity=cap, **args)
