"""Batch administration scenarios: the shipped caches against the oracle's.

Each scenario builds the same caches twice -- the shipped torch caches
(mlx_qsdpa_amd.cache, on the GPU or on CPU with conftest.cpu_kernels) and
the oracle's numpy caches (oracle/caches.py) -- from the same seeded
tokens, runs an administration step (finalize, filter, extend, extract,
merge) and then keeps updating both.  After every step the two must agree
bit-exactly on every buffer (packed words, scale and bias bits, over the
whole capacity), on offset / left_padding / _idx and on the views an update
returns.

On a GPU, every administration call and every update runs under
torch.cuda.set_sync_debug_mode("error"): a host read of device memory or a
blocking copy there fails the scenario.  Token inputs are uploaded before.

Independent of either implementation, ``check_sequences`` pins the admin
semantics: after each step every sequence's ``extract`` (its tokens in
temporal order) must equal the tokens that sequence had before the step.
"""

from __future__ import annotations

import contextlib

import numpy as np
import torch

from conftest import from_np, to_np, torch_dtype
from oracle import affine
from oracle import caches as oc
from window_model import assert_same_rows

import mlx_qsdpa_amd.cache as pc

H, D = 2, 64


@contextlib.contextmanager
def no_sync(device):
    """Host reads of device memory and blocking copies raise inside."""
    if device is None or torch.device(device).type != "cuda":
        yield
        return
    torch.cuda.synchronize()
    torch.cuda.set_sync_debug_mode("error")
    try:
        yield
    finally:
        torch.cuda.set_sync_debug_mode("default")


def _np3(t):
    return tuple(to_np(x) for x in t)


class Pair:
    """A shipped cache and an oracle cache fed the same tokens."""

    def __init__(self, prod, orc, dtype, device, rng):
        self.p, self.o, self.dtype, self.device, self.rng = prod, orc, dtype, device, rng

    def tokens(self, B, S):
        k = affine.random_T(self.rng, (B, H, S, D), self.dtype, outlier_frac=0.02)
        v = affine.random_T(self.rng, (B, H, S, D), self.dtype)
        tdt = torch_dtype(self.dtype)
        return k, v, from_np(k, tdt, self.device), from_np(v, tdt, self.device)

    def update(self, B, S, ctx):
        k, v, tk, tv = self.tokens(B, S)
        with no_sync(self.device):
            pk, pv = self.p.update_and_fetch(tk, tv)
        ok, ov = self.o.update_and_fetch(k, v)
        assert_same_rows(_np3(pk), ok, self.dtype, ctx + ": returned keys")
        assert_same_rows(_np3(pv), ov, self.dtype, ctx + ": returned values")
        self.check(ctx)

    def check(self, ctx):
        same_cache(self.p, self.o, self.dtype, ctx)


def same_cache(p, o, dtype, ctx):
    """Buffers (whole capacity) and counters of a shipped and an oracle cache."""
    assert (p._keys is None) == (o._keys is None), f"{ctx}: one cache has no buffers"
    for name in ("offset", "left_padding"):
        if hasattr(o, name):
            pv, ov = getattr(p, name), getattr(o, name)
            pv = pv.tolist() if isinstance(pv, torch.Tensor) else pv
            ov = ov.tolist() if isinstance(ov, np.ndarray) else ov
            assert pv == ov, f"{ctx}: {name} {pv} vs {ov}"
    if hasattr(o, "_idx"):
        assert p._idx == o._idx, f"{ctx}: _idx {p._idx} vs {o._idx}"
    if p._keys is None:
        return
    assert p._keys[0].shape == o._keys[0].shape, f"{ctx}: buffer {tuple(p._keys[0].shape)} vs {o._keys[0].shape}"
    assert_same_rows(_np3(p._keys), o._keys, dtype, ctx + ": key buffers")
    assert_same_rows(_np3(p._values), o._values, dtype, ctx + ": value buffers")


def sequences(cache):
    """Every sequence's (keys, values) in temporal order via extract()."""
    out = []
    for i in range(len(cache.offset)):
        e = cache.extract(i)
        if e._keys is None:
            out.append(None)
            continue
        k, v = e.state
        if isinstance(k[0], torch.Tensor):
            k, v = _np3(k), _np3(v)
        out.append((k, v))
    return out


def check_sequences(got, want, dtype, ctx):
    assert len(got) == len(want), f"{ctx}: {len(got)} sequences vs {len(want)}"
    for i, (g, w) in enumerate(zip(got, want)):
        if w is None or (w[0][0].shape[2] == 0):
            assert g is None or g[0][0].shape[2] == 0, f"{ctx}: sequence {i} should be empty"
            continue
        assert g is not None, f"{ctx}: sequence {i} lost its tokens"
        assert_same_rows(g[0], w[0], dtype, f"{ctx}: sequence {i} keys")
        assert_same_rows(g[1], w[1], dtype, f"{ctx}: sequence {i} values")


# ---------------------------------------------------------------------------
# BatchQuantizedSDPACache
# ---------------------------------------------------------------------------
def _batch(lp, bits, gs, dtype, device, rng):
    return Pair(pc.BatchQuantizedSDPACache(lp, bits=bits, group_size=gs),
                oc.BatchQuantizedSDPACache(lp, bits=bits, group_size=gs, dtype=dtype), dtype, device, rng)


def batch_scenario(name, bits=4, gs=32, dtype="f16", device=None, seed=0):
    rng = np.random.default_rng(seed)
    if name == "finalize":
        for S in (7, 256):  # 256 fills the capacity: the roll wraps the padding tokens round
            x = _batch([0, 1, 0], bits, gs, dtype, device, rng)
            with no_sync(device):
                x.p.prepare(right_padding=[2, 0, 3])
            x.o.prepare(right_padding=[2, 0, 3])
            x.update(3, S, f"prefill {S}")
            with no_sync(device):
                x.p.finalize()
            x.o.finalize()
            x.check(f"finalize after {S}")
            for i in range(3):
                x.update(3, 1, f"decode {i} after finalize")
    elif name == "filter":
        x = _batch([3, 0, 5, 2], bits, gs, dtype, device, rng)
        x.update(4, 6, "prefill")
        x.update(4, 1, "decode")
        x.p.trim(1)
        x.o.trim(1)  # a trimmed column stays in the buffer past _idx
        before = sequences(x.o)
        for idx in ([2, 0], torch.tensor([1, 1]), [-1]):
            with no_sync(device):
                x.p.filter(idx)
            x.o.filter(np.asarray(idx))
            x.check(f"filter {idx}")
            sel = [before[int(i)] for i in np.asarray(idx).reshape(-1)]
            check_sequences(sequences(x.p), sel, dtype, f"filter {idx}")
            before = sequences(x.o)
            x.update(len(x.o.offset), 1, f"decode after filter {idx}")
            before = sequences(x.o)
    elif name == "extend":
        for swap in (False, True):
            a = _batch([0, 2], bits, gs, dtype, device, rng)
            a.update(2, 5, "a prefill")
            b = _batch([1], bits, gs, dtype, device, rng)
            b.update(1, 300, "b prefill")  # capacity 512 against a's 256
            b.update(1, 1, "b decode")
            x, y = (b, a) if swap else (a, b)
            want = sequences(x.o) + sequences(y.o)
            with no_sync(device):
                x.p.extend(y.p)
            x.o.extend(y.o)
            x.check(f"extend (swap={swap})")
            check_sequences(sequences(x.p), want, dtype, f"extend (swap={swap})")
            for i in range(2):
                x.update(3, 1, f"decode {i} after extend")
            x.update(3, 4, "chunk after extend")
        # a side without buffers contributes zero rows
        a = _batch([0, 1], bits, gs, dtype, device, rng)
        a.update(2, 9, "a prefill")
        e = _batch([0], bits, gs, dtype, device, rng)
        with no_sync(device):
            a.p.extend(e.p)
        a.o.extend(e.o)
        a.check("extend by an empty batch")
        a.update(3, 2, "chunk after extend by an empty batch")
    elif name == "extract":
        x = _batch([4, 0, 1], bits, gs, dtype, device, rng)
        x.update(3, 10, "prefill")
        x.update(3, 1, "decode")
        for i in (0, 1, 2, -1):
            with no_sync(device):
                pe = x.p.extract(i)
            oe = x.o.extract(i)
            s = Pair(pe, oe, dtype, device, rng)
            s.check(f"extract {i}")
            s.update(1, 1, f"decode after extract {i}")
            s.update(1, 3, f"chunk after extract {i}")
    elif name == "merge":
        singles = []
        for n in (4, 2, 0, 300, 1):
            s = Pair(pc.QuantizedSDPACache(bits=bits, group_size=gs),
                     oc.QuantizedSDPACache(bits=bits, group_size=gs, dtype=dtype), dtype, device, rng)
            if n:
                s.update(1, n, f"single {n}")
            singles.append(s)
        with no_sync(device):
            pb = pc.BatchQuantizedSDPACache.merge([s.p for s in singles])
        ob = oc.BatchQuantizedSDPACache.merge([s.o for s in singles])
        x = Pair(pb, ob, dtype, device, rng)
        x.check("merge")
        want = [(s.o.state if s.o._keys is not None else None) for s in singles]
        check_sequences(sequences(x.p), want, dtype, "merge")
        x.update(5, 1, "decode after merge")
        x.update(5, 2, "chunk after merge")
    else:
        raise ValueError(name)


BATCH_SCENARIOS = ["finalize", "filter", "extend", "extract", "merge"]


# ---------------------------------------------------------------------------
# BatchQuantizedRotatingSDPACache
# ---------------------------------------------------------------------------
def _rot_batch(lp, max_size, keep, bits, gs, dtype, device, rng):
    return Pair(pc.BatchQuantizedRotatingSDPACache(lp, max_size, keep=keep, bits=bits, group_size=gs),
                oc.BatchQuantizedRotatingSDPACache(lp, max_size, keep=keep, bits=bits, group_size=gs,
                                                   dtype=dtype), dtype, device, rng)


def _rot_single(max_size, keep, bits, gs, dtype, device, rng):
    return Pair(pc.QuantizedRotatingSDPACache(max_size, keep=keep, bits=bits, group_size=gs),
                oc.QuantizedRotatingSDPACache(max_size, keep=keep, bits=bits, group_size=gs, dtype=dtype),
                dtype, device, rng)


def _feed(x, B, chunks, ctx):
    for i, S in enumerate(chunks):
        x.update(B, S, f"{ctx} update {i} (S={S})")


def rotating_scenario(name, max_size=8, keep=0, bits=4, gs=32, dtype="f16", device=None, seed=0):
    rng = np.random.default_rng(seed)
    W = max_size
    if name == "filter":
        x = _rot_batch([0, 0, 0], W, keep, bits, gs, dtype, device, rng)
        _feed(x, 3, [3] + [1] * (W + 3), "fill past the wrap")
        before = sequences(x.o)
        with no_sync(device):
            x.p.filter([2, 0])
        x.o.filter([2, 0])
        x.check("filter")
        check_sequences(sequences(x.p), [before[2], before[0]], dtype, "filter")
        _feed(x, 2, [1, 1, 3, 1], "after filter")
    elif name == "extend":
        # (first side's chunks, second side's chunks): unwrapped with equal
        # and unequal fill, one side wrapped, both wrapped at different ring
        # positions, a prefill longer than the window.
        plans = [([5], [5]), ([5], [2, 1]), ([3] + [1] * (W + 2), [4]), ([1] * (W + 3), [2] + [1] * (W + 5)),
                 ([W + 5], [1, 1])]
        for pa, pb in plans:
            ctx = f"extend {pa} + {pb}"
            a = _rot_batch([0, 0], W, keep, bits, gs, dtype, device, rng)
            b = _rot_batch([0], W, keep, bits, gs, dtype, device, rng)
            _feed(a, 2, pa, ctx + " a")
            _feed(b, 1, pb, ctx + " b")
            want = sequences(a.o) + sequences(b.o)
            with no_sync(device):
                a.p.extend(b.p)
            a.o.extend(b.o)
            a.check(ctx)
            check_sequences(sequences(a.p), want, dtype, ctx)
            check_sequences(sequences(a.o), want, dtype, ctx + " (oracle)")
            _feed(a, 3, [1] * (W + 2) + [3, 1], ctx + " then")
        e = _rot_batch([0], W, keep, bits, gs, dtype, device, rng)
        a = _rot_batch([0, 0], W, keep, bits, gs, dtype, device, rng)
        _feed(a, 2, [4, 1], "a")
        with no_sync(device):
            e.p.extend(a.p)
        e.o.extend(a.o)
        e.check("empty batch extended")
        _feed(e, 3, [1, 1, 2], "after extending an empty batch")
    elif name == "extract":
        x = _rot_batch([2, 0], W, keep, bits, gs, dtype, device, rng)
        for step, S in enumerate([3, 1, 1] + [1] * (W + 1) + [3, 1]):
            x.update(2, S, f"update {step}")
            for i in (0, 1):
                with no_sync(device):
                    pe = x.p.extract(i)
                oe = x.o.extract(i)
                same_cache(pe, oe, dtype, f"extract {i} after update {step}")
        s = Pair(x.p.extract(1), x.o.extract(1), dtype, device, rng)
        _feed(s, 1, [1, 1, 2, 1], "single after extract")
    elif name == "merge":
        singles = []
        for chunks in ([1, 1, 1], [5], [], [1] * (W + 4), [W + 3, 1]):
            s = _rot_single(W, keep, bits, gs, dtype, device, rng)
            _feed(s, 1, chunks, f"single {chunks}")
            singles.append(s)
        with no_sync(device):
            pb = pc.BatchQuantizedRotatingSDPACache.merge([s.p for s in singles])
        ob = oc.BatchQuantizedRotatingSDPACache.merge([s.o for s in singles])
        x = Pair(pb, ob, dtype, device, rng)
        x.check("merge")
        want = [(s.o.state if s.o._keys is not None else None) for s in singles]
        check_sequences(sequences(x.p), want, dtype, "merge")
        _feed(x, 5, [1] * (W + 2) + [2, 1], "after merge")
    else:
        raise ValueError(name)


ROTATING_SCENARIOS = ["filter", "extend", "extract", "merge"]
