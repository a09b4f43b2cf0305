"""A logical model of a rotating quantized window, for invariant tests.

The model keeps the cache's tokens as a list in temporal order (per batch
and head), each with its current quantized form, and knows nothing about
ring pointers, write positions, rotations or buffer slots.  The rules are
the observable behaviour of the reference's rotating caches
(mlx_qsdpa/cache.py:574-591 decode, 593-620 prefill, 662-678 state) with
the first ``keep`` tokens held as attention sinks:

* one new token (decode): quantize it, append it; when the window holds
  more than ``max_size`` tokens, drop the oldest token after the sinks
  (with keep = 0: the oldest token);
* several new tokens (prefill): dequantize the window, append the new
  tokens, keep the first ``keep`` and the newest ``max_size - keep`` when
  the total exceeds ``max_size``, and quantize the result again.

It uses only the affine quantizer / dequantizer of the oracle, which the
known-answer fixtures pin (tests/golden/affine_known_answers.json).  A cache
whose ring arithmetic overwrites a sink, wraps onto the wrong slot, or
returns its state out of temporal order disagrees with this model.
"""

from __future__ import annotations

import numpy as np

from oracle import affine


def _cat(a, b):
    return tuple(np.concatenate([x, y], axis=2) for x, y in zip(a, b))


def _take(t, idx):
    return tuple(x[:, :, idx] for x in t)


class WindowModel:
    """Tokens of a rotating window in temporal order, quantized as the cache holds them."""

    def __init__(self, max_size: int, keep: int, bits: int, group_size: int, dtype: str):
        self.max_size, self.keep = max_size, keep
        self.bits, self.gs, self.dtype = bits, group_size, dtype
        self.k = None  # (packed, scales, biases), each [B, H, n, .]
        self.v = None
        self.raw_first = None  # the first `keep` raw key tokens, as appended

    def __len__(self):
        return 0 if self.k is None else self.k[0].shape[2]

    def _quant(self, x):
        return affine.quantize(x, self.gs, self.bits, self.dtype)

    def _deq(self, t):
        return affine.dequantize(*t, self.gs, self.bits, self.dtype)

    def update(self, k_raw: np.ndarray, v_raw: np.ndarray) -> None:
        S = k_raw.shape[2]
        if self.raw_first is None:
            self.raw_first = k_raw[:, :, : self.keep]
        elif self.raw_first.shape[2] < self.keep:
            self.raw_first = np.concatenate([self.raw_first, k_raw], axis=2)[:, :, : self.keep]
        if S == 1:
            qk, qv = self._quant(k_raw), self._quant(v_raw)
            self.k = qk if self.k is None else _cat(self.k, qk)
            self.v = qv if self.v is None else _cat(self.v, qv)
            n = len(self)
            if n > self.max_size:
                idx = [i for i in range(n) if i != self.keep]  # drop the oldest non-sink
                self.k, self.v = _take(self.k, idx), _take(self.v, idx)
            return
        ak, av = k_raw, v_raw
        if self.k is not None:
            ak = np.concatenate([self._deq(self.k), k_raw], axis=2)
            av = np.concatenate([self._deq(self.v), v_raw], axis=2)
        total = ak.shape[2]
        if total > self.max_size:
            tail = self.max_size - self.keep
            idx = list(range(self.keep)) + list(range(total - tail, total))
            ak, av = ak[:, :, idx], av[:, :, idx]
        self.k, self.v = self._quant(ak), self._quant(av)


def rows_bits(t, dtype):
    """One byte string per (batch, head, token) row: packed words + scale / bias bits."""
    p, s, b = t
    pb = np.ascontiguousarray(p).view(np.uint8).reshape(*p.shape[:3], p.shape[3] * 4)
    sb = np.ascontiguousarray(affine.T_bits(s, dtype).astype(np.uint16)).view(np.uint8)
    bb = np.ascontiguousarray(affine.T_bits(b, dtype).astype(np.uint16)).view(np.uint8)
    sb = sb.reshape(*s.shape[:3], s.shape[3] * 2)
    bb = bb.reshape(*b.shape[:3], b.shape[3] * 2)
    return np.concatenate([pb, sb, bb], axis=-1)


def assert_same_rows(got, want, dtype, ctx):
    """Bit-exact equality of two (packed, scales, biases) triples in the same order."""
    g, w = rows_bits(got, dtype), rows_bits(want, dtype)
    assert g.shape == w.shape, f"{ctx}: shape {g.shape} vs {w.shape}"
    bad = np.argwhere(~np.all(g == w, axis=-1))
    assert bad.size == 0, f"{ctx}: {len(bad)} rows differ, first (b, h, t) = {tuple(bad[0])}"


def assert_same_multiset(got, want, dtype, ctx):
    """The same rows per (batch, head) in any order (a ring holds the window rotated)."""
    g, w = rows_bits(got, dtype), rows_bits(want, dtype)
    assert g.shape == w.shape, f"{ctx}: shape {g.shape} vs {w.shape}"
    for bi in range(g.shape[0]):
        for hi in range(g.shape[1]):
            gs = sorted(map(bytes, g[bi, hi]))
            ws = sorted(map(bytes, w[bi, hi]))
            assert gs == ws, f"{ctx}: rows of (b={bi}, h={hi}) differ as a set"


def random_chunks(rng: np.random.Generator, max_size: int, total: int, prefill_every: int = 7):
    """Chunk lengths summing to at least `total`: mostly single tokens, with
    prefill chunks from 2 to max_size + 3 tokens now and then."""
    out, n = [], 0
    while n < total:
        if len(out) % prefill_every == prefill_every - 1:
            S = int(rng.integers(2, max_size + 4))
        else:
            S = 1
        out.append(S)
        n += S
    return out
