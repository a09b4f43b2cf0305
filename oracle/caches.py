"""The four quantized KV caches of mlx_qsdpa/cache.py, restated in numpy.

TEST INFRASTRUCTURE.  Each buffer is a 3-tuple (packed uint32, scales,
biases) with scales/biases T-valued float32 (see affine.py).  Index logic
follows the reference line by line; the citations are on each method.

Extension (the reference asserts keep == 0 at cache.py:512, 732):
``keep > 0`` keeps the first ``keep`` slots as attention sinks.  Ring
writes then cycle over [keep, max_size): the slot after the last one is
``keep`` instead of 0, temporal order is
[0:keep] + [ring pointer:max_size] + [keep:ring pointer], and a prefill that
overflows the window keeps the first ``keep`` and the newest
``max_size - keep`` tokens.  With keep == 0 every rule reduces to the
reference's.

Masks after the ring wraps (the reference's mask width
min(offset, max_size) + N disagrees with the returned key length there,
cache.py:636-644 vs 588-591): ``make_mask`` below reproduces the reference
exactly while offset + N <= max_size and otherwise returns the lower-right
aligned causal mask over the returned window.

Both extensions are pinned by tests/test_cache_invariants.py: a logical
window model (tests/window_model.py, temporal order only, no ring
arithmetic) must agree with these caches after every update of random
decode / prefill sequences across several wraps, and a mask taken before an
update must be lower-right causal over exactly the keys it returns.
"""

from __future__ import annotations

import numpy as np

from . import affine
from .attention import create_causal_mask


def _zeros_q(shape3, dim, bits, gs):
    per = 32 // bits
    return (np.zeros((*shape3, dim // per), np.uint32),
            np.zeros((*shape3, dim // gs), np.float32),
            np.zeros((*shape3, dim // gs), np.float32))


def _cat(a, b, axis=2):
    return tuple(np.concatenate([x, y], axis=axis) for x, y in zip(a, b))


def _sl(tup, start, stop):
    return tuple(t[:, :, start:stop, :] for t in tup)


def _dynamic_roll(x, shifts, axis):
    """cache.py:46-51."""
    n = x.shape[axis]
    idx = (np.arange(n)[None, :] - shifts[:, None]) % n            # (B, n)
    idx = idx[:, None, :, None]
    idx = np.broadcast_to(idx, (x.shape[0], x.shape[1], n, x.shape[3]))
    return np.take_along_axis(x, idx, axis=axis)


def _from_end(idx, B):
    """Extension: a negative sequence index counts from the end (the
    reference's slice [idx:idx + 1] is empty for idx = -1)."""
    idx = int(idx)
    if not -B <= idx < B:
        raise IndexError(idx)
    return idx % B


def _ring_temporal(t, keep, ptr, n_visible):
    """[0:keep] + [ptr:n_visible] + [keep:ptr]  (identity when ptr <= keep)."""
    if ptr <= keep or ptr >= n_visible:
        return t[:, :, :n_visible]
    return np.concatenate([t[:, :, :keep], t[:, :, ptr:n_visible], t[:, :, keep:ptr]],
                          axis=2)


class QuantizedSDPACache:
    """cache.py:54-231."""

    def __init__(self, bits=4, group_size=32, step=256, dtype="f16"):
        if bits not in (4, 8):
            raise ValueError(f"bits must be 4 or 8, got {bits}")
        self.bits, self.group_size, self.step, self.dtype = bits, group_size, step, dtype
        self.offset = 0
        self._keys = None
        self._values = None

    def empty(self):
        return self._keys is None

    @property
    def nbytes(self):                                               # cache.py:87-96
        if self._keys is None:
            return 0
        tot = 0
        for tup in (self._keys, self._values):
            for i, t in enumerate(tup):
                tot += t.size * (4 if i == 0 else 2)
        return tot

    def size(self):
        return self.offset

    def trim(self, n):                                              # cache.py:104-108
        n = min(self.offset, n)
        self.offset -= n
        return n

    def update_and_fetch(self, keys, values):                       # cache.py:163-197
        B, H, S, Dk = keys.shape
        Dv = values.shape[-1]
        prev = self.offset
        if self._keys is None or prev + S > self._keys[0].shape[2]:
            self._grow(B, H, S, Dk, Dv, prev)
        self.offset += S
        nk = affine.quantize(keys, self.group_size, self.bits, self.dtype)
        nv = affine.quantize(values, self.group_size, self.bits, self.dtype)
        for i in range(3):
            self._keys[i][:, :, prev:self.offset] = nk[i]
            self._values[i][:, :, prev:self.offset] = nv[i]
        return _sl(self._keys, 0, self.offset), _sl(self._values, 0, self.offset)

    def _grow(self, B, H, S, Dk, Dv, prev):                         # cache.py:199-231
        new_alloc = ((self.step + S - 1) // self.step) * self.step
        shape = (B, H, new_alloc)
        nk = _zeros_q(shape, Dk, self.bits, self.group_size)
        nv = _zeros_q(shape, Dv, self.bits, self.group_size)
        if self._keys is not None:
            if prev % self.step != 0:
                self._keys = _sl(self._keys, 0, prev)
                self._values = _sl(self._values, 0, prev)
            self._keys = _cat(self._keys, nk)
            self._values = _cat(self._values, nv)
        else:
            self._keys, self._values = nk, nv

    def make_mask(self, N, return_array=False, window_size=None):   # cache.py:116-125
        if window_size is not None:
            return create_causal_mask(N, self.offset, window_size=window_size)
        if N == 1:
            return None
        if return_array:
            return create_causal_mask(N, self.offset)
        return "causal"

    @property
    def state(self):                                                # cache.py:127-134
        if self._keys is None:
            return None, None
        return _sl(self._keys, 0, self.offset), _sl(self._values, 0, self.offset)


class BatchQuantizedSDPACache:
    """cache.py:234-492."""

    step = 256

    def __init__(self, left_padding, bits=4, group_size=32, dtype="f16"):
        self.bits, self.group_size, self.dtype = bits, group_size, dtype
        self.left_padding = np.array(left_padding, dtype=np.int64)
        self.offset = -self.left_padding.copy()
        self._idx = 0
        self._keys = None
        self._values = None
        self._right_padding = None

    def empty(self):
        return self._keys is None

    def size(self):
        return self._idx

    def trim(self, n):                                              # cache.py:273-277
        n = min(self._idx, n)
        self._idx -= n
        self.offset = self.offset - n
        return n

    def update_and_fetch(self, keys, values):                       # cache.py:279-322
        B, H, S, Dk = keys.shape
        Dv = values.shape[-1]
        prev = self._idx
        if self._keys is None or prev + S > self._keys[0].shape[2]:
            new_alloc = ((self.step + S - 1) // self.step) * self.step
            shape = (B, H, new_alloc)
            nk = _zeros_q(shape, Dk, self.bits, self.group_size)
            nv = _zeros_q(shape, Dv, self.bits, self.group_size)
            if self._keys is not None:
                if prev % self.step != 0:
                    self._keys = _sl(self._keys, 0, prev)
                    self._values = _sl(self._values, 0, prev)
                self._keys = _cat(self._keys, nk)
                self._values = _cat(self._values, nv)
            else:
                self._keys, self._values = nk, nv
        self.offset = self.offset + S
        self._idx += S
        qk = affine.quantize(keys, self.group_size, self.bits, self.dtype)
        qv = affine.quantize(values, self.group_size, self.bits, self.dtype)
        for i in range(3):
            self._keys[i][:, :, prev:self._idx] = qk[i]
            self._values[i][:, :, prev:self._idx] = qv[i]
        return _sl(self._keys, 0, self._idx), _sl(self._values, 0, self._idx)

    def prepare(self, *, left_padding=None, lengths=None, right_padding=None):
        if left_padding is not None:                                # cache.py:325-332
            if self._keys is not None:
                raise ValueError(
                    "Left padding can only be added to an empty BatchQuantizedSDPACache")
            lp = np.asarray(left_padding, dtype=np.int64)
            self.left_padding = self.left_padding + lp
            self.offset = self.offset - lp
        if right_padding is not None and max(right_padding) > 0:
            self._right_padding = np.asarray(right_padding, dtype=np.int64)

    def finalize(self):                                             # cache.py:337-348
        if self._right_padding is not None:
            pad = self._right_padding
            self._keys = tuple(_dynamic_roll(t, pad, 2) for t in self._keys)
            self._values = tuple(_dynamic_roll(t, pad, 2) for t in self._values)
            self.offset = self.offset - pad
            self.left_padding = self.left_padding + pad
            self._right_padding = None

    @property
    def state(self):                                                # cache.py:350-359
        if self._keys is None:
            return None, None, self.offset, self.left_padding
        k, v = self._keys, self._values
        if self._idx < k[0].shape[2]:
            k = _sl(k, 0, self._idx)
            v = _sl(v, 0, self._idx)
        return k, v, self.offset, self.left_padding

    def make_mask(self, N, return_array=False, **kw):               # cache.py:369-376
        return create_causal_mask(N, offset=self.offset, left_padding=self.left_padding,
                                  window_size=kw.get("window_size"))

    def filter(self, batch_indices):                                # cache.py:378-391
        bi = np.asarray(batch_indices, dtype=np.int64).reshape(-1)
        self.offset = self.offset[bi]
        self.left_padding = self.left_padding[bi]
        if self._keys is None:      # (the reference would trim a None buffer)
            return
        self._keys = tuple(t[bi] for t in self._keys)
        self._values = tuple(t[bi] for t in self._values)
        min_pad = int(self.left_padding.min()) if bi.size else 0
        if min_pad > 0:
            self._keys = tuple(t[:, :, min_pad:] for t in self._keys)
            self._values = tuple(t[:, :, min_pad:] for t in self._values)
            self._idx -= min_pad
            self.left_padding = self.left_padding - min_pad

    def extend(self, other):                                        # cache.py:393-427
        """Other's rows after this batch's; both sides padded on the left by
        max(_idx) - own _idx and on the right to the larger capacity (cut
        when the left pad pushes columns past it).  Extension: a side
        without buffers contributes zero rows (the reference needs both)."""
        top = max(self._idx, other._idx)
        sides = (self, other)
        filled = [c for c in sides if c._keys is not None]
        if filled:
            cap = max(c._keys[0].shape[2] for c in filled)
            like = filled[0]

            def placed(c, tup, like_tup):
                left = top - c._idx
                out = []
                for j, ref in enumerate(like_tup):
                    B = c.offset.shape[0]
                    z = np.zeros((B, ref.shape[1], cap, ref.shape[3]), ref.dtype)
                    if tup is not None:
                        t = tup[j]
                        n = min(t.shape[2], cap - left)
                        z[:, :, left:left + n] = t[:, :, :n]
                    out.append(z)
                return out

            ks = [placed(c, c._keys, like._keys) for c in sides]
            vs = [placed(c, c._values, like._values) for c in sides]
            self._keys = tuple(np.concatenate([a, b], axis=0) for a, b in zip(*ks))
            self._values = tuple(np.concatenate([a, b], axis=0) for a, b in zip(*vs))
        self.offset = np.concatenate([self.offset, other.offset])
        self.left_padding = np.concatenate([self.left_padding + (top - self._idx),
                                            other.left_padding + (top - other._idx)])
        self._idx = top

    def extract(self, idx):                                         # cache.py:429-444
        c = QuantizedSDPACache(bits=self.bits, group_size=self.group_size, dtype=self.dtype)
        if self._keys is None:
            return c
        idx = _from_end(idx, self.offset.shape[0])
        pad = int(self.left_padding[idx])
        c._keys = tuple(t[idx:idx + 1, :, pad:self._idx].copy() for t in self._keys)
        c._values = tuple(t[idx:idx + 1, :, pad:self._idx].copy() for t in self._values)
        c.offset = self._idx - pad
        return c

    @classmethod
    def merge(cls, caches):                                         # cache.py:446-492
        if not caches:
            return cls([0])
        bits, gs, dtype = caches[0].bits, caches[0].group_size, caches[0].dtype
        lengths = [c.offset for c in caches]
        max_len = max(lengths)
        padding = [max_len - l for l in lengths]
        batch = cls(padding, bits=bits, group_size=gs, dtype=dtype)
        if all(c.empty() for c in caches):
            return batch
        B = len(caches)
        ref = next(c for c in caches if not c.empty())
        H = ref._keys[0].shape[1]

        def alloc(tup):
            return tuple(np.zeros((B, H, max_len, t.shape[3]), t.dtype) for t in tup)

        batch._keys = alloc(ref._keys)
        batch._values = alloc(ref._values)
        for i, (p, c) in enumerate(zip(padding, caches)):
            if c.empty():
                continue
            for j in range(3):
                batch._keys[j][i:i + 1, :, p:p + c.offset] = c._keys[j][:, :, :c.offset]
                batch._values[j][i:i + 1, :, p:p + c.offset] = c._values[j][:, :, :c.offset]
        batch.offset = batch.offset + max_len
        batch._idx = max_len
        return batch


class QuantizedRotatingSDPACache:
    """cache.py:495-711, with the keep > 0 extension described above."""

    def __init__(self, max_size, keep=0, bits=4, group_size=32, dtype="f16"):
        if bits not in (4, 8):
            raise ValueError(f"bits must be 4 or 8, got {bits}")
        if not 0 <= keep < max_size:
            raise ValueError("keep must satisfy 0 <= keep < max_size")
        self.max_size, self.keep = max_size, keep
        self.bits, self.group_size, self.dtype = bits, group_size, dtype
        self.offset = 0
        self._idx = 0
        self._keys = None
        self._values = None

    def empty(self):
        return self._keys is None

    def size(self):
        return min(self.offset, self.max_size)

    def is_trimmable(self):
        return self.offset < self.max_size

    def update_and_fetch(self, keys, values):                       # cache.py:554-572
        B, H, S, Dk = keys.shape
        if self._keys is None:
            shape = (B, H, self.max_size)
            self._keys = _zeros_q(shape, Dk, self.bits, self.group_size)
            self._values = _zeros_q(shape, values.shape[-1], self.bits, self.group_size)
        if S == 1:
            return self._update_decode(keys, values)
        return self._update_prefill(keys, values)

    def _write_pos(self):
        """Reference: _idx % max_size (cache.py:578); wraps to keep at max_size."""
        return self._idx if self._idx < self.max_size else self.keep

    def _update_decode(self, keys, values):                         # cache.py:574-591
        nk = affine.quantize(keys, self.group_size, self.bits, self.dtype)
        nv = affine.quantize(values, self.group_size, self.bits, self.dtype)
        wp = self._write_pos()
        for i in range(3):
            self._keys[i][:, :, wp:wp + 1] = nk[i]
            self._values[i][:, :, wp:wp + 1] = nv[i]
        self._idx = wp + 1
        self.offset += 1
        nv_ = min(self.offset, self.max_size)
        return _sl(self._keys, 0, nv_), _sl(self._values, 0, nv_)

    def _ring_ptr(self):
        """Oldest ring slot once wrapped (reference: _idx, cache.py:630)."""
        return self._idx

    def _dequant_temporal(self, tup):                               # cache.py:622-634
        n_visible = min(self.offset, self.max_size)
        fp = affine.dequantize(*_sl(tup, 0, n_visible), self.group_size, self.bits,
                               self.dtype)
        if self.offset > self.max_size:
            fp = _ring_temporal(fp, self.keep, self._ring_ptr(), n_visible)
        return fp

    def _update_prefill(self, keys, values):                        # cache.py:593-620
        S = keys.shape[2]
        if self.offset > 0:
            all_k = np.concatenate([self._dequant_temporal(self._keys), keys], axis=2)
            all_v = np.concatenate([self._dequant_temporal(self._values), values], axis=2)
        else:
            all_k, all_v = keys, values
        total = all_k.shape[2]
        if total > self.max_size:
            tail = self.max_size - self.keep
            all_k = np.concatenate([all_k[:, :, :self.keep], all_k[:, :, total - tail:]], 2)
            all_v = np.concatenate([all_v[:, :, :self.keep], all_v[:, :, total - tail:]], 2)
            total = self.max_size
        qk = affine.quantize(all_k, self.group_size, self.bits, self.dtype)
        qv = affine.quantize(all_v, self.group_size, self.bits, self.dtype)
        for i in range(3):
            self._keys[i][:, :, :total] = qk[i]
            self._values[i][:, :, :total] = qv[i]
        self.offset += S
        self._idx = total if total < self.max_size else self.keep   # = total % max_size at keep 0
        nv_ = min(self.offset, self.max_size)
        return _sl(self._keys, 0, nv_), _sl(self._values, 0, nv_)

    def make_mask(self, N, return_array=False, window_size=None):   # cache.py:636-644
        if N == 1:
            return None
        if return_array or window_size is not None:
            eff = min(self.offset, self.max_size)
            if self.offset + N > self.max_size:
                eff = min(self.offset + N, self.max_size) - N
            return create_causal_mask(N, eff, window_size=window_size)
        return "causal"

    def trim(self, n):                                              # cache.py:646-651
        n = min(self.offset, n)
        self.offset -= n
        self._idx -= n
        return n

    @property
    def state(self):                                                # cache.py:662-678
        if self._keys is None:
            return None, None
        n_visible = min(self.offset, self.max_size)
        if self.offset > self.max_size:
            return (tuple(_ring_temporal(t, self.keep, self._ring_ptr(), n_visible)
                          for t in self._keys),
                    tuple(_ring_temporal(t, self.keep, self._ring_ptr(), n_visible)
                          for t in self._values))
        return _sl(self._keys, 0, n_visible), _sl(self._values, 0, n_visible)


class BatchQuantizedRotatingSDPACache:
    """cache.py:714-1010, with the keep > 0 extension described above."""

    def __init__(self, left_padding, max_size, keep=0, bits=4, group_size=32, dtype="f16"):
        if not 0 <= keep < max_size:
            raise ValueError("keep must satisfy 0 <= keep < max_size")
        self.max_size, self.keep = max_size, keep
        self.bits, self.group_size, self.dtype = bits, group_size, dtype
        self.left_padding = np.array(left_padding, dtype=np.int64)
        self.offset = -self.left_padding.copy()
        self._idx = 0
        self._keys = None
        self._values = None

    def empty(self):
        return self._keys is None

    def size(self):
        return min(self._idx, self.max_size)

    def _write_pos(self):
        """Reference: _idx % max_size (cache.py:800); _idx never wraps."""
        if self._idx < self.max_size:
            return self._idx
        return self.keep + (self._idx - self.max_size) % (self.max_size - self.keep)

    def update_and_fetch(self, keys, values):                       # cache.py:764-794
        B, H, S, Dk = keys.shape
        if self._keys is None:
            shape = (B, H, self.max_size)
            self._keys = _zeros_q(shape, Dk, self.bits, self.group_size)
            self._values = _zeros_q(shape, values.shape[-1], self.bits, self.group_size)
        if S == 1:
            return self._update_decode(keys, values)
        return self._update_prefill(keys, values)

    def _update_decode(self, keys, values):                         # cache.py:796-811
        nk = affine.quantize(keys, self.group_size, self.bits, self.dtype)
        nv = affine.quantize(values, self.group_size, self.bits, self.dtype)
        wp = self._write_pos()
        for i in range(3):
            self._keys[i][:, :, wp:wp + 1] = nk[i]
            self._values[i][:, :, wp:wp + 1] = nv[i]
        self.offset = self.offset + 1
        self._idx += 1
        n = min(self._idx, self.max_size)
        return _sl(self._keys, 0, n), _sl(self._values, 0, n)

    def _ring_ptr(self):
        return self._write_pos()

    def _dequant_temporal(self, tup):                               # cache.py:842-857
        n_visible = min(self._idx, self.max_size)
        fp = affine.dequantize(*_sl(tup, 0, n_visible), self.group_size, self.bits,
                               self.dtype)
        if self._idx > self.max_size:
            fp = _ring_temporal(fp, self.keep, self._ring_ptr(), n_visible)
        return fp

    def _update_prefill(self, keys, values):                        # cache.py:813-840
        S = keys.shape[2]
        if self._idx > 0:
            all_k = np.concatenate([self._dequant_temporal(self._keys), keys], axis=2)
            all_v = np.concatenate([self._dequant_temporal(self._values), values], axis=2)
        else:
            all_k, all_v = keys, values
        total = all_k.shape[2]
        if total > self.max_size:
            tail = self.max_size - self.keep
            all_k = np.concatenate([all_k[:, :, :self.keep], all_k[:, :, total - tail:]], 2)
            all_v = np.concatenate([all_v[:, :, :self.keep], all_v[:, :, total - tail:]], 2)
            total = self.max_size
        qk = affine.quantize(all_k, self.group_size, self.bits, self.dtype)
        qv = affine.quantize(all_v, self.group_size, self.bits, self.dtype)
        for i in range(3):
            self._keys[i][:, :, :total] = qk[i]
            self._values[i][:, :, :total] = qv[i]
        self.offset = self.offset + S
        self._idx = total
        return _sl(self._keys, 0, total), _sl(self._values, 0, total)

    def make_mask(self, N, return_array=False, **kw):               # cache.py:859-866
        off = np.minimum(self.offset, self.max_size)
        if int(off.max()) + N > self.max_size:
            off = np.minimum(self.offset + N, self.max_size) - N
        return create_causal_mask(N, offset=off, left_padding=self.left_padding,
                                  window_size=kw.get("window_size"))

    def filter(self, batch_indices):                                # cache.py:868-874
        bi = np.asarray(batch_indices, dtype=np.int64).reshape(-1)
        if self._keys is not None:
            self._keys = tuple(t[bi] for t in self._keys)
            self._values = tuple(t[bi] for t in self._values)
        self.offset = self.offset[bi]
        self.left_padding = self.left_padding[bi]

    def _temporal(self, tup):
        """The visible window of every row, in temporal order."""
        n_visible = min(self._idx, self.max_size)
        res = tuple(t[:, :, :n_visible] for t in tup)
        if self._idx > self.max_size:
            res = tuple(_ring_temporal(t, self.keep, self._ring_ptr(), n_visible) for t in res)
        return res

    def extend(self, other):                                        # cache.py:876-912
        """Other's rows after this batch's.  The reference pads each side on
        the left by max(_idx) - own _idx and concatenates the buffers as
        they lie.  Extension, for every pair of batches: each side's window
        is first put in temporal order (the reference's shift of a wrapped
        ring mixes old and new tokens) and right-aligned at the longer
        window n in max_size-wide buffers (the reference's concatenation
        fails on unequal widths); _idx = n, so the ring starts unrotated.
        While neither side has wrapped, n - own visible = max(_idx) - own
        _idx: the reference's shift.  A side without buffers contributes zero
        rows (the reference keeps only the other side's)."""
        sides = (self, other)
        vis = [min(c._idx, c.max_size) if c._keys is not None else 0 for c in sides]
        n = max(vis)
        filled = [c for c in sides if c._keys is not None]
        if filled:
            like = filled[0]
            W = self.max_size

            def placed(c, v, tup, like_tup):
                out = []
                tt = c._temporal(tup) if tup is not None else None
                for j, ref in enumerate(like_tup):
                    z = np.zeros((c.offset.shape[0], ref.shape[1], W, ref.shape[3]), ref.dtype)
                    if tt is not None:
                        z[:, :, n - v:n] = tt[j]
                    out.append(z)
                return out

            ks = [placed(c, v, c._keys, like._keys) for c, v in zip(sides, vis)]
            vs = [placed(c, v, c._values, like._values) for c, v in zip(sides, vis)]
            self._keys = tuple(np.concatenate([a, b], axis=0) for a, b in zip(*ks))
            self._values = tuple(np.concatenate([a, b], axis=0) for a, b in zip(*vs))
        self.offset = np.concatenate([self.offset, other.offset])
        self.left_padding = np.concatenate([self.left_padding + (n - vis[0]),
                                            other.left_padding + (n - vis[1])])
        self._idx = n

    def extract(self, idx):                                         # cache.py:914-961
        c = QuantizedRotatingSDPACache(max_size=self.max_size, keep=self.keep,
                                       bits=self.bits, group_size=self.group_size,
                                       dtype=self.dtype)
        if self._keys is None:
            return c
        idx = _from_end(idx, self.offset.shape[0])
        visible = min(self._idx, self.max_size)
        n_tokens = max(0, min(int(self.offset[idx]), self.max_size))
        if n_tokens == 0:
            return c

        def ext(tup):
            res = tuple(t[idx:idx + 1, :, :visible].copy() for t in tup)
            if self._idx > self.max_size:
                res = tuple(_ring_temporal(t, self.keep, self._ring_ptr(), visible)
                            for t in res)
            pad = visible - n_tokens
            if pad > 0:
                res = tuple(t[:, :, pad:visible].copy() for t in res)
            return res

        c._keys = ext(self._keys)
        c._values = ext(self._values)
        c.offset = n_tokens
        c._idx = n_tokens
        if n_tokens < self.max_size:
            padl = self.max_size - n_tokens
            c._keys = tuple(np.pad(t, ((0, 0), (0, 0), (0, padl), (0, 0))) for t in c._keys)
            c._values = tuple(np.pad(t, ((0, 0), (0, 0), (0, padl), (0, 0)))
                              for t in c._values)
        return c

    @classmethod
    def merge(cls, caches):                                         # cache.py:963-1010
        if not caches:
            return cls([0], max_size=4096)
        max_size, bits, gs = caches[0].max_size, caches[0].bits, caches[0].group_size
        dtype, keep = caches[0].dtype, caches[0].keep
        lengths = [c.size() for c in caches]
        max_len = max(lengths)
        padding = [max_len - l for l in lengths]
        batch = cls(padding, max_size=max_size, keep=keep, bits=bits, group_size=gs,
                    dtype=dtype)
        if all(c.empty() for c in caches):
            return batch
        B = len(caches)
        ref = next(c for c in caches if not c.empty())
        H = ref._keys[0].shape[1]
        ks, vs = ref.state
        # Extension: max_size columns, not max_len, so the merged batch can
        # take its next decode (at column max_len).
        batch._keys = tuple(np.zeros((B, H, max_size, t.shape[3]), t.dtype) for t in ks)
        batch._values = tuple(np.zeros((B, H, max_size, t.shape[3]), t.dtype) for t in vs)
        for i, (p, c) in enumerate(zip(padding, caches)):
            if c.empty():
                continue
            kst, vst = c.state
            n = kst[0].shape[2]
            for j in range(3):
                batch._keys[j][i:i + 1, :, p:p + n] = kst[j]
                batch._values[j][i:i + 1, :, p:p + n] = vst[j]
        batch.offset = batch.offset + max_len
        batch._idx = max_len
        return batch
