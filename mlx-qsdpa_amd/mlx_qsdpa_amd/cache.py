"""Quantized KV caches on ROCm tensors (the update_and_fetch protocol).

Same classes, constructor arguments, attributes and return structure as
mlx_qsdpa/cache.py.  Each cache write runs the HIP quantize-on-append kernel
straight into the cache buffers (no per-step temporaries), and the rotating
prefill dequantizes with the ring reorder fused into the HIP dequantize
kernel.  ``update_and_fetch`` returns strided views of the capacity-padded
buffers; the decode kernel reads them by stride, so no copy precedes a
decode (the reference copies there, cache.py:195-197 + kernels.py:190).

Host bookkeeping (``offset``, ``left_padding``) lives in CPU int64 tensors,
so no cache method synchronizes the device.

Extensions over the reference (documented in each method):
* ``keep > 0`` attention sinks for the rotating caches (the reference
  asserts keep == 0, cache.py:512, 732): the first ``keep`` slots are never
  overwritten, ring writes cycle over [keep, max_size).
* rotating ``make_mask`` once offset + N exceeds max_size returns the causal
  mask over the returned window (the reference's width no longer matches the
  returned keys there, cache.py:636-644).
"""

from __future__ import annotations

from typing import List

import torch

from . import kernels


def _create_causal_mask(N, offset, window_size=None, left_padding=None, device=None):
    """cache.py:15-43.  Batched offsets give a bool (B, 1, N, max(offset)+N).

    With a GPU `device` the mask is computed there from the (B,) offsets and
    left padding, which are the only host-to-device copy (pinned, no wait)."""
    on_gpu = device is not None and torch.device(device).type == "cuda"
    if isinstance(offset, torch.Tensor) and offset.dim() > 0:
        off = offset.to("cpu", torch.int64)
        total = int(off.max()) + N
        dev = device if on_gpu else None
        if on_gpu:
            lp = None if left_padding is None else left_padding.to("cpu", torch.int64)
            both = off if lp is None else torch.stack([off, lp])
            both = kernels.to_device(both, device)
            off_d, lp_d = (both, None) if lp is None else (both[0], both[1])
        else:
            off_d = off
            lp_d = None if left_padding is None else left_padding.to("cpu", torch.int64)
        q_pos = torch.arange(N, device=dev)[None, :] + off_d[:, None]
        k_pos = torch.arange(total, device=dev)[None, :]
        mask = q_pos[:, :, None] >= k_pos[:, None, :]
        if lp_d is not None:
            mask = mask & (k_pos[:, None, :] >= lp_d[:, None, None])
        if window_size is not None:
            mask = mask & (q_pos[:, :, None] - k_pos[:, None, :] < window_size)
        mask = mask[:, None, :, :]
        return mask if dev is not None or device is None else mask.to(device)
    offset = int(offset)
    dev = device if on_gpu else None
    q_idx = torch.arange(offset, offset + N, device=dev)
    k_idx = torch.arange(offset + N, device=dev)
    mask = q_idx[:, None] >= k_idx[None]
    if window_size is not None:
        mask = mask & (q_idx[:, None] - k_idx[None] < window_size)
    return mask if dev is not None or device is None else mask.to(device)


def _zeros_q(shape3, dim, bits, group_size, dtype, device):
    per = 32 // bits
    return (torch.zeros((*shape3, dim // per), dtype=torch.uint32, device=device),
            torch.zeros((*shape3, dim // group_size), dtype=dtype, device=device),
            torch.zeros((*shape3, dim // group_size), dtype=dtype, device=device))


def _sl(tup, start, stop):
    return tuple(t[:, :, start:stop, :] for t in tup)


def _ring_runs(keep, ptr, n):
    """Column runs (start, length) that read a ring's first n slots in
    temporal order: the sinks [0, keep), the oldest other tokens [ptr, n),
    then the newest [keep, ptr).  With ptr <= keep or ptr >= n the slots are
    already in temporal order."""
    if ptr <= keep or ptr >= n:
        return [(0, n)] if n > 0 else []
    return [r for r in ((0, keep), (ptr, n - ptr), (keep, ptr - keep)) if r[1] > 0]


def _drop_front(runs, k):
    """The runs without their first k columns."""
    out = []
    for c, n in runs:
        if k >= n:
            k -= n
            continue
        out.append((c + k, n - k))
        k = 0
    return out


def _ring_temporal(t, keep, ptr, n_visible):
    """A ring buffer's first n_visible slots in temporal order (a new tensor)."""
    runs = _ring_runs(keep, ptr, n_visible)
    if len(runs) <= 1:
        return t[:, :, :n_visible]
    return torch.cat([t[:, :, c:c + n] for c, n in runs], dim=2)


def _indices(batch_indices, B):
    """Batch indices (list, range or tensor; negative counts from the end) as
    a list of host ints.  A device tensor is read back, which waits for it."""
    if isinstance(batch_indices, torch.Tensor):
        batch_indices = batch_indices.reshape(-1).tolist()
    out = []
    for i in batch_indices:
        i = int(i)
        if not -B <= i < B:
            raise IndexError(f"batch index {i} out of range for {B} sequences")
        out.append(i % B)
    return out


class _Relayout:
    """New (B, H, width, .) buffers shaped and typed like the six (packed,
    scales, biases of keys and values) of a cache, filled row by row from
    token runs of other buffers -- the batch administration's only device
    work, one qsdpa_move_rows call (kernel-argument descriptors, no host
    read, no synchronization).  Every slot of the new buffers is written:
    the runs, and zeros around them."""

    def __init__(self, like, B, width):
        self.kv = tuple(tuple(torch.empty((B, t.shape[1], width, t.shape[3]), dtype=t.dtype, device=t.device)
                              for t in tup) for tup in like)
        self.width = width
        self._moves = []

    def row(self, row, start=0, src=None, src_row=0, runs=()):
        """Batch row `row`: the columns `runs` ((start, length), in order) of
        batch row `src_row` of `src` (a (keys, values) pair of buffer
        triples) back to back from column `start`, cut at the width; zeros
        before and after them (a row of zeros without runs)."""
        dst = self.kv[0] + self.kv[1]
        segs, col = [], start
        for c, n in runs:
            n = min(n, self.width - col)
            if n > 0:
                segs.append((col, n, c))
                col += n
        if not segs:
            self._moves += [kernels.RowMove(d, row, 0, self.width) for d in dst]
            return
        srcs = src[0] + src[1]
        for i, (col, n, c) in enumerate(segs):
            # The first move also zeroes the columns before the runs, the
            # last one those after them.
            lo = 0 if i == 0 else col
            hi = self.width if i == len(segs) - 1 else col + n
            for d, sbuf in zip(dst, srcs):
                self._moves.append(kernels.RowMove(d, row, lo, hi - lo, sbuf, src_row, c, col - lo, col + n - lo))

    def run(self):
        kernels.move_rows(self._moves)
        return self.kv


def _prefill_target(cache):
    """Fresh buffers shaped like the rotating cache's window, the target of a
    prefill's requantization (which may not overwrite the window it reads).
    The old window is dropped once the launch is queued: the allocator
    reuses its memory in stream order, so a cache holds one window between
    prefills, as the reference's does.  Uninitialised: the requantization
    writes rows [0, total) and _zero_tail clears the rest when the window
    is not yet full (torch.zeros_like for the six buffers took the C5
    rotating prefill chunk from 113.6 to 132.1 us per chunk: six fill
    launches and their host calls every prefill)."""
    return (tuple(torch.empty_like(t) for t in cache._keys),
            tuple(torch.empty_like(t) for t in cache._values))


def _zero_tail(dst, total):
    """Rows [total, capacity) of a prefill target: zeros, as the rows of a
    window that were never written."""
    for t in dst[0] + dst[1]:
        if total < t.shape[2]:
            t[:, :, total:].zero_()


def _nbytes(tup):
    return sum(t.numel() * t.element_size() for t in tup)


class QuantizedSDPACache:
    """KV cache storing quantized keys/values (cache.py:54-231).

    ``update_and_fetch`` returns ``(packed_uint32, scales, biases)`` tuples
    for keys and values covering tokens [0, offset).
    """

    # Marker for an attention router (cache.py:69-71).
    _use_fused_sdpa = True

    def __init__(self, bits: int = 4, group_size: int = 32, step: int = 256):
        if bits not in (4, 8):
            raise ValueError(f"bits must be 4 or 8, got {bits}")
        self.bits = bits
        self.group_size = group_size
        self.step = step
        self.offset = 0
        self._keys = None
        self._values = None

    def empty(self):
        return self._keys is None

    @property
    def nbytes(self):
        if self._keys is None:
            return 0
        return _nbytes(self._keys) + _nbytes(self._values)

    def is_trimmable(self):
        return True

    def size(self):
        return self.offset

    def trim(self, n):
        n = min(self.offset, n)
        self.offset -= n
        return n

    def rewind(self, num_to_trim):
        num_to_trim = min(self.offset, num_to_trim)
        self.offset -= num_to_trim
        return num_to_trim > 0

    def make_mask(self, N, return_array=False, window_size=None):
        dev = self._keys[0].device if self._keys is not None else None
        if window_size is not None:
            return _create_causal_mask(N, self.offset, window_size=window_size, device=dev)
        if N == 1:
            return None
        if return_array:
            return _create_causal_mask(N, self.offset, device=dev)
        return "causal"

    @property
    def state(self):
        if self._keys is None:
            return None, None
        return _sl(self._keys, 0, self.offset), _sl(self._values, 0, self.offset)

    @state.setter
    def state(self, v):
        keys, values = v
        self._keys = keys
        self._values = values

    @property
    def meta_state(self):
        return tuple(map(str, (self.offset, self.bits, self.group_size)))

    @meta_state.setter
    def meta_state(self, v):
        self.offset, self.bits, self.group_size = map(int, v)

    @classmethod
    def from_state(cls, state, meta_state):
        obj = cls.__new__(cls)
        obj.step = 256
        obj.meta_state = meta_state
        obj.state = state
        return obj

    @classmethod
    def merge(cls, caches):
        return BatchQuantizedSDPACache.merge(caches)

    def update_and_fetch(self, keys, values):
        """Quantize keys/values (B, H_kv, S, D) and append them (cache.py:163-197)."""
        B, H, S, Dk = keys.shape
        Dv = values.shape[-1]
        prev = self.offset
        if self._keys is None or prev + S > self._keys[0].shape[2]:
            self._grow(B, H, S, Dk, Dv, keys.dtype, keys.device, prev)
        self.offset += S
        kernels.quantize_kv_into(keys, values, self._keys, self._values, prev, self.bits,
                                 self.group_size)
        return _sl(self._keys, 0, self.offset), _sl(self._values, 0, self.offset)

    def _grow(self, B, H, S, Dk, Dv, dtype, device, prev):
        """Capacity grows by ceil(S/step)*step after trimming to prev (cache.py:199-231)."""
        new_alloc = ((self.step + S - 1) // self.step) * self.step
        shape = (B, H, new_alloc)
        nk = _zeros_q(shape, Dk, self.bits, self.group_size, dtype, device)
        nv = _zeros_q(shape, Dv, self.bits, self.group_size, dtype, device)
        if self._keys is not None:
            if prev % self.step != 0:
                self._keys = _sl(self._keys, 0, prev)
                self._values = _sl(self._values, 0, prev)
            self._keys = tuple(torch.cat([o, n], dim=2) for o, n in zip(self._keys, nk))
            self._values = tuple(torch.cat([o, n], dim=2) for o, n in zip(self._values, nv))
        else:
            self._keys, self._values = nk, nv


class BatchQuantizedSDPACache:
    """Batch-aware quantized cache with left padding (cache.py:234-492)."""

    _use_fused_sdpa = True
    step = 256

    def __init__(self, left_padding: List[int], bits: int = 4, group_size: int = 32):
        self.bits = bits
        self.group_size = group_size
        self.left_padding = torch.tensor(list(left_padding), dtype=torch.int64)
        self.offset = -self.left_padding.clone()
        self._idx = 0
        self._keys = None
        self._values = None
        self._right_padding = None

    def empty(self):
        return self._keys is None

    @property
    def nbytes(self):
        if self._keys is None:
            return 0
        return _nbytes(self._keys) + _nbytes(self._values)

    def is_trimmable(self):
        return True

    def size(self):
        return self._idx

    def trim(self, n):
        n = min(self._idx, n)
        self._idx -= n
        self.offset = self.offset - n
        return n

    def kv_start(self, device=None):
        """Per-sequence first valid slot (= left padding), int32 on `device`.
        The device copy is kept until left_padding changes, so a decode loop
        uploads it once."""
        if device is None:
            return self.left_padding.to(torch.int32)
        tag = (id(self.left_padding), self.left_padding._version, str(device))
        held = getattr(self, "_kv_start_dev", None)
        if held is None or held[0] != tag:
            held = (tag, kernels.to_device(self.left_padding.to(torch.int32), device), self.left_padding)
            self._kv_start_dev = held
        return held[1]

    def update_and_fetch(self, keys, values):
        """cache.py:279-322: all sequences append at the shared column _idx."""
        B, H, S, Dk = keys.shape
        Dv = values.shape[-1]
        prev = self._idx
        if self._keys is None or prev + S > self._keys[0].shape[2]:
            new_alloc = ((self.step + S - 1) // self.step) * self.step
            shape = (B, H, new_alloc)
            nk = _zeros_q(shape, Dk, self.bits, self.group_size, keys.dtype, keys.device)
            nv = _zeros_q(shape, Dv, self.bits, self.group_size, keys.dtype, keys.device)
            if self._keys is not None:
                if prev % self.step != 0:
                    self._keys = _sl(self._keys, 0, prev)
                    self._values = _sl(self._values, 0, prev)
                self._keys = tuple(torch.cat([o, n], dim=2) for o, n in zip(self._keys, nk))
                self._values = tuple(torch.cat([o, n], dim=2) for o, n in zip(self._values, nv))
            else:
                self._keys, self._values = nk, nv
        self.offset = self.offset + S
        self._idx += S
        kernels.quantize_kv_into(keys, values, self._keys, self._values, prev, self.bits,
                                 self.group_size)
        return _sl(self._keys, 0, self._idx), _sl(self._values, 0, self._idx)

    def prepare(self, *, left_padding=None, lengths=None, right_padding=None):
        """cache.py:324-335."""
        if left_padding is not None:
            if self._keys is not None:
                raise ValueError(
                    "Left padding can only be added to an empty BatchQuantizedSDPACache")
            lp = torch.as_tensor(left_padding, dtype=torch.int64)
            self.left_padding = self.left_padding + lp
            self.offset = self.offset - lp
        if right_padding is not None and max(right_padding) > 0:
            self._right_padding = torch.as_tensor(right_padding, dtype=torch.int64)

    def finalize(self):
        """cache.py:337-348: sequences prefilled with right padding (prepare)
        are rotated so that the padding sits on the left, where it joins
        left_padding: column t of row b takes column (t - pad[b]) mod the
        capacity."""
        if self._right_padding is None:
            return
        pad = self._right_padding
        if self._keys is not None:
            kv = (self._keys, self._values)
            B, cap = self._keys[0].shape[0], self._keys[0].shape[2]
            rl = _Relayout(kv, B, cap)
            for b, p in enumerate(pad.tolist()):
                p = p % cap if cap else 0
                rl.row(b, 0, kv, b, [(cap - p, p), (0, cap - p)])
            self._keys, self._values = rl.run()
        self.offset = self.offset - pad
        self.left_padding = self.left_padding + pad
        self._right_padding = None

    @property
    def state(self):
        if self._keys is None:
            return None, None, self.offset, self.left_padding
        keys, values = self._keys, self._values
        if self._idx < keys[0].shape[2]:
            keys = _sl(keys, 0, self._idx)
            values = _sl(values, 0, self._idx)
        return keys, values, self.offset, self.left_padding

    @state.setter
    def state(self, v):
        self._keys, self._values, self.offset, self.left_padding = v
        self.offset = torch.as_tensor(self.offset, dtype=torch.int64).cpu()
        self.left_padding = torch.as_tensor(self.left_padding, dtype=torch.int64).cpu()
        self._idx = 0 if self._keys is None else self._keys[0].shape[2]

    @property
    def meta_state(self):
        """Extension (the reference's batch cache has none): the settings a
        saved state needs to come back (offsets travel in ``state``)."""
        return tuple(map(str, (self.bits, self.group_size)))

    @meta_state.setter
    def meta_state(self, v):
        self.bits, self.group_size = map(int, v)

    @classmethod
    def from_state(cls, state, meta_state):
        obj = cls.__new__(cls)
        obj._right_padding = None
        obj.meta_state = meta_state
        obj.state = state
        return obj

    def make_mask(self, N, return_array=False, **kwargs):
        """cache.py:369-376 (logical offsets for queries, buffer index for keys)."""
        dev = self._keys[0].device if self._keys is not None else None
        return _create_causal_mask(N, offset=self.offset, left_padding=self.left_padding,
                                   window_size=kwargs.get("window_size"), device=dev)

    def filter(self, batch_indices):
        """cache.py:378-391: keep the listed sequences, in that order; the
        leading columns that are left padding in every kept sequence are
        dropped (capacity, _idx and left_padding shrink by their number)."""
        keep = _indices(batch_indices, self.offset.shape[0])
        lp = self.left_padding[keep]
        drop = 0
        if self._keys is not None:
            drop = int(lp.min()) if keep else 0
            kv = (self._keys, self._values)
            width = self._keys[0].shape[2] - drop
            rl = _Relayout(kv, len(keep), width)
            for j, b in enumerate(keep):
                rl.row(j, 0, kv, b, [(drop, width)])
            self._keys, self._values = rl.run()
            self._idx -= drop
        self.offset = self.offset[keep]
        self.left_padding = lp - drop

    def extend(self, other):
        """cache.py:393-427: other's sequences are appended after this
        batch's.  Each side is shifted right so that both write at the larger
        _idx (the shift joins its left padding), into buffers as wide as the
        wider capacity; a side without buffers contributes zero rows."""
        sides = (self, other)
        end = max(c._idx for c in sides)
        filled = [c for c in sides if c._keys is not None]
        if filled:
            width = max(c._keys[0].shape[2] for c in filled)
            rl = _Relayout((filled[0]._keys, filled[0]._values), sum(c.offset.shape[0] for c in sides), width)
            row = 0
            for c in sides:
                for b in range(c.offset.shape[0]):
                    if c._keys is None:
                        rl.row(row, end - c._idx)
                    else:
                        rl.row(row, end - c._idx, (c._keys, c._values), b, [(0, c._keys[0].shape[2])])
                    row += 1
            self._keys, self._values = rl.run()
        self.offset = torch.cat([self.offset, other.offset])
        self.left_padding = torch.cat([self.left_padding + (end - self._idx),
                                       other.left_padding + (end - other._idx)])
        self._idx = end

    def extract(self, idx):
        """cache.py:429-444: sequence idx as a QuantizedSDPACache holding the
        columns after its left padding up to _idx (capacity = that count)."""
        cache = QuantizedSDPACache(bits=self.bits, group_size=self.group_size)
        if self._keys is None:
            return cache
        (b,) = _indices([idx], self.offset.shape[0])
        start = int(self.left_padding[b])
        n = self._idx - start
        kv = (self._keys, self._values)
        rl = _Relayout(kv, 1, n)
        rl.row(0, 0, kv, b, [(start, n)])
        cache._keys, cache._values = rl.run()
        cache.offset = n
        return cache

    @classmethod
    def merge(cls, caches):
        """cache.py:446-492: single caches stacked into one batch, each
        right-aligned at the longest (the shorter get left padding)."""
        if not caches:
            return cls([0])
        lengths = [c.offset for c in caches]
        width = max(lengths)
        batch = cls([width - n for n in lengths], bits=caches[0].bits, group_size=caches[0].group_size)
        filled = [c for c in caches if not c.empty()]
        if not filled:
            return batch
        rl = _Relayout((filled[0]._keys, filled[0]._values), len(caches), width)
        for i, c in enumerate(caches):
            if c.empty():
                rl.row(i)
            else:
                rl.row(i, width - c.offset, (c._keys, c._values), 0, [(0, c.offset)])
        batch._keys, batch._values = rl.run()
        batch.offset = batch.offset + width
        batch._idx = width
        return batch


class QuantizedRotatingSDPACache:
    """Fixed-size quantized ring buffer (cache.py:495-711), plus ``keep`` sinks."""

    _use_fused_sdpa = True

    def __init__(self, max_size: int, keep: int = 0, bits: int = 4, group_size: int = 32):
        if bits not in (4, 8):
            raise ValueError(f"bits must be 4 or 8, got {bits}")
        if not 0 <= keep < max_size:
            raise ValueError(f"keep must satisfy 0 <= keep < max_size, got {keep}")
        self.max_size = max_size
        self.keep = keep
        self.bits = bits
        self.group_size = group_size
        self.offset = 0
        self._idx = 0
        self._keys = None
        self._values = None

    def empty(self):
        return self._keys is None

    @property
    def nbytes(self):
        if self._keys is None:
            return 0
        return _nbytes(self._keys) + _nbytes(self._values)

    def size(self):
        return min(self.offset, self.max_size)

    def is_trimmable(self):
        return self.offset < self.max_size

    def _alloc(self, B, H, Dk, Dv, dtype, device):
        shape = (B, H, self.max_size)
        self._keys = _zeros_q(shape, Dk, self.bits, self.group_size, dtype, device)
        self._values = _zeros_q(shape, Dv, self.bits, self.group_size, dtype, device)

    def update_and_fetch(self, keys, values):
        """cache.py:554-572: S == 1 writes one ring slot, S > 1 re-quantizes the window."""
        B, H, S, Dk = keys.shape
        if self._keys is None:
            self._alloc(B, H, Dk, values.shape[-1], keys.dtype, keys.device)
        if S == 1:
            return self._update_decode(keys, values)
        return self._update_prefill(keys, values)

    def _write_pos(self):
        # Reference: _idx % max_size with _idx kept at max_size as a sentinel
        # (cache.py:578, 584-587); the slot after the last is `keep`.
        return self._idx if self._idx < self.max_size else self.keep

    def _update_decode(self, keys, values):
        """cache.py:574-591."""
        wp = self._write_pos()
        kernels.quantize_kv_into(keys, values, self._keys, self._values, wp, self.bits,
                                 self.group_size)
        self._idx = wp + 1
        self.offset += 1
        n_visible = min(self.offset, self.max_size)
        return _sl(self._keys, 0, n_visible), _sl(self._values, 0, n_visible)

    def _ring_rot(self, n_visible):
        """`rot` of the fused dequantize that yields temporal order."""
        if self.offset > self.max_size and self.keep < self._idx < n_visible:
            return self._idx - self.keep
        return 0

    def _update_prefill(self, keys, values):
        """cache.py:593-634: the window dequantized in temporal order, the chunk
        appended, the first `keep` and the newest max_size - keep kept,
        quantized again -- one launch for K and V (qsdpa_requant_window) into
        the spare buffer set, which then becomes the window."""
        S = keys.shape[2]
        n_old = min(self.offset, self.max_size)
        rot = self._ring_rot(n_old) if n_old else 0
        dst = _prefill_target(self)
        total = kernels.requant_window((self._keys, self._values), (keys, values), dst, n_old, self.keep,
                                       rot, self.max_size, self.bits, self.group_size)
        _zero_tail(dst, total)
        self._keys, self._values = dst
        self.offset += S
        self._idx = total if total < self.max_size else self.keep
        n_visible = min(self.offset, self.max_size)
        return _sl(self._keys, 0, n_visible), _sl(self._values, 0, n_visible)

    def make_mask(self, N, return_array=False, window_size=None):
        """cache.py:636-644; past the window, the causal mask over the returned keys."""
        if N == 1:
            return None
        if return_array or window_size is not None:
            eff = min(self.offset, self.max_size)
            if self.offset + N > self.max_size:
                eff = min(self.offset + N, self.max_size) - N
            dev = self._keys[0].device if self._keys is not None else None
            return _create_causal_mask(N, eff, window_size=window_size, device=dev)
        return "causal"

    def trim(self, n):
        n = min(self.offset, n)
        self.offset -= n
        self._idx -= n
        return n

    def rewind(self, num_to_trim):
        if self.offset >= self.max_size:
            return False
        num_to_trim = min(self.offset, num_to_trim)
        self.offset -= num_to_trim
        self._idx -= num_to_trim
        return num_to_trim > 0

    def _temporal_runs(self):
        """Column runs of the window in temporal order."""
        n = min(self.offset, self.max_size)
        if self.offset > self.max_size:
            return _ring_runs(self.keep, self._idx, n)
        return [(0, n)] if n > 0 else []

    @property
    def state(self):
        """cache.py:662-678: tensors in temporal order."""
        if self._keys is None:
            return None, None
        n_visible = min(self.offset, self.max_size)
        if self.offset > self.max_size:
            ptr = self._idx
            return (tuple(_ring_temporal(t, self.keep, ptr, n_visible) for t in self._keys),
                    tuple(_ring_temporal(t, self.keep, ptr, n_visible) for t in self._values))
        return _sl(self._keys, 0, n_visible), _sl(self._values, 0, n_visible)

    @state.setter
    def state(self, v):
        """cache.py:680-711: re-expand a temporal snapshot to max_size slots."""
        keys, values = v
        if keys is None:
            self._keys = None
            self._values = None
            return
        n_visible = keys[0].shape[2]
        # The snapshot is in temporal order: the ring restarts unrotated and
        # the next write goes to slot n_visible, or to `keep` (the oldest
        # token after the sinks) when the window is full.  (Extension: the
        # reference leaves _idx to the caller.)
        self._idx = n_visible
        pad_len = self.max_size - n_visible
        if pad_len <= 0:
            self._keys = keys
            self._values = values
            return
        self._keys = tuple(torch.nn.functional.pad(t, (0, 0, 0, pad_len)) for t in keys)
        self._values = tuple(torch.nn.functional.pad(t, (0, 0, 0, pad_len)) for t in values)

    @property
    def meta_state(self):
        """Extension (the reference's rotating cache has none): the settings
        and token count a saved temporal-order state needs to come back."""
        return tuple(map(str, (self.keep, self.max_size, self.offset, self.bits, self.group_size)))

    @meta_state.setter
    def meta_state(self, v):
        self.keep, self.max_size, self.offset, self.bits, self.group_size = map(int, v)

    @classmethod
    def from_state(cls, state, meta_state):
        obj = cls.__new__(cls)
        obj._keys = obj._values = None
        obj.meta_state = meta_state
        obj._idx = 0
        obj.state = state
        return obj


class BatchQuantizedRotatingSDPACache:
    """Batched quantized ring buffer (cache.py:714-1010), plus ``keep`` sinks."""

    _use_fused_sdpa = True

    def __init__(self, left_padding, max_size, keep=0, bits=4, group_size=32):
        if not 0 <= keep < max_size:
            raise ValueError(f"keep must satisfy 0 <= keep < max_size, got {keep}")
        self.max_size = max_size
        self.keep = keep
        self.bits = bits
        self.group_size = group_size
        self.left_padding = torch.tensor(list(left_padding), dtype=torch.int64)
        self.offset = -self.left_padding.clone()
        self._idx = 0
        self._keys = None
        self._values = None

    def empty(self):
        return self._keys is None

    @property
    def nbytes(self):
        if self._keys is None:
            return 0
        return _nbytes(self._keys) + _nbytes(self._values)

    def size(self):
        return min(self._idx, self.max_size)

    def is_trimmable(self):
        return self._idx < self.max_size

    def trim(self, n):
        n = min(self._idx, n)
        self._idx -= n
        self.offset = self.offset - n
        return n

    def _write_pos(self):
        # Reference: _idx % max_size, _idx never wraps (cache.py:800, 806-807).
        if self._idx < self.max_size:
            return self._idx
        return self.keep + (self._idx - self.max_size) % (self.max_size - self.keep)

    def update_and_fetch(self, keys, values):
        """cache.py:764-794."""
        B, H, S, Dk = keys.shape
        if self._keys is None:
            shape = (B, H, self.max_size)
            self._keys = _zeros_q(shape, Dk, self.bits, self.group_size, keys.dtype, keys.device)
            self._values = _zeros_q(shape, values.shape[-1], self.bits, self.group_size,
                                    keys.dtype, keys.device)
        if S == 1:
            return self._update_decode(keys, values)
        return self._update_prefill(keys, values)

    def _update_decode(self, keys, values):
        """cache.py:796-811."""
        wp = self._write_pos()
        kernels.quantize_kv_into(keys, values, self._keys, self._values, wp, self.bits,
                                 self.group_size)
        self.offset = self.offset + 1
        self._idx += 1
        n = min(self._idx, self.max_size)
        return _sl(self._keys, 0, n), _sl(self._values, 0, n)

    def _ring_rot(self):
        if self._idx > self.max_size:
            ptr = self._write_pos()
            if ptr > self.keep:
                return ptr - self.keep
        return 0

    def _update_prefill(self, keys, values):
        """cache.py:813-857: as QuantizedRotatingSDPACache._update_prefill, for
        the batch (one launch for K and V into the spare buffer set)."""
        S = keys.shape[2]
        n_old = min(self._idx, self.max_size)
        rot = self._ring_rot() if n_old else 0
        dst = _prefill_target(self)
        total = kernels.requant_window((self._keys, self._values), (keys, values), dst, n_old, self.keep,
                                       rot, self.max_size, self.bits, self.group_size)
        _zero_tail(dst, total)
        self._keys, self._values = dst
        self.offset = self.offset + S
        self._idx = total
        return _sl(self._keys, 0, total), _sl(self._values, 0, total)

    def make_mask(self, N, return_array=False, **kwargs):
        """cache.py:859-866; past the window, causal over the returned keys."""
        off = torch.minimum(self.offset, torch.tensor(self.max_size))
        if int(off.max()) + N > self.max_size:
            off = torch.minimum(self.offset + N, torch.tensor(self.max_size)) - N
        dev = self._keys[0].device if self._keys is not None else None
        return _create_causal_mask(N, offset=off, left_padding=self.left_padding,
                                   window_size=kwargs.get("window_size"), device=dev)

    @property
    def state(self):
        """Extension (the reference's batched rotating cache has no state):
        the window of every sequence in temporal order, offset and
        left_padding -- the form a saved batch comes back from."""
        if self._keys is None:
            return None, None, self.offset, self.left_padding
        n, ptr = min(self._idx, self.max_size), self._write_pos()
        if self._idx > self.max_size:
            return (tuple(_ring_temporal(t, self.keep, ptr, n) for t in self._keys),
                    tuple(_ring_temporal(t, self.keep, ptr, n) for t in self._values),
                    self.offset, self.left_padding)
        return _sl(self._keys, 0, n), _sl(self._values, 0, n), self.offset, self.left_padding

    @state.setter
    def state(self, v):
        """A temporal-order window back into max_size slots; the ring restarts
        unrotated (_idx = the window length)."""
        keys, values, offset, left_padding = v
        self.offset = torch.as_tensor(offset, dtype=torch.int64).cpu()
        self.left_padding = torch.as_tensor(left_padding, dtype=torch.int64).cpu()
        if keys is None:
            self._keys = self._values = None
            self._idx = 0
            return
        n = keys[0].shape[2]
        pad = self.max_size - n
        self._keys = tuple(torch.nn.functional.pad(t, (0, 0, 0, pad)) if pad > 0 else t for t in keys)
        self._values = tuple(torch.nn.functional.pad(t, (0, 0, 0, pad)) if pad > 0 else t for t in values)
        self._idx = n

    @property
    def meta_state(self):
        return tuple(map(str, (self.keep, self.max_size, self.bits, self.group_size)))

    @meta_state.setter
    def meta_state(self, v):
        self.keep, self.max_size, self.bits, self.group_size = map(int, v)

    @classmethod
    def from_state(cls, state, meta_state):
        obj = cls.__new__(cls)
        obj.meta_state = meta_state
        obj.state = state
        return obj

    def _temporal_runs(self):
        """Column runs of the window in temporal order (shared by all rows)."""
        n = min(self._idx, self.max_size)
        if self._idx > self.max_size:
            return _ring_runs(self.keep, self._write_pos(), n)
        return [(0, n)] if n > 0 else []

    def filter(self, batch_indices):
        """cache.py:868-874: keep the listed sequences, in that order (rows
        move as they are: the ring layout is shared by the batch)."""
        keep = _indices(batch_indices, self.offset.shape[0])
        if self._keys is not None:
            kv = (self._keys, self._values)
            width = self._keys[0].shape[2]
            rl = _Relayout(kv, len(keep), width)
            for j, b in enumerate(keep):
                rl.row(j, 0, kv, b, [(0, width)])
            self._keys, self._values = rl.run()
        self.offset = self.offset[keep]
        self.left_padding = self.left_padding[keep]

    def extend(self, other):
        """cache.py:876-912: other's sequences are appended after this
        batch's.  Each side's window is laid out in temporal order and
        right-aligned at the longer window n (the shorter side's shift joins
        its left padding) in max_size-wide buffers, and the layout starts
        unrotated (_idx = n).  While neither ring has wrapped this is the
        reference's left shift by the _idx difference; the reference needs
        equal buffer widths there, and after a wrap it shifts the ring as it
        lies, out of temporal order.  A side without buffers contributes
        zero rows."""
        if other.max_size != self.max_size or other.keep != self.keep:
            raise ValueError("extend needs caches with the same max_size and keep")
        sides = (self, other)
        vis = [min(c._idx, c.max_size) if c._keys is not None else 0 for c in sides]
        n = max(vis)
        filled = [c for c in sides if c._keys is not None]
        if filled:
            rl = _Relayout((filled[0]._keys, filled[0]._values), sum(c.offset.shape[0] for c in sides),
                           self.max_size)
            row = 0
            for c, v in zip(sides, vis):
                runs = c._temporal_runs() if c._keys is not None else []
                for b in range(c.offset.shape[0]):
                    if runs:
                        rl.row(row, n - v, (c._keys, c._values), b, runs)
                    else:
                        rl.row(row)
                    row += 1
            self._keys, self._values = rl.run()
        self.offset = torch.cat([self.offset, other.offset])
        self.left_padding = torch.cat([self.left_padding + (n - vis[0]), other.left_padding + (n - vis[1])])
        self._idx = n

    def extract(self, idx):
        """cache.py:914-961: sequence idx as a QuantizedRotatingSDPACache:
        its last min(offset[idx], max_size) tokens in temporal order (the
        window without the sequence's left padding) in a max_size buffer."""
        cache = QuantizedRotatingSDPACache(max_size=self.max_size, keep=self.keep,
                                           bits=self.bits, group_size=self.group_size)
        if self._keys is None:
            return cache
        (b,) = _indices([idx], self.offset.shape[0])
        n = max(0, min(int(self.offset[b]), self.max_size))
        if n == 0:
            return cache
        visible = min(self._idx, self.max_size)
        kv = (self._keys, self._values)
        rl = _Relayout(kv, 1, self.max_size)
        rl.row(0, 0, kv, b, _drop_front(self._temporal_runs(), visible - n))
        cache._keys, cache._values = rl.run()
        cache.offset = n
        cache._idx = n
        return cache

    @classmethod
    def merge(cls, caches):
        """cache.py:963-1010: single rotating caches stacked into one batch,
        each window in temporal order and right-aligned at the longest (the
        shorter get left padding).  The buffers are max_size wide, so the
        merged batch can go on decoding (the reference allocates only the
        longest window, which leaves the next decode no slot)."""
        if not caches:
            return cls([0], max_size=4096)
        c0 = caches[0]
        lengths = [c.size() for c in caches]
        width = max(lengths)
        batch = cls([width - n for n in lengths], max_size=c0.max_size, keep=c0.keep, bits=c0.bits,
                    group_size=c0.group_size)
        filled = [c for c in caches if not c.empty()]
        if not filled:
            return batch
        rl = _Relayout((filled[0]._keys, filled[0]._values), len(caches), c0.max_size)
        for i, c in enumerate(caches):
            runs = [] if c.empty() else c._temporal_runs()
            if runs:
                rl.row(i, width - c.size(), (c._keys, c._values), 0, runs)
            else:
                rl.row(i)
        batch._keys, batch._values = rl.run()
        batch.offset = batch.offset + width
        batch._idx = width
        return batch
