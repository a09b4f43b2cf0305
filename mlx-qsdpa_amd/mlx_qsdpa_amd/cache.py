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
    """cache.py:15-43.  Batched offsets give a bool (B, 1, N, max(offset)+N)."""
    if isinstance(offset, torch.Tensor) and offset.dim() > 0:
        off = offset.to("cpu", torch.int64)
        max_off = int(off.max())
        total = max_off + N
        q_pos = torch.arange(N)[None, :] + off[:, None]
        k_pos = torch.arange(total)[None, :]
        mask = q_pos[:, :, None] >= k_pos[:, None, :]
        if left_padding is not None:
            lp = left_padding.to("cpu", torch.int64)
            mask = mask & (k_pos[:, None, :] >= lp[:, None, None])
        if window_size is not None:
            mask = mask & (q_pos[:, :, None] - k_pos[:, None, :] < window_size)
        mask = mask[:, None, :, :]
    else:
        offset = int(offset)
        q_idx = torch.arange(offset, offset + N)
        k_idx = torch.arange(offset + N)
        mask = q_idx[:, None] >= k_idx[None]
        if window_size is not None:
            mask = mask & (q_idx[:, None] - k_idx[None] < window_size)
    return mask if device is None else mask.to(device)


def _dynamic_roll(x, shifts, axis):
    """cache.py:46-51 for axis 2 of a (B, H, N, d) tensor, shifts (B,)."""
    n = x.shape[axis]
    idx = (torch.arange(n)[None, :] - shifts.to("cpu", torch.int64)[:, None]) % n
    idx = idx.to(x.device)[:, None, :, None].expand(x.shape[0], x.shape[1], n, x.shape[3])
    src = x.view(torch.int32) if x.dtype == torch.uint32 else x
    out = torch.gather(src, axis, idx)
    return out.view(torch.uint32) if x.dtype == torch.uint32 else out


def _zeros_q(shape3, dim, bits, group_size, dtype, device):
    per = 32 // bits
    return (torch.zeros((*shape3, dim // per), dtype=torch.uint32, device=device),
            torch.zeros((*shape3, dim // group_size), dtype=dtype, device=device),
            torch.zeros((*shape3, dim // group_size), dtype=dtype, device=device))


def _sl(tup, start, stop):
    return tuple(t[:, :, start:stop, :] for t in tup)


def _ring_temporal(t, keep, ptr, n_visible):
    """Slots in temporal order: [0:keep] + [ptr:n] + [keep:ptr]."""
    if ptr <= keep or ptr >= n_visible:
        return t[:, :, :n_visible]
    return torch.cat([t[:, :, :keep], t[:, :, ptr:n_visible], t[:, :, keep:ptr]], dim=2)


def _spare_for(cache):
    """The rotating cache's second buffer set (the target of a prefill's
    requantization, which may not overwrite the window it reads), allocated
    on first use and whenever the window's buffers changed shape.  It is
    working memory, not cache state: nbytes does not count it."""
    spare = getattr(cache, "_spare", None)
    if spare is None or any(a.shape != b.shape or a.dtype != b.dtype or a.device != b.device
                            for a, b in zip(spare[0] + spare[1], cache._keys + cache._values)):
        spare = (tuple(torch.zeros_like(t) for t in cache._keys),
                 tuple(torch.zeros_like(t) for t in cache._values))
    return spare


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
        if window_size is not None:
            return _create_causal_mask(N, self.offset, window_size=window_size)
        if N == 1:
            return None
        if return_array:
            return _create_causal_mask(N, self.offset)
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
        """Per-sequence first valid slot (= left padding), int32 on `device`."""
        lp = self.left_padding.to(torch.int32)
        return lp if device is None else lp.to(device, non_blocking=True)

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
        """cache.py:337-348: roll right padding to the left."""
        if self._right_padding is not None:
            pad = self._right_padding
            self._keys = tuple(_dynamic_roll(t, pad, 2) for t in self._keys)
            self._values = tuple(_dynamic_roll(t, pad, 2) for t in self._values)
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

    def make_mask(self, N, return_array=False, **kwargs):
        """cache.py:369-376 (logical offsets for queries, buffer index for keys)."""
        dev = self._keys[0].device if self._keys is not None else None
        return _create_causal_mask(N, offset=self.offset, left_padding=self.left_padding,
                                   window_size=kwargs.get("window_size"), device=dev)

    def filter(self, batch_indices):
        """cache.py:378-391."""
        bi = torch.as_tensor(batch_indices, dtype=torch.int64)
        if self._keys is not None:
            dev_bi = bi.to(self._keys[0].device)
            self._keys = tuple(t.index_select(0, dev_bi) for t in self._keys)
            self._values = tuple(t.index_select(0, dev_bi) for t in self._values)
        self.offset = self.offset[bi]
        self.left_padding = self.left_padding[bi]
        min_pad = int(self.left_padding.min())
        if min_pad > 0:
            self._keys = tuple(t[:, :, min_pad:] for t in self._keys)
            self._values = tuple(t[:, :, min_pad:] for t in self._values)
            self._idx -= min_pad
            self.left_padding = self.left_padding - min_pad

    def extend(self, other):
        """cache.py:393-427."""
        max_idx = max(self._idx, other._idx)
        max_size = max(self._keys[0].shape[2], other._keys[0].shape[2])

        def pad_quant(c_idx, tuples):
            left = max_idx - c_idx
            right = max_size - tuples[0].shape[2] - left
            res = []
            for t in tuples:
                tr = t
                if right < 0:
                    tr = tr[:, :, :right]
                    right_actual = 0
                else:
                    right_actual = right
                if left != 0 or right_actual != 0:
                    tr = torch.nn.functional.pad(tr, (0, 0, left, right_actual))
                res.append(tr)
            return tuple(res), left

        sk, s_left = pad_quant(self._idx, self._keys)
        sv, _ = pad_quant(self._idx, self._values)
        ok, o_left = pad_quant(other._idx, other._keys)
        ov, _ = pad_quant(other._idx, other._values)
        self._keys = tuple(torch.cat([s, o]) for s, o in zip(sk, ok))
        self._values = tuple(torch.cat([s, o]) for s, o in zip(sv, ov))
        self.offset = torch.cat([self.offset, other.offset])
        self.left_padding = torch.cat([self.left_padding + s_left, other.left_padding + o_left])
        self._idx = max_idx

    def extract(self, idx):
        """cache.py:429-444."""
        cache = QuantizedSDPACache(bits=self.bits, group_size=self.group_size)
        if self._keys is None:
            return cache
        padding = int(self.left_padding[idx])
        cache._keys = tuple(t[idx:idx + 1, :, padding:self._idx].contiguous() for t in self._keys)
        cache._values = tuple(t[idx:idx + 1, :, padding:self._idx].contiguous()
                              for t in self._values)
        cache.offset = self._idx - padding
        return cache

    @classmethod
    def merge(cls, caches):
        """cache.py:446-492: left-pad single caches into one batch."""
        if not caches:
            return cls([0])
        bits = caches[0].bits
        gs = caches[0].group_size
        lengths = [c.offset for c in caches]
        max_len = max(lengths)
        padding = [max_len - l for l in lengths]
        batch = cls(padding, bits=bits, group_size=gs)
        if all(c.empty() for c in caches):
            return batch
        B = len(caches)
        ref = next(c for c in caches if not c.empty())
        H = ref._keys[0].shape[1]

        def alloc(tup):
            return tuple(torch.zeros((B, H, max_len, t.shape[3]), dtype=t.dtype, device=t.device)
                         for t in tup)

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
        spare = _spare_for(self)
        total = kernels.requant_window((self._keys, self._values), (keys, values), spare, n_old, self.keep,
                                       rot, self.max_size, self.bits, self.group_size)
        self._spare = (self._keys, self._values)
        self._keys, self._values = spare
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
        pad_len = self.max_size - n_visible
        if pad_len <= 0:
            self._keys = keys
            self._values = values
            return
        self._keys = tuple(torch.nn.functional.pad(t, (0, 0, 0, pad_len)) for t in keys)
        self._values = tuple(torch.nn.functional.pad(t, (0, 0, 0, pad_len)) for t in values)


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
        spare = _spare_for(self)
        total = kernels.requant_window((self._keys, self._values), (keys, values), spare, n_old, self.keep,
                                       rot, self.max_size, self.bits, self.group_size)
        self._spare = (self._keys, self._values)
        self._keys, self._values = spare
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

    def filter(self, batch_indices):
        """cache.py:868-874."""
        bi = torch.as_tensor(batch_indices, dtype=torch.int64)
        if self._keys is not None:
            dev_bi = bi.to(self._keys[0].device)
            self._keys = tuple(t.index_select(0, dev_bi) for t in self._keys)
            self._values = tuple(t.index_select(0, dev_bi) for t in self._values)
        self.offset = self.offset[bi]
        self.left_padding = self.left_padding[bi]

    def extend(self, other):
        """cache.py:876-912."""
        if self._keys is None and other._keys is None:
            self.offset = torch.cat([self.offset, other.offset])
            self.left_padding = torch.cat([self.left_padding, other.left_padding])
            return
        max_idx = max(self._idx, other._idx)

        def pad_quant(tuples, c_idx):
            left = max_idx - c_idx
            if left == 0:
                return tuples
            return tuple(torch.nn.functional.pad(t, (0, 0, left, 0)) for t in tuples)

        sk = pad_quant(self._keys, self._idx) if self._keys is not None else None
        sv = pad_quant(self._values, self._idx) if self._values is not None else None
        ok = pad_quant(other._keys, other._idx) if other._keys is not None else None
        ov = pad_quant(other._values, other._idx) if other._values is not None else None
        if sk is not None and ok is not None:
            self._keys = tuple(torch.cat([s, o]) for s, o in zip(sk, ok))
            self._values = tuple(torch.cat([s, o]) for s, o in zip(sv, ov))
        elif ok is not None:
            self._keys = ok
            self._values = ov
        s_left = max_idx - self._idx
        o_left = max_idx - other._idx
        self.offset = torch.cat([self.offset, other.offset])
        self.left_padding = torch.cat([self.left_padding + s_left, other.left_padding + o_left])
        self._idx = max_idx

    def extract(self, idx):
        """cache.py:914-961: one sequence as a single rotating cache, temporal order."""
        cache = QuantizedRotatingSDPACache(max_size=self.max_size, keep=self.keep,
                                           bits=self.bits, group_size=self.group_size)
        if self._keys is None:
            return cache
        visible = min(self._idx, self.max_size)
        n_tokens = max(0, min(int(self.offset[idx]), self.max_size))
        if n_tokens == 0:
            return cache
        ptr = self._write_pos()

        def extract_temporal(tuples):
            res = tuple(t[idx:idx + 1, :, :visible].contiguous() for t in tuples)
            if self._idx > self.max_size:
                res = tuple(_ring_temporal(t, self.keep, ptr, visible) for t in res)
            padding = visible - n_tokens
            if padding > 0:
                res = tuple(t[:, :, padding:visible].contiguous() for t in res)
            return res

        cache._keys = extract_temporal(self._keys)
        cache._values = extract_temporal(self._values)
        cache.offset = n_tokens
        cache._idx = n_tokens
        if n_tokens < self.max_size:
            pad_len = self.max_size - n_tokens
            cache._keys = tuple(torch.nn.functional.pad(t, (0, 0, 0, pad_len)) for t in cache._keys)
            cache._values = tuple(torch.nn.functional.pad(t, (0, 0, 0, pad_len))
                                  for t in cache._values)
        return cache

    @classmethod
    def merge(cls, caches):
        """cache.py:963-1010."""
        if not caches:
            return cls([0], max_size=4096)
        max_size = caches[0].max_size
        bits = caches[0].bits
        gs = caches[0].group_size
        keep = caches[0].keep
        lengths = [c.size() for c in caches]
        max_len = max(lengths)
        padding = [max_len - l for l in lengths]
        batch = cls(padding, max_size=max_size, keep=keep, bits=bits, group_size=gs)
        if all(c.empty() for c in caches):
            return batch
        B = len(caches)
        ref = next(c for c in caches if not c.empty())
        H = ref._keys[0].shape[1]
        ks_ref, vs_ref = ref.state

        def alloc(tup):
            return tuple(torch.zeros((B, H, max_len, t.shape[3]), dtype=t.dtype, device=t.device)
                         for t in tup)

        batch._keys = alloc(ks_ref)
        batch._values = alloc(vs_ref)
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
