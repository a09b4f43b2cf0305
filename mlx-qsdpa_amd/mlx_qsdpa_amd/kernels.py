"""torch-facing wrappers of the HIP kernels (C ABI: include/qsdpa.h).

Every function here launches on the tensor's device, on torch's current
stream, and never synchronizes.  Tensors must live on a ROCm device; CPU
tensors raise (the library has no CPU implementation).
"""

from __future__ import annotations

import ctypes
import threading
from typing import NamedTuple, Optional

import torch

from . import _lib

_DTYPE_CODE = {torch.float16: _lib.QSDPA_F16, torch.bfloat16: _lib.QSDPA_BF16}
# Head dims the decode kernels are compiled for (qsdpa_decode returns
# QSDPA_ERR_UNSUPPORTED for any other D).
HEAD_DIMS = (64, 128, 256)
_MASK_CODE = {torch.float16: _lib.QSDPA_F16, torch.bfloat16: _lib.QSDPA_BF16,
              torch.float32: _lib.QSDPA_F32, torch.bool: _lib.QSDPA_BOOL}


def _require_device(*tensors):
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise RuntimeError(
                "mlx_qsdpa_amd kernels run on a ROCm GPU only; got a tensor on "
                f"{t.device} (there is no CPU implementation)")


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return _DTYPE_CODE[dtype]
    except KeyError:
        raise ValueError(f"dtype must be float16 or bfloat16, got {dtype}") from None


def _view(t: torch.Tensor | None) -> _lib.View:
    """View of a [B, H, N, inner] tensor (innermost stride must be 1)."""
    if t is None:
        return _lib.View(None, 0, 0, 0)
    if t.dim() != 4:
        raise ValueError(f"expected a 4-D tensor, got shape {tuple(t.shape)}")
    if t.shape[-1] > 1 and t.stride(-1) != 1:
        raise ValueError("innermost dimension must be contiguous")
    s = t.stride()
    return _lib.View(t.data_ptr(), s[0], s[1], s[2])


def _rows_in_storage(t: torch.Tensor) -> int:
    """Token rows (dim 2) a [B, H, N, inner] view could address within its
    storage with its own strides: the largest n such that element
    (B-1, H-1, n-1, inner-1) lies inside the storage."""
    B, H, _, inner = t.shape
    sb, sh, sn, _ = t.stride()
    elems = t.untyped_storage().nbytes() // t.element_size()
    last_other = t.storage_offset() + (B - 1) * sb + (H - 1) * sh + inner - 1
    if sn <= 0:
        return t.shape[2]
    return max(0, (elems - 1 - last_other) // sn + 1)


def to_device(t: torch.Tensor, device) -> torch.Tensor:
    """A small host tensor (mask, offsets) on a GPU `device`, copied in
    stream order from pinned memory: the host does not wait for the GPU."""
    if t.device.type == "cuda" or torch.device(device).type != "cuda":
        return t.to(device)
    return t.pin_memory().to(device, non_blocking=True)


_RAW_STREAM = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream(t: torch.Tensor) -> int:
    """The current stream of t's device (raw handle)."""
    if _RAW_STREAM is not None:
        return _RAW_STREAM(t.get_device())
    return torch.cuda.current_stream(t.device).cuda_stream


def _inner_contig(t: torch.Tensor) -> torch.Tensor:
    return t if (t.shape[-1] <= 1 or t.stride(-1) == 1) else t.contiguous()


# ---------------------------------------------------------------------------
# quantize / dequantize
# ---------------------------------------------------------------------------
def _expect_shape(name, t, shape):
    if t is not None and tuple(t.shape) != tuple(shape):
        raise ValueError(f"{name}: expected shape {tuple(shape)}, got {tuple(t.shape)}")


def _quantize_args(src: torch.Tensor, dst: tuple, t0: int, bits: int, group_size: int):
    _require_device(src, *dst)
    src = _inner_contig(src)
    B, H, S, D = src.shape
    if bits not in (4, 8) or D % group_size:
        raise ValueError(f"bad bits={bits} / group_size={group_size} for D={D}")
    cap = dst[0].shape[2]
    if t0 < 0 or t0 + S > cap:
        raise ValueError(f"tokens [{t0}, {t0 + S}) do not fit a buffer of {cap}")
    _expect_shape("dst_packed", dst[0], (B, H, cap, D * bits // 32))
    _expect_shape("dst_scales", dst[1], (B, H, cap, D // group_size))
    _expect_shape("dst_biases", dst[2], (B, H, cap, D // group_size))
    if dst[0].dtype != torch.uint32 or dst[1].dtype != src.dtype or dst[2].dtype != src.dtype:
        raise ValueError("destination dtypes must be (uint32, src.dtype, src.dtype)")
    # (the caller keeps `src` alive until the launch is queued)
    return src, _lib.QuantizeArgs(B, H, S, D, bits, group_size, dtype_code(src.dtype), int(t0),
                                  _view(src), _view(dst[0]), _view(dst[1]), _view(dst[2]))


def quantize_into(src: torch.Tensor, dst: tuple, t0: int, bits: int, group_size: int) -> None:
    """dst[b, h, t0 + s, :] = quantize(src[b, h, s, :]) for the 3 dst tensors."""
    src, a = _quantize_args(src, dst, t0, bits, group_size)
    _lib.check(_lib.load().qsdpa_quantize(ctypes.byref(a), _stream(src)))


def quantize_kv_into(keys: torch.Tensor, values: torch.Tensor, kdst: tuple, vdst: tuple, t0: int,
                     bits: int, group_size: int) -> None:
    """quantize_into for the keys and the values of one cache update, in one launch."""
    if keys.dtype != values.dtype:
        raise ValueError("keys and values must share a dtype")
    keys, ka = _quantize_args(keys, kdst, t0, bits, group_size)
    values, va = _quantize_args(values, vdst, t0, bits, group_size)
    jobs = (_lib.QuantizeArgs * 2)(ka, va)
    _lib.check(_lib.load().qsdpa_quantize_batch(jobs, 2, _stream(keys)))


def quantize(w: torch.Tensor, group_size: int = 64, bits: int = 4):
    """mx.quantize for [..., D] float16/bfloat16 tensors -> (packed, scales, biases)."""
    if w.dim() < 1:
        raise ValueError("w must have at least one dimension")
    shape = w.shape
    D = shape[-1]
    if D % group_size:
        raise ValueError(f"last dim {D} not divisible by group_size {group_size}")
    if bits not in (4, 8):
        raise ValueError(f"bits must be 4 or 8, got {bits}")
    w4 = w.reshape(1, 1, -1, D)
    rows = w4.shape[2]
    packed = torch.empty((1, 1, rows, D * bits // 32), dtype=torch.uint32, device=w.device)
    scales = torch.empty((1, 1, rows, D // group_size), dtype=w.dtype, device=w.device)
    biases = torch.empty_like(scales)
    quantize_into(w4, (packed, scales, biases), 0, bits, group_size)
    return (packed.reshape(*shape[:-1], -1), scales.reshape(*shape[:-1], -1),
            biases.reshape(*shape[:-1], -1))


def dequantize_into(src: tuple, dst: torch.Tensor, bits: int, group_size: int,
                    keep: int = 0, rot: int = 0) -> None:
    """dst = dequantize(src) with the ring reorder described in qsdpa.h."""
    packed, scales, biases = src
    _require_device(packed, scales, biases, dst)
    B, H, N, W = packed.shape
    D = dst.shape[-1]
    if bits not in (4, 8) or W * (32 // bits) != D or D % group_size:
        raise ValueError(f"packed width {W} does not match D={D}, bits={bits}, gs={group_size}")
    if packed.dtype != torch.uint32:
        raise ValueError("packed must be uint32")
    _expect_shape("scales", scales, (B, H, N, D // group_size))
    _expect_shape("biases", biases, (B, H, N, D // group_size))
    _expect_shape("dst", dst, (B, H, N, D))
    if not 0 <= keep <= N or rot < 0 or (rot > 0 and keep >= N):
        raise ValueError(f"bad keep={keep} / rot={rot} for N={N}")
    a = _lib.DequantizeArgs(B, H, N, D, bits, group_size, dtype_code(dst.dtype), int(keep),
                            int(rot), _view(packed), _view(scales), _view(biases), _view(dst))
    _lib.check(_lib.load().qsdpa_dequantize(ctypes.byref(a), _stream(dst)))


def requant_window(old: tuple, new: tuple, dst: tuple, n_old: int, keep: int, rot: int,
                   max_size: int, bits: int, group_size: int) -> int:
    """A rotating window's prefill in one launch for K and V (qsdpa.h:
    qsdpa_requant_window): the old window (ring order `keep` / `rot`, its
    first n_old rows) in temporal order, then the new tokens, trimmed to the
    first `keep` and the newest max_size - keep, quantized again into rows
    [0, total) of `dst`.  old / dst: ((packed, scales, biases) of K, of V);
    new: (keys, values) [B, H, S, D].  Returns total."""
    keys, values = (_inner_contig(x) for x in new)
    _require_device(keys, values, *dst[0], *dst[1], *(t for tup in old for t in tup))
    if keys.dtype != values.dtype:
        raise ValueError("keys and values must share a dtype")
    B, H, S, D = keys.shape
    if bits not in (4, 8) or D % group_size:
        raise ValueError(f"bad bits={bits} / group_size={group_size} for D={D}")
    if not (0 <= keep < max_size and 0 <= n_old <= max_size and rot >= 0 and (rot == 0 or n_old > keep)):
        raise ValueError(f"bad window: max_size={max_size} keep={keep} n_old={n_old} rot={rot}")
    total = min(n_old + S, max_size)
    jobs = (_lib.RequantArgs * 2)()
    for j, (o, x, d) in enumerate(zip(old, (keys, values), dst)):
        if d[0].shape[2] < total or (n_old and o[0].shape[2] < n_old):
            raise ValueError("window buffers too short")
        if n_old and d[0].data_ptr() == o[0].data_ptr():
            raise ValueError("the destination must not be the old window")
        jobs[j] = _lib.RequantArgs(B, H, D, bits, group_size, dtype_code(keys.dtype), int(n_old), int(keep),
                                   int(rot), S, int(max_size), _view(o[0]), _view(o[1]), _view(o[2]),
                                   _view(x), _view(d[0]), _view(d[1]), _view(d[2]))
    _lib.check(_lib.load().qsdpa_requant_window(jobs, 2, _stream(keys)))
    return total


class RowMove(NamedTuple):
    """Fill token columns [dst_col, dst_col + tokens) of batch row `dst_row` of
    a (B, H, N, W) buffer, every head: the columns dst_col + [copy_begin,
    copy_end) from `src` (batch row `src_row`, starting at column `src_col`),
    the others with zeros (all of them when src is None)."""
    dst: torch.Tensor
    dst_row: int
    dst_col: int
    tokens: int
    src: Optional[torch.Tensor] = None
    src_row: int = 0
    src_col: int = 0
    copy_begin: int = 0
    copy_end: int = 0


def _check_rows(name, t, row, col, n):
    if t.dim() != 4 or (t.shape[3] > 1 and t.stride(3) != 1):
        raise ValueError(f"{name}: expected a (B, H, N, W) tensor with contiguous W, got {tuple(t.shape)}")
    if not (0 <= row < t.shape[0] and 0 <= col and col + n <= t.shape[2]):
        raise ValueError(f"{name}: rows {row}, columns [{col}, {col + n}) outside shape {tuple(t.shape)}")


def move_rows(moves) -> None:
    """Run RowMoves with qsdpa_move_rows (kernel-argument descriptors, one
    launch per 48 moves, no synchronization).  Bounds, dtypes, head counts
    and row widths are checked here; no destination may overlap another
    destination or a source of the same call."""
    moves = [m for m in moves if m.tokens > 0 and m.dst.shape[1] > 0]
    if not moves:
        return
    dev = moves[0].dst.device
    _require_device(*(m.dst for m in moves), *(m.src for m in moves))
    arr = (_lib.RowMove * len(moves))()
    for i, m in enumerate(moves):
        d = m.dst
        _check_rows("dst", d, m.dst_row, m.dst_col, m.tokens)
        if d.device != dev:
            raise ValueError("all moves of one call must be on one device")
        es = d.element_size()
        dst_ptr = d.data_ptr() + (m.dst_row * d.stride(0) + m.dst_col * d.stride(2)) * es
        src_ptr, shs, sts, lo, hi = None, 0, 0, 0, 0
        if m.src is not None and m.copy_end > m.copy_begin:
            s = m.src
            lo, hi = int(m.copy_begin), int(m.copy_end)
            if not 0 <= lo < hi <= m.tokens:
                raise ValueError(f"copy range [{lo}, {hi}) outside [0, {m.tokens})")
            _check_rows("src", s, m.src_row, m.src_col, hi - lo)
            if s.dtype != d.dtype or s.shape[1] != d.shape[1] or s.shape[3] != d.shape[3] or s.device != dev:
                raise ValueError(f"src {tuple(s.shape)} {s.dtype} does not match dst {tuple(d.shape)} {d.dtype}")
            src_ptr = s.data_ptr() + (m.src_row * s.stride(0) + m.src_col * s.stride(2)) * es
            shs, sts = s.stride(1) * es, s.stride(2) * es
        arr[i] = _lib.RowMove(src_ptr, dst_ptr, shs, sts, d.stride(1) * es, d.stride(2) * es,
                              d.shape[1], int(m.tokens), d.shape[3] * es, lo, hi)
    _lib.check(_lib.load().qsdpa_move_rows(arr, len(moves), _stream(moves[0].dst)))


def dequantize(packed: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor | None = None,
               group_size: int = 64, bits: int = 4, keep: int = 0, rot: int = 0):
    """mx.dequantize for [..., N, W] packed tensors (biases None = zero)."""
    lead = packed.shape[:-1]
    D = packed.shape[-1] * (32 // bits)
    p4 = packed.reshape(-1, 1, packed.shape[-2] if packed.dim() > 1 else 1, packed.shape[-1])
    s4 = scales.reshape(p4.shape[0], 1, p4.shape[2], scales.shape[-1])
    b4 = None if biases is None else biases.reshape(p4.shape[0], 1, p4.shape[2], biases.shape[-1])
    out = torch.empty((p4.shape[0], 1, p4.shape[2], D), dtype=scales.dtype, device=packed.device)
    dequantize_into((p4, s4, b4), out, bits, group_size, keep, rot)
    return out.reshape(*lead, D)


# ---------------------------------------------------------------------------
# decode
# ---------------------------------------------------------------------------
def _decode_args(q, pk, pv, ks, vs, kb, vb, out, scale, bits, group_size, mask, kv_start,
                 num_splits, causal=False, append=None):
    B, Hq, qL, D = q.shape
    _, Hkv, N, _ = pk.shape
    if qL < 1:
        raise ValueError("q must hold at least one query position")
    if bits not in (4, 8) or D % group_size:
        raise ValueError(f"bad bits={bits} / group_size={group_size} for D={D}")
    for name, t, inner, dt in (("packed_k", pk, D * bits // 32, torch.uint32),
                               ("packed_v", pv, D * bits // 32, torch.uint32),
                               ("k_scales", ks, D // group_size, q.dtype),
                               ("v_scales", vs, D // group_size, q.dtype),
                               ("k_biases", kb, D // group_size, q.dtype),
                               ("v_biases", vb, D // group_size, q.dtype)):
        _expect_shape(name, t, (B, Hkv, N, inner))
        if t is not None and t.dtype != dt:
            raise ValueError(f"{name}: dtype {t.dtype}, expected {dt}")
    _expect_shape("out", out, (B, Hq, qL, D))
    if kv_start is not None and tuple(kv_start.shape) != (B,):
        raise ValueError(f"kv_start must have shape ({B},)")
    mview = _lib.View(None, 0, 0, 0)
    mcode = 0
    mask_sq = 0
    if mask is not None:
        if mask.dtype not in _MASK_CODE:
            raise ValueError(f"unsupported mask dtype {mask.dtype}")
        m = mask
        while m.dim() < 4:
            m = m.unsqueeze(0)
        if m.shape[-1] != N:
            raise ValueError(f"mask last dim {m.shape[-1]} != number of keys {N}")
        if m.shape[-2] not in (1, qL):
            raise ValueError(f"mask query dim {m.shape[-2]} must be 1 or {qL}")
        m = m.expand(B, Hq, m.shape[-2], N)
        if m.stride(-1) != 1:
            m = m.contiguous()
        if m.dtype == torch.bool:
            m = m.view(torch.uint8)
        s = m.stride()
        mview = _lib.View(m.data_ptr(), s[0], s[1], s[3])
        mask_sq = s[2] if m.shape[-2] > 1 else 0
        mcode = _MASK_CODE[mask.dtype]
        mask = m
    ks_ptr = None
    if kv_start is not None:
        ks_t = kv_start
        ks_ptr = ks_t.data_ptr()
    a = _lib.DecodeArgs()
    a.B, a.H_q, a.H_kv, a.N, a.D = B, Hq, Hkv, N, D
    a.bits, a.group_size, a.dtype = bits, group_size, dtype_code(q.dtype)
    a.scale = float(scale)
    a.q = _view(q)
    a.k_packed, a.v_packed = _view(pk), _view(pv)
    a.k_scales, a.v_scales = _view(ks), _view(vs)
    a.k_biases, a.v_biases = _view(kb), _view(vb)
    a.out = _view(out)
    a.mask, a.mask_dtype = mview, mcode
    a.kv_start = ks_ptr
    a.num_splits = int(num_splits)
    a.q_len = qL
    a.causal = int(bool(causal))
    if append is not None:
        k_new, v_new = append
        if kb is None or vb is None:
            raise ValueError("an append writes biases: the cache views must carry k / v biases")
        for name, t in (("k_new", k_new), ("v_new", v_new)):
            _expect_shape(name, t, (B, Hkv, 1, D))
            if t.dtype != q.dtype or t.device != q.device or t.stride(-1) != 1:
                raise ValueError(f"{name}: expected a {q.dtype} tensor on {q.device} with contiguous rows")
        a.k_new, a.v_new = _view(k_new), _view(v_new)
    a.mask_stride_q = mask_sq
    return a, mask


def decode_plan(q, pk, pv, ks, vs, kb, vb, *, scale, bits, group_size, num_splits=0):
    """(num_splits, workspace_bytes) the library would use for these inputs.

    Raises QsdpaError (code QSDPA_ERR_UNSUPPORTED) for inputs no kernel takes."""
    out = torch.empty_like(q)
    a, _ = _decode_args(q, pk, pv, ks, vs, kb, vb, out, scale, bits, group_size, None, None,
                        num_splits)
    n = ctypes.c_int32(0)
    ws = _lib.check(_lib.load().qsdpa_decode_workspace_size(ctypes.byref(a), ctypes.byref(n)))
    return int(n.value), int(ws)


class DecodePlan:
    """A decode whose argument block is built once and re-launched cheaply.

    For tight decode loops (and the benchmark): the output and workspace are
    allocated at construction; each call re-issues the same launch on the
    current stream of the inputs' device with one ctypes call.  The caller
    updates the input tensors in place between calls.
    """

    def __init__(self, q, pk, pv, ks, vs, kb, vb, *, scale, bits, group_size, mask=None,
                 kv_start=None, num_splits=0, capacity=None, causal=False, append=None):
        """append: optional (k_new, v_new), [B, H_kv, 1, D] tensors of q's
        dtype, whose rows every call first quantizes into key N - 1 of the
        caches (the one-token update of a decode step, in the same launch
        where the kernel takes it: qsdpa_decode_args.k_new).  The caller
        writes the new token into them and moves N past it (set_keys) before
        each call."""
        # Rows set_keys may reach: the views' own length unless the caller
        # states how many rows the underlying buffers hold, never more than
        # every buffer's storage holds, and never past a mask's last key.
        n0 = int(pk.shape[2])
        self.capacity = int(capacity) if capacity is not None else n0
        if self.capacity < n0:
            raise ValueError(f"capacity {self.capacity} is below the views' {n0} keys")
        if self.capacity > n0:
            if mask is not None:
                raise ValueError("a mask covers the construction-time keys only: give capacity "
                                 "without a mask, or build a new plan per mask")
            for name, t in (("packed_k", pk), ("packed_v", pv), ("k_scales", ks), ("v_scales", vs),
                            ("k_biases", kb), ("v_biases", vb)):
                if t is not None and _rows_in_storage(t) < self.capacity:
                    raise ValueError(f"{name}: its storage holds {_rows_in_storage(t)} rows, "
                                     f"fewer than capacity {self.capacity}")
        _require_device(q, pk, pv, ks, vs, kb, vb, mask, kv_start, *(append or ()))
        self.q = _inner_contig(q)
        self.out = torch.empty(q.shape, dtype=q.dtype, device=q.device)
        if kv_start is not None:
            kv_start = kv_start.to(device=q.device, dtype=torch.int32).contiguous()
        self._refs = (pk, pv, ks, vs, kb, vb, kv_start, append)
        self.args, self._mask = _decode_args(self.q, pk, pv, ks, vs, kb, vb, self.out, scale, bits,
                                             group_size, mask, kv_start, num_splits, causal, append)
        self.lib = _lib.load()
        n = ctypes.c_int32(0)
        ws = _lib.check(self.lib.qsdpa_decode_workspace_size(ctypes.byref(self.args),
                                                             ctypes.byref(n)))
        self.num_splits = int(n.value)
        self.workspace = None
        if ws > 0:
            # Zero-filled: the split merge's counters at its start must be
            # zero before the first call (each call leaves them zero).
            self.workspace = torch.zeros(ws, dtype=torch.uint8, device=q.device)
            self.args.workspace = self.workspace.data_ptr()
            self.args.workspace_bytes = ws
        self._args_ref = ctypes.byref(self.args)
        self.device = q.device
        self.args.num_splits = self.num_splits  # fixed from here on (set_keys)

    def set_keys(self, n: int) -> None:
        """Re-target the plan to the first n keys of the same buffers (a cache
        that grew in place); the split count chosen at construction is kept."""
        if not 1 <= n <= self.capacity:
            raise ValueError(f"n={n} outside [1, {self.capacity}]")
        self.args.N = int(n)

    def __call__(self, prof_events=None):
        if prof_events is not None:
            self.args.prof_begin, self.args.prof_end = prof_events
        else:
            self.args.prof_begin = self.args.prof_end = None
        _lib.check(self.lib.qsdpa_decode(self._args_ref, _stream(self.q)))
        return self.out


# Argument blocks of recent decode calls, per thread: a call whose tensors
# have the geometry of an earlier one -- shapes except the key count, strides,
# dtypes, pointer alignments, the same scalars and stream -- re-uses that call's validated
# argument block and workspace, rewriting only the data pointers and the key
# count (a decode loop over a growing cache hits every step).  The workspace
# is re-used in the order of the stream it was cached for, so it never races.
_ARGS = threading.local()
_ARGS_MAX = 32


def _cache_key(q, pk, pv, ks, vs, kb, vb, kv_start, scale, bits, group_size, num_splits, causal, stream):
    """The argument block's key: everything the block encodes except the key
    count N and the data pointers (but with each pointer's offset from a
    16-byte boundary), plus the device and stream, or None when
    the tensors disagree with one another (the full path then raises).  pv
    must have pk's shape, the scales and biases one shape with pk's (B, H,
    N)."""
    sk, ss = pk.shape, ks.shape
    if pv.shape != sk or vs.shape != ss or ss[:3] != sk[:3] or (kb is not None and kb.shape != ss) \
            or (vb is not None and vb.shape != ss):
        return None
    # The plan (kernel, split count, workspace size) also depends on each
    # pointer's alignment: a view 2 bytes off its allocation's start can
    # take another kernel.
    align = tuple(None if t is None else t.data_ptr() % 16 for t in (q, pk, pv, ks, vs, kb, vb))
    return (q.shape, q.stride(), q.dtype, sk[0], sk[1], sk[3], pk.dtype, pv.dtype, pk.stride(), pv.stride(), ss[3],
            ks.dtype, vs.dtype, ks.stride(), vs.stride(), None if kb is None else (kb.dtype, kb.stride()),
            None if vb is None else (vb.dtype, vb.stride()), None if kv_start is None else kv_start.shape,
            float(scale), bits, group_size, int(num_splits), bool(causal), q.get_device(), stream, align)


def _cached_decode(q, pk, pv, ks, vs, kb, vb, scale, bits, group_size, kv_start, num_splits,
                   causal, prof_events):
    """The decode through a cached argument block; (None, slot) when this
    geometry has not been seen (the caller then takes the full path and
    stores its block in `slot`), (None, None) when it cannot be cached."""
    if not q.is_cuda:
        return None, None
    stream = _stream(q)
    key = _cache_key(q, pk, pv, ks, vs, kb, vb, kv_start, scale, bits, group_size, num_splits, causal, stream)
    if key is None:
        return None, None  # inconsistent shapes: the full path raises
    cache = getattr(_ARGS, "d", None)
    if cache is None:
        cache = _ARGS.d = {}
    hit = cache.get(key)
    if hit is None:
        return None, (cache, key)
    a = hit[0]
    lib = _lib.load()
    N = pk.shape[2]
    a.q.ptr = q.data_ptr()
    a.k_packed.ptr, a.v_packed.ptr = pk.data_ptr(), pv.data_ptr()
    a.k_scales.ptr, a.v_scales.ptr = ks.data_ptr(), vs.data_ptr()
    a.k_biases.ptr = None if kb is None else kb.data_ptr()
    a.v_biases.ptr = None if vb is None else vb.data_ptr()
    a.kv_start = None if kv_start is None else kv_start.data_ptr()
    if N != hit[2]:  # the workspace depends on the geometry and N alone
        a.N = N
        ws = _lib.check(lib.qsdpa_decode_workspace_size(ctypes.byref(a), None))
        if ws > a.workspace_bytes:
            hit[1] = torch.zeros(ws, dtype=torch.uint8, device=q.device)
            a.workspace, a.workspace_bytes = hit[1].data_ptr(), ws
        hit[2] = N
    out = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    a.out.ptr = out.data_ptr()
    a.prof_begin, a.prof_end = prof_events if prof_events is not None else (None, None)
    _lib.check(lib.qsdpa_decode(ctypes.byref(a), stream))
    return out, None


def decode_repeat(q, pk, pv, ks, vs, kb, vb, *, scale, bits, group_size):
    """A decode (no mask, kv_start or explicit split count) that repeats an
    earlier call's geometry, through its argument block; None when there is
    no such block or a packed row is not 16-byte aligned (the caller then
    takes the full path).  Every tensor must be on the GPU (checked)."""
    if q.is_cuda and pk.is_cuda and pv.is_cuda and ks.is_cuda and vs.is_cuda and (kb is None or kb.is_cuda) \
            and (vb is None or vb.is_cuda) and q.stride(-1) == 1 and not (pk.data_ptr() | pv.data_ptr()) & 15:
        out, _ = _cached_decode(q, pk, pv, ks, vs, kb, vb, scale, bits, group_size, None, 0, False, None)
        return out
    return None


# Split-K workspaces of uncached decode calls, one per (device, stream): the
# calls of a stream run in order, so they can share one buffer, zero-filled
# once (the split merge's counters at its start are zero between calls).
_WORKSPACES = {}


def _stream_workspace(device, stream, nbytes):
    key = (device.index, stream)
    ws = _WORKSPACES.get(key)
    if ws is None or ws.numel() < nbytes:
        ws = torch.zeros(nbytes, dtype=torch.uint8, device=device)
        _WORKSPACES[key] = ws
    return ws


def decode(q, pk, pv, ks, vs, kb, vb, *, scale, bits, group_size, mask=None, kv_start=None,
           num_splits=0, out=None, workspace=None, prof_events=None, causal=False, append=None):
    """Fused quantized attention; returns out [B, H_q, qL, D] (dtype of q).

    qL > 1 query positions (speculative or chunked decoding, prefill) run on
    the matrix-core kernel; ``causal`` aligns the causal mask to the last
    key (query i sees keys t <= N - qL + i).

    ``prof_events``: optional (begin, end) raw hipEvent_t handles recorded
    around the main decode kernel (see qsdpa_decode_args.prof_begin).

    Without a mask, ``out`` or ``workspace``, a call that repeats an earlier
    call's tensor geometry re-launches that call's argument block.  A
    caller's ``workspace`` (uint8, at least qsdpa_decode_workspace_size
    bytes) must be zero-filled before its first use; the library leaves the
    counters at its start zero after every call, so it can be re-used.

    ``append``: optional (k_new, v_new) [B, H_kv, 1, D] rows quantized into
    key N - 1 of the caches before the attention (see DecodePlan).
    """
    _require_device(q, pk, pv, ks, vs, kb, vb, mask, kv_start, *(append or ()))
    slot = None
    if mask is None and out is None and workspace is None and append is None:
        q = _inner_contig(q)
        if kv_start is not None and (kv_start.dtype != torch.int32 or kv_start.device != q.device
                                     or not kv_start.is_contiguous()):
            kv_start = kv_start.to(device=q.device, dtype=torch.int32).contiguous()
        res, slot = _cached_decode(q, pk, pv, ks, vs, kb, vb, scale, bits, group_size, kv_start,
                                   num_splits, causal, prof_events)
        if res is not None:
            return res
    q = _inner_contig(q)
    if out is None:
        out = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    if kv_start is not None:
        kv_start = kv_start.to(device=q.device, dtype=torch.int32).contiguous()
    a, keep_alive = _decode_args(q, pk, pv, ks, vs, kb, vb, out, scale, bits, group_size, mask,
                                 kv_start, num_splits, causal, append)
    lib = _lib.load()
    n = ctypes.c_int32(0)
    ws = _lib.check(lib.qsdpa_decode_workspace_size(ctypes.byref(a), ctypes.byref(n)))
    if ws > 0:
        if workspace is None or workspace.numel() < ws:
            workspace = _stream_workspace(q.device, _stream(q), ws)
        a.workspace = workspace.data_ptr()
        a.workspace_bytes = ws
    if prof_events is not None:
        a.prof_begin, a.prof_end = prof_events
    _lib.check(lib.qsdpa_decode(ctypes.byref(a), _stream(q)))
    del keep_alive
    if slot is not None:
        cache, key = slot
        if len(cache) >= _ARGS_MAX:
            cache.pop(next(iter(cache)))
        if ws <= 0:
            a.workspace, a.workspace_bytes, workspace = None, 0, None
        cache[key] = [a, workspace, a.N]
    return out
