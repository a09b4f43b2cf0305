"""Batch administration on the GPU (qsdpa_move_rows).

* The row-move kernel itself: random moves over buffers of every unit
  width (16 / 8 / 4 / 2 / 1-byte aligned rows and views), zero moves, copy
  ranges with zero margins and more moves than one launch carries, against
  the same moves done by torch slicing on CPU copies.
* finalize / filter / extend / extract / merge of both batch caches on the
  HIP kernels, bit-exact against the oracle caches after every step (whole
  buffers and counters; tests/admin_scenarios.py), each administration call
  and update under torch.cuda.set_sync_debug_mode("error").
* A 48-sequence merge, filter and extend (several launches per call).
* The reference's own expectations for these methods
  (tests/golden/reference_fixtures.json: tests/test_cache.py:264-288,
  tests/test_batch_rotating_cache.py:57-181).
"""

import json

import numpy as np
import pytest
import torch

from admin_scenarios import (BATCH_SCENARIOS, ROTATING_SCENARIOS, Pair, batch_scenario, check_sequences,
                             no_sync, rotating_scenario, sequences)
from conftest import GOLDEN, _cpu_move_rows, from_np, to_np
from oracle import affine
from oracle import caches as oc

import mlx_qsdpa_amd.cache as pc
from mlx_qsdpa_amd import kernels

pytestmark = pytest.mark.gpu

REF = json.loads((GOLDEN / "reference_fixtures.json").read_text())


def _disjoint_moves(rng, dst, srcs):
    """RowMoves that fill disjoint column spans of every row of `dst`: zero
    moves, and copies from the `srcs` with random copy ranges inside."""
    B, _, N, _ = dst.shape
    moves = []
    for row in range(B):
        col = int(rng.integers(0, 3))
        while True:
            n = int(rng.integers(1, 7))
            if col + n > N:
                break
            if rng.random() < 0.2:
                moves.append(kernels.RowMove(dst, row, col, n))
            else:
                s = srcs[int(rng.integers(len(srcs)))]
                lo = int(rng.integers(0, n + 1))
                hi = int(rng.integers(lo, n + 1))
                scol = int(rng.integers(0, s.shape[2] - (hi - lo) + 1))
                moves.append(kernels.RowMove(dst, row, col, n, s, int(rng.integers(s.shape[0])), scol, lo, hi))
            col += n + int(rng.integers(0, 3))
    return moves


@pytest.mark.parametrize("dtype,width,offset", [
    (torch.int32, 8, 0),      # 32-byte rows: 16-byte units
    (torch.int32, 2, 1),      # 8-byte rows at a 4-byte offset: 4-byte units
    (torch.float16, 4, 0),    # 8-byte rows: 8-byte units
    (torch.bfloat16, 1, 3),   # 2-byte rows
    (torch.uint8, 3, 1),      # 3-byte rows: 1-byte units
])
def test_move_rows_matches_slicing(device, dtype, width, offset):
    rng = np.random.default_rng(width * 10 + offset)
    shape = (8, 3, 37, width)
    # Views that start `offset` elements into their storage (unaligned bases).
    host = []
    for _ in range(3):
        flat = torch.randint(0, 120, (offset + int(np.prod(shape)),), dtype=torch.int32).to(dtype)
        host.append(flat[offset:].view(shape))
    dev = [h.to(device) for h in host]
    for di in range(3):
        others = [i for i in range(3) if i != di]
        moves = _disjoint_moves(rng, host[di], [host[i] for i in others])
        assert len(moves) > 48  # more than one launch
        to_dev = {id(h): d for h, d in zip(host, dev)}
        moves_d = [m._replace(dst=to_dev[id(m.dst)], src=None if m.src is None else to_dev[id(m.src)])
                   for m in moves]
        print(f"move_rows {dtype} width={width} offset={offset} dst={di}: {len(moves)} moves", flush=True)
        _cpu_move_rows(moves)
        kernels.move_rows(moves_d)
        torch.cuda.synchronize()
        for i, (h, d) in enumerate(zip(host, dev)):
            assert torch.equal(d.cpu().view(torch.uint8), h.view(torch.uint8)), f"dst {di}: buffer {i} differs"


def test_sync_guard_detects_host_reads(device):
    """The guard the scenarios run under does catch a device-to-host read."""
    x = torch.ones(4, device=device)
    with pytest.raises(RuntimeError):
        with no_sync(device):
            x.sum().item()


def test_move_rows_rejects_bad_moves(device):
    a = torch.zeros((2, 2, 8, 4), dtype=torch.uint32, device=device)
    b = torch.zeros((2, 2, 8, 4), dtype=torch.float16, device=device)
    with pytest.raises(ValueError):
        kernels.move_rows([kernels.RowMove(a, 0, 6, 3)])  # past the last column
    with pytest.raises(ValueError):
        kernels.move_rows([kernels.RowMove(a, 2, 0, 1)])  # no row 2
    with pytest.raises(ValueError):
        kernels.move_rows([kernels.RowMove(a, 0, 0, 4, b, 0, 0, 0, 4)])  # dtype mismatch
    with pytest.raises(ValueError):
        kernels.move_rows([kernels.RowMove(a, 0, 0, 4, a[:, :1], 0, 0, 0, 4)])  # head mismatch


@pytest.mark.parametrize("bits,gs,dtype", [(4, 32, "f16"), (8, 64, "bf16")])
@pytest.mark.parametrize("name", BATCH_SCENARIOS)
def test_batch_admin_bit_exact(device, name, bits, gs, dtype):
    print(f"batch {name} bits={bits} gs={gs} {dtype}", flush=True)
    batch_scenario(name, bits=bits, gs=gs, dtype=dtype, device=device, seed=3)


@pytest.mark.parametrize("keep", [0, 2])
@pytest.mark.parametrize("name", ROTATING_SCENARIOS)
def test_rotating_batch_admin_bit_exact(device, name, keep):
    print(f"rotating {name} keep={keep}", flush=True)
    rotating_scenario(name, max_size=8, keep=keep, bits=4, gs=32, dtype="f16", device=device, seed=4)
    rotating_scenario(name, max_size=16, keep=keep, bits=8, gs=32, dtype="bf16", device=device, seed=5)


def test_many_sequences(device):
    """48 single caches merged (several launches per call), filtered to a
    random subset in a new order, extended by a second merged batch."""
    rng = np.random.default_rng(6)
    dtype, bits, gs = "bf16", 4, 64

    def singles(lengths):
        out = []
        for n in lengths:
            s = Pair(pc.QuantizedSDPACache(bits=bits, group_size=gs),
                     oc.QuantizedSDPACache(bits=bits, group_size=gs, dtype=dtype), dtype, device, rng)
            s.update(1, int(n), f"single {n}")
            out.append(s)
        return out

    def merged(ss):
        with no_sync(device):
            p = pc.BatchQuantizedSDPACache.merge([s.p for s in ss])
        x = Pair(p, oc.BatchQuantizedSDPACache.merge([s.o for s in ss]), dtype, device, rng)
        x.check("merge")
        return x

    x = merged(singles(rng.integers(1, 300, size=48)))
    x.update(48, 1, "decode")
    keep = rng.permutation(48)[:29]
    before = sequences(x.o)
    with no_sync(device):
        x.p.filter(keep.tolist())
    x.o.filter(keep)
    x.check("filter")
    check_sequences(sequences(x.p), [before[i] for i in keep], "bf16", "filter")
    y = merged(singles(rng.integers(1, 500, size=7)))
    with no_sync(device):
        x.p.extend(y.p)
    x.o.extend(y.o)
    x.check("extend")
    x.update(36, 1, "decode after extend")


# ---- the reference's expectations ------------------------------------------
def _kv(rng, B, S, Hkv=2, D_=64):
    k = affine.random_T(rng, (B, Hkv, S, D_), "f16")
    v = affine.random_T(rng, (B, Hkv, S, D_), "f16")
    return k, v


def test_reference_cache_merge_extract(device):
    """tests/test_cache.py:264-288."""
    g = REF["cache_merge_extract"]
    rng = np.random.default_rng(7)
    cs, raw = [], []
    for n in g["lengths"]:
        c = pc.QuantizedSDPACache(bits=4, group_size=32)
        k, v = _kv(rng, 1, n, D_=256)
        c.update_and_fetch(from_np(k, torch.float16, device), from_np(v, torch.float16, device))
        cs.append(c)
        raw.append(k)
    b = pc.QuantizedSDPACache.merge(cs)
    st = b.state
    assert st[2].shape[0] == g["state_batch"] and st[3].shape[0] == g["state_batch"]
    assert [b.extract(i).offset for i in range(2)] == g["extract_offsets"]
    for i, k in enumerate(raw):
        packed = to_np(b.extract(i).state[0][0])
        assert np.array_equal(packed, affine.quantize(k, 32, 4, "f16")[0])


def _decode_n(cache, rng, n, B=1, Hkv=2, device=None):
    keys = []
    for _ in range(n):
        k, v = _kv(rng, B, 1, Hkv)
        keys.append(k)
        cache.update_and_fetch(from_np(k, torch.float16, device), from_np(v, torch.float16, device))
    return keys


def test_reference_batch_rotating_admin(device):
    """tests/test_batch_rotating_cache.py:57-181: filter, extract, merge,
    extract after a wrap (== quantize of the last 4 keys)."""
    rng = np.random.default_rng(8)
    g = REF["batch_rotating_filter"]
    c = pc.BatchQuantizedRotatingSDPACache([0, 0], max_size=g["max_size"], bits=4, group_size=32)
    _decode_n(c, rng, g["decodes"], B=2, device=device)
    c.filter(torch.tensor(g["keep_index"]))
    assert c._keys[0].shape[0] == g["B_after"] and c.offset.shape[0] == g["B_after"]
    g = REF["batch_rotating_extract"]
    c = pc.BatchQuantizedRotatingSDPACache([0, 0], max_size=g["max_size"], bits=4, group_size=32)
    _decode_n(c, rng, g["decodes"], B=2, device=device)
    e = c.extract(0)
    assert isinstance(e, pc.QuantizedRotatingSDPACache)
    assert e.offset == g["offset"] and e.max_size == g["max_size"]
    singles = []
    for n in (3, 5):
        s = pc.QuantizedRotatingSDPACache(max_size=16, bits=4, group_size=32)
        _decode_n(s, rng, n, device=device)
        singles.append(s)
    b = pc.BatchQuantizedRotatingSDPACache.merge(singles)
    assert b._keys[0].shape[0] == 2 and b.max_size == 16
    g = REF["batch_rotating_extract_after_wrap"]
    c = pc.BatchQuantizedRotatingSDPACache([0], max_size=g["max_size"], bits=4, group_size=32)
    keys = _decode_n(c, rng, g["decodes"], Hkv=1, device=device)
    e = c.extract(0)
    want = affine.quantize(np.concatenate(keys[-g["last"]:], axis=2), 32, 4, "f16")[0]
    assert e.offset == g["offset"]
    assert np.array_equal(to_np(e.state[0][0]), want)
