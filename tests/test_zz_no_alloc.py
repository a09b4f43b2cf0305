"""qsdpa_decode_noalloc against qsdpa_decode, through the C ABI.

The allocation-free entry point keeps the split-K partials in a static
device array (the last call's contents stay there), so it is called several
times in a row, a larger input first and a smaller one after it, and each
output must equal qsdpa_decode's on the same inputs bit for bit (the same
kernels on the same partial layout) and lie within the parity tolerance of
the oracle.  Arguments whose partials exceed the static array are refused
with QSDPA_ERR_WORKSPACE.
"""

import ctypes

import numpy as np
import pytest
import torch

from conftest import from_np, torch_dtype
from oracle import affine, attention

from mlx_qsdpa_amd import _lib, kernels

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-3, 1e-2


def _inputs(rng, B, Hq, Hkv, N, D, bits, gs, dt, device, qL=1):
    T = torch_dtype(dt)
    q = affine.random_T(rng, (B, Hq, qL, D), dt)
    kq = affine.quantize(affine.random_T(rng, (B, Hkv, N, D), dt), gs, bits, dt)
    vq = affine.quantize(affine.random_T(rng, (B, Hkv, N, D), dt), gs, bits, dt)
    dev = lambda x: from_np(x, T, device)  # noqa: E731  (uint32 arrays keep their type)
    return (q, kq, vq), (dev(q), tuple(map(dev, kq)), tuple(map(dev, vq)))


def _run_both(host, devt, bits, gs, dt, kv_start=None, num_splits=0, causal=False):
    """qsdpa_decode (with a workspace) and qsdpa_decode_noalloc on the same
    inputs; returns both outputs and the split count."""
    lib = _lib.load()
    q, kq, vq = devt
    D = q.shape[-1]
    outs = []
    for noalloc in (False, True):
        out = torch.full_like(q, float("nan"))
        a, keep = kernels._decode_args(q, kq[0], vq[0], kq[1], vq[1], kq[2], vq[2], out, D ** -0.5, bits, gs,
                                       None, kv_start, num_splits, causal=causal)
        n = ctypes.c_int32(0)
        ws = _lib.check(lib.qsdpa_decode_workspace_size(ctypes.byref(a), ctypes.byref(n)))
        stream = torch.cuda.current_stream(q.device).cuda_stream
        if noalloc:
            _lib.check(lib.qsdpa_decode_noalloc(ctypes.byref(a), stream))
        else:
            wsbuf = torch.zeros(max(ws, 1), dtype=torch.uint8, device=q.device)  # zero-filled before first use
            a.workspace, a.workspace_bytes = wsbuf.data_ptr(), ws
            _lib.check(lib.qsdpa_decode(ctypes.byref(a), stream))
        torch.cuda.synchronize()
        outs.append(out.float().cpu().numpy())
        del keep
    return outs[0], outs[1], int(n.value)


def _oracle(host, bits, gs, dt, mask=None):
    q, kq, vq = host
    return attention.quantized_sdpa_reference(q, kq[0], vq[0], kq[1], vq[1], kq[2], vq[2], bits=bits,
                                              group_size=gs, dtype=dt, mask=mask)


def test_noalloc_matches_decode_on_calls_in_a_row(device):
    rng = np.random.default_rng(123)
    cases = [
        # (B, Hq, Hkv, N, D, bits, gs, dtype): larger first, then smaller
        (1, 32, 2, 16384, 256, 4, 32, "f16"),   # C3-like, 128 splits
        (2, 8, 2, 3000, 128, 8, 64, "bf16"),    # smaller: fewer rows and splits
        (1, 4, 4, 700, 128, 4, 32, "f16"),      # smaller again
    ]
    for case in cases:
        B, Hq, Hkv, N, D, bits, gs, dt = case
        host, devt = _inputs(rng, B, Hq, Hkv, N, D, bits, gs, dt, device)
        ref, got, splits = _run_both(host, devt, bits, gs, dt)
        assert splits > 1, f"{case}: expected a split-K plan"
        assert np.array_equal(got, ref), f"{case}: noalloc output differs from qsdpa_decode"
        want = _oracle(host, bits, gs, dt)
        err = np.abs(got - want)
        assert np.all(err <= ATOL + RTOL * np.abs(want)), f"{case}: max err {err.max():.3e}"


def test_noalloc_streamk_schedule_and_single_pass(device):
    """Left-padded batch (stream-K schedule, its table in the scratch too),
    then a single pass (no scratch at all)."""
    rng = np.random.default_rng(124)
    B, Hq, Hkv, N, D, bits, gs, dt = 5, 32, 8, 1100, 128, 4, 64, "f16"
    host, devt = _inputs(rng, B, Hq, Hkv, N, D, bits, gs, dt, device)
    starts = np.array([0, 1099, 37, 600, 1100])
    ks = torch.tensor(starts, dtype=torch.int32, device=device)
    ref, got, splits = _run_both(host, devt, bits, gs, dt, kv_start=ks, num_splits=3)
    assert splits == 3
    assert np.array_equal(got, ref)
    add = np.where(np.arange(N)[None, :] >= starts[:, None], 0.0, -np.inf)[:, None, None, :]
    want = _oracle(host, bits, gs, dt, mask=add)
    want[starts >= N] = 0.0
    assert np.all(np.abs(got - want) <= ATOL + RTOL * np.abs(want))
    ref, got, splits = _run_both(host, devt, bits, gs, dt, num_splits=1)
    assert splits == 1 and np.array_equal(got, ref)


def test_noalloc_prefill_key_splits(device):
    """Several query positions per kv head on the prefill kernel with key
    splits (float32 partials of many rows in the scratch, merged by the row
    merge), then a smaller chunk on the same scratch."""
    rng = np.random.default_rng(125)
    cases = [
        # (B, Hq, Hkv, N, qL, D, bits, gs, dtype)
        (1, 16, 4, 3000, 128, 128, 8, 128, "bf16"),   # 16 row groups: 11 key splits
        (1, 8, 2, 1500, 64, 128, 4, 64, "f16"),       # smaller: 4 row groups, float16 partial rows
    ]
    for case in cases:
        B, Hq, Hkv, N, qL, D, bits, gs, dt = case
        host, devt = _inputs(rng, B, Hq, Hkv, N, D, bits, gs, dt, device, qL=qL)
        ref, got, splits = _run_both(host, devt, bits, gs, dt, causal=True)
        assert splits > 1, f"{case}: expected key splits"
        assert np.array_equal(got, ref), f"{case}: noalloc output differs from qsdpa_decode"
        want = _oracle(host, bits, gs, dt, mask="causal")  # aligned to the last key
        err = np.abs(got - want)
        assert np.all(err <= ATOL + RTOL * np.abs(want)), f"{case}: max err {err.max():.3e}"


def test_noalloc_refuses_partials_beyond_the_scratch(device):
    """Many query rows and splits need more than the static array: refused
    with QSDPA_ERR_WORKSPACE, nothing launched."""
    lib = _lib.load()
    B, Hq, Hkv, N, D, bits, gs = 64, 64, 8, 4096, 256, 4, 32
    T = torch.float16
    q = torch.zeros((B, Hq, 1, D), dtype=T, device=device)
    kp = torch.zeros((B, Hkv, N, D * bits // 32), dtype=torch.uint32, device=device)
    sc = torch.zeros((B, Hkv, N, D // gs), dtype=T, device=device)
    out = torch.zeros_like(q)
    a, keep = kernels._decode_args(q, kp, kp, sc, sc, sc, sc, out, 1.0, bits, gs, None, None, 64)
    n = ctypes.c_int32(0)
    ws = _lib.check(lib.qsdpa_decode_workspace_size(ctypes.byref(a), ctypes.byref(n)))
    assert ws > _lib.NOALLOC_SCRATCH_BYTES
    rc = lib.qsdpa_decode_noalloc(ctypes.byref(a), torch.cuda.current_stream(device).cuda_stream)
    assert rc == _lib.QSDPA_ERR_WORKSPACE
    assert b"static scratch" in lib.qsdpa_last_error()
    del keep
