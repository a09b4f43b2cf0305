"""Rows past a sequence's end read as zero: the hardware behaviour behind
the decode and prefill kernels' partial tiles, and parity with NaN past N.

The matrix-core kernels read a tile's rows through buffer descriptors whose
range ends at the sequence's last row; a partial last tile and the
pipeline's prefetch past the end address rows beyond it through the load's
scalar offset, and rely on the range check to return zero for them (a
masked key then multiplies P = 0 by 0, never by whatever lies in memory
past the row).

* test_buffer_range_check_includes_soffset: a raw buffer load returns zero
  past num_records whether the offset is in voffset or in soffset (a probe
  kernel whose addresses all lie inside its allocation).
* test_nan_past_the_end_*: K / V codes, scales and biases as [:, :, :N]
  slices of buffers whose rows past N hold NaN scales / biases and all-ones
  codes, N not a multiple of the 32- or 64-key tile, with and without
  kv_start, for decode (one query position) and the prefill kernel: the
  outputs match the oracle on the unpadded data, so no row past N is read.

Tolerance (north star): |out - ref| <= 2e-3 + 1e-2 |ref|.
"""

import ctypes
from pathlib import Path

import numpy as np
import pytest
import torch

from conftest import from_np, to_np, torch_dtype
from oracle import affine, attention

import mlx_qsdpa_amd as mq

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-3, 1e-2
PROBE = Path(__file__).resolve().parent / "hip" / "libbuffer_range.so"


def test_buffer_range_check_includes_soffset(device):
    if not PROBE.exists():
        pytest.fail(f"{PROBE} not built (python tests/hip/build_probe.py)")
    lib = ctypes.CDLL(str(PROBE))
    lib.buffer_range_probe.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]
    lib.buffer_range_probe.restype = ctypes.c_int
    base = (torch.arange(16384, dtype=torch.int64) + 0x1000000).to(torch.int32).to(device)  # 64 KiB
    out = torch.full((10, 64), -1, dtype=torch.int32, device=device)
    stream = torch.cuda.current_stream(device).cuda_stream
    assert lib.buffer_range_probe(base.data_ptr(), out.data_ptr(), stream) == 0
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    lane = np.arange(64)
    for i, off in enumerate((0, 2048, 3968, 4096, 8192)):
        word = (lane * 4 + off) // 4
        want = np.where(lane * 4 + off < 4096, 0x1000000 + word, 0)
        assert np.array_equal(got[2 * i], want), f"voffset {off}: {got[2 * i][:4]} ..."
        assert np.array_equal(got[2 * i + 1], want), f"soffset {off}: past-the-end rows are not zero"


def _padded(x, N, pad, T, device, fill):
    """x [B, H, N, W] in a [B, H, N + pad, W] buffer whose rows past N hold
    `fill`; returns the [:, :, :N] view."""
    B, H, _, W = x.shape
    if x.dtype == np.uint32:
        buf = torch.full((B, H, N + pad, W), -1, dtype=torch.int32, device=device).view(torch.uint32)
        buf.view(torch.int32)[:, :, :N] = torch.from_numpy(np.ascontiguousarray(x)).view(torch.int32).to(device)
    else:
        buf = torch.full((B, H, N + pad, W), fill, dtype=T, device=device)
        buf[:, :, :N] = from_np(x, T, device)
    return buf[:, :, :N]


def _run(case, device, qL, causal):
    B, Hq, Hkv, N, D, bits, gs, dt = case
    T = torch_dtype(dt)
    rng = np.random.default_rng(N + qL)
    q = affine.random_T(rng, (B, Hq, qL, D), dt)
    kq = affine.quantize(affine.random_T(rng, (B, Hkv, N, D), dt), gs, bits, dt)
    vq = affine.quantize(affine.random_T(rng, (B, Hkv, N, D), dt), gs, bits, dt)
    dk = [_padded(x, N, 200, T, device, float("nan")) for x in kq]
    dv = [_padded(x, N, 200, T, device, float("nan")) for x in vq]
    starts = np.array([0, 45] + [7] * (B - 2))[:B]
    for kv_start in (None, starts):
        for splits in ((None, 1, 3) if qL == 1 else (None,)):
            ks = None if kv_start is None else torch.tensor(kv_start, dtype=torch.int32, device=device)
            got = mq.quantized_sdpa(from_np(q, T, device), dk[0], dv[0], dk[1], dv[1], dk[2], dv[2], bits=bits,
                                    group_size=gs, mask="causal" if causal else None, kv_start=ks,
                                    num_splits=splits)
            torch.cuda.synchronize()
            mask = "causal" if causal else None
            if kv_start is not None:
                keep = np.arange(N)[None, None, None, :] >= kv_start[:, None, None, None]
                if causal:
                    qi = np.arange(qL)[:, None] + (N - qL)
                    keep = keep & (qi >= np.arange(N)[None, :])[None, None]
                mask = np.broadcast_to(keep, (B, 1, qL, N))
            want = attention.quantized_sdpa_reference(q, kq[0], vq[0], kq[1], vq[1], kq[2], vq[2], bits=bits,
                                                      group_size=gs, dtype=dt, mask=mask)
            g = to_np(got)
            ctx = f"{case} qL={qL} kv_start={kv_start is not None} splits={splits}"
            assert np.isfinite(g).all(), f"{ctx}: non-finite output (a row past N was read)"
            err = np.abs(g - want)
            assert (err <= ATOL + RTOL * np.abs(want)).all(), f"{ctx}: max err {err.max():.3e}"


@pytest.mark.parametrize("case", [
    (2, 16, 2, 777, 128, 4, 32, "f16"),
    (1, 32, 2, 1000, 256, 4, 32, "f16"),
    (2, 2, 2, 999, 256, 8, 64, "bf16"),
    (2, 8, 2, 333, 64, 4, 32, "bf16"),
], ids=["D128-G8", "D256-G16", "D256-G1-bf16", "D64-valu"])
def test_nan_past_the_end_decode(device, case):
    _run(case, device, 1, False)


@pytest.mark.parametrize("case,qL", [
    ((2, 8, 2, 1001, 128, 8, 128, "bf16"), 64),
    ((1, 16, 4, 650, 128, 4, 32, "f16"), 40),
], ids=["prefill-G4-q64-bf16", "prefill-G4-q40"])
def test_nan_past_the_end_prefill(device, case, qL):
    _run(case, device, qL, True)


@pytest.mark.parametrize("dt", ["f16", "bf16"])
def test_nan_past_the_end_prefill_d256(device, dt):
    """The D = 256 prefill kernel (32-key tiles; the call meets its routing
    threshold: 256 rows per kv head, 2^24 row-key pairs), N = 32785 (17 keys
    into the last tile), rows past N NaN / all-ones, with and without
    kv_start; checked against the float64 torch oracle on the unpadded data
    (the numpy oracle takes about 15 s at this size)."""
    import torch_oracle as to
    from mlx_qsdpa_amd import kernels

    B, Hq, Hkv, N, D, bits, gs, qL = 1, 16, 2, 32785, 256, 4, 32, 32
    assert Hq // Hkv * qL >= 256 and B * Hq * qL * N >= 1 << 24
    T = torch_dtype(dt)
    g = torch.Generator(device="cpu").manual_seed(41)
    q = torch.randn(B, Hq, qL, D, generator=g).to(T).to(device)
    kq = kernels.quantize(torch.randn(B, Hkv, N, D, generator=g).to(T).to(device), gs, bits)
    vq = kernels.quantize(torch.randn(B, Hkv, N, D, generator=g).to(T).to(device), gs, bits)

    def padded(x):
        shape = (B, Hkv, N + 200, x.shape[-1])
        if x.is_floating_point():
            buf = torch.full(shape, float("nan"), dtype=x.dtype, device=device)
            buf[:, :, :N] = x
            return buf[:, :, :N]
        buf = torch.full(shape, -1, dtype=torch.int32, device=device)  # all-ones codes
        buf[:, :, :N] = x.view(torch.int32)
        return buf.view(x.dtype)[:, :, :N]

    dk, dv = [padded(x) for x in kq], [padded(x) for x in vq]
    for kv_start in (None, torch.tensor([45], dtype=torch.int32, device=device)):
        got = mq.quantized_sdpa(q, dk[0], dv[0], dk[1], dv[1], dk[2], dv[2], bits=bits, group_size=gs,
                                mask="causal", kv_start=kv_start)
        keep = torch.arange(N, device=device)[None, :] <= (N - qL) + torch.arange(qL, device=device)[:, None]
        if kv_start is not None:
            keep = keep & (torch.arange(N, device=device) >= int(kv_start[0]))[None, :]
        want = to.quantized_sdpa(q, kq, vq, bits=bits, group_size=gs, scale=D ** -0.5, mask=keep[None, None])
        torch.cuda.synchronize()
        ctx = f"D=256 prefill {dt} kv_start={kv_start is not None}"
        assert bool(torch.isfinite(got).all()), f"{ctx}: non-finite output (a row past N was read)"
        err = (got.double() - want).abs()
        assert bool((err <= ATOL + RTOL * want.abs()).all()), f"{ctx}: max err {float(err.max()):.3e}"
