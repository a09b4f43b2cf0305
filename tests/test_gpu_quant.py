"""Quantize-on-append and dequantize kernels vs the oracle: bit-exact."""

import json

import numpy as np
import pytest
import torch

from conftest import GOLDEN, from_np, to_np, torch_dtype
from oracle import affine

from mlx_qsdpa_amd import kernels

pytestmark = pytest.mark.gpu

KAT = json.loads((GOLDEN / "affine_known_answers.json").read_text())


def _bits_equal(a, b, dtype):
    return np.array_equal(affine.T_bits(a, dtype), affine.T_bits(b, dtype))


@pytest.mark.parametrize("case", KAT["quantize"], ids=lambda c: c["name"])
def test_quantize_kernel_known_answers(device, case):
    dt = torch_dtype(case["dtype"])
    w = from_np(np.array(case["w"], np.float32)[None], dt, device)
    p, s, b = kernels.quantize(w, case["group_size"], case["bits"])
    p = to_np(p)
    assert affine.unpack(p, case["bits"])[0].tolist() == case["codes"]
    if "words" in case:
        assert p[0].tolist() == [int(x, 16) for x in case["words"]]
    assert affine.T_bits(to_np(b), case["dtype"])[0, 0] == int(case["bias_bits"], 16)
    if "scale_bits" in case:
        assert affine.T_bits(to_np(s), case["dtype"])[0, 0] == int(case["scale_bits"], 16)


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
@pytest.mark.parametrize("bits,gs,D", [(4, 32, 256), (4, 64, 128), (4, 128, 128),
                                       (8, 32, 64), (8, 64, 256), (8, 128, 128)])
def test_quantize_kernel_matches_oracle(device, dtype, bits, gs, D):
    rng = np.random.default_rng(bits * 1000 + gs + D)
    w = affine.random_T(rng, (3, 4, 257, D), dtype, outlier_frac=0.02)
    w[0, 0, 0] = 0.0                      # all-zero row
    w[0, 0, 1] = w[0, 0, 1, :1]           # constant row
    w[0, 0, 2] = -np.abs(w[0, 0, 2])      # all-negative row
    want = affine.quantize(w, gs, bits, dtype)
    got = kernels.quantize(from_np(w, torch_dtype(dtype), device), gs, bits)
    assert np.array_equal(to_np(got[0]), want[0])
    assert _bits_equal(to_np(got[1]), want[1], dtype)
    assert _bits_equal(to_np(got[2]), want[2], dtype)


@pytest.mark.parametrize("dtype,bits,gs", [("f16", 4, 32), ("bf16", 8, 64)])
def test_quantize_bulk_matches_oracle(device, dtype, bits, gs):
    """A prompt-sized job (>= 2^18 groups) takes the one-lane-per-group
    kernel; bit-exact like the per-token appends."""
    rng = np.random.default_rng(bits * 7 + gs)
    D = 128
    S = (1 << 18) * gs // D // 8  # 8 heads x S rows x D / gs groups = 2^18
    w = affine.random_T(rng, (1, 8, S, D), dtype, outlier_frac=0.01)
    want = affine.quantize(w, gs, bits, dtype)
    got = kernels.quantize(from_np(w, torch_dtype(dtype), device), gs, bits)
    assert np.array_equal(to_np(got[0]), want[0])
    assert _bits_equal(to_np(got[1]), want[1], dtype)
    assert _bits_equal(to_np(got[2]), want[2], dtype)


@pytest.mark.parametrize("bulk", [False, True], ids=["append", "bulk"])
@pytest.mark.parametrize("dtype,bits", [("f16", 4), ("bf16", 8), ("bf16", 4), ("f16", 8)])
def test_quantize_ties_round_half_to_even(device, dtype, bits, bulk):
    """Groups spanning [0, 2^bits - 1] with values at half-integers: the
    snapped scale is -1 (times a power of two), so every such value's code
    is an exact tie, which the kernel's reciprocal path must hand to the
    exactly rounded quotient (round half to even).  Small jobs (8 values per
    lane) and bulk ones (32 values per lane)."""
    gs, D = 128, 128
    bins = (1 << bits) - 1
    top = min(bins, 127)  # k + 1/2 exact in bf16 for k < 128
    row = np.array([0.0, float(bins)] + [k + 0.5 for k in range(top)] * (D // top + 1), np.float32)[:D]
    S = (1 << 18) // 8 if bulk else 5  # bulk: 8 heads x S rows x one group = 2^18 groups
    heads = np.float32([1.0, 0.25, 4.0, 0.5, 2.0, 1.0, 8.0, 0.125])  # exact scalings, one per head
    w = np.ascontiguousarray(np.broadcast_to(row, (1, 8, S, D)) * heads[None, :, None, None])
    assert np.array_equal(affine.to_T(w, dtype), w)  # every value exact in T
    want = affine.quantize(w, gs, bits, dtype)
    codes = affine.unpack(want[0], bits)
    assert np.any(codes[..., 2:] % 2 == 0)  # the ties went to even codes
    got = kernels.quantize(from_np(w, torch_dtype(dtype), device), gs, bits)
    assert np.array_equal(to_np(got[0]), want[0])
    assert _bits_equal(to_np(got[1]), want[1], dtype)
    assert _bits_equal(to_np(got[2]), want[2], dtype)


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_quantize_into_strided_destination(device, dtype):
    """Writes land at [t0, t0+S) of a capacity-padded buffer; nothing else changes."""
    rng = np.random.default_rng(3)
    B, H, S, D, cap, t0, gs, bits = 2, 3, 5, 128, 40, 17, 64, 4
    T = torch_dtype(dtype)
    src = affine.random_T(rng, (B, H, S, D), dtype)
    dst = (torch.full((B, H, cap, D * bits // 32), 0xDEAD, dtype=torch.int32, device=device)
           .view(torch.uint32),
           torch.full((B, H, cap, D // gs), 7.0, dtype=T, device=device),
           torch.full((B, H, cap, D // gs), 7.0, dtype=T, device=device))
    # a transposed (non-contiguous) source view
    src_t = from_np(np.ascontiguousarray(src.transpose(1, 0, 2, 3)), T, device).transpose(0, 1)
    kernels.quantize_into(src_t, dst, t0, bits, gs)
    want = affine.quantize(src, gs, bits, dtype)
    p = to_np(dst[0])
    assert np.array_equal(p[:, :, t0:t0 + S], want[0])
    assert np.all(p[:, :, :t0] == 0xDEAD) and np.all(p[:, :, t0 + S:] == 0xDEAD)
    assert _bits_equal(to_np(dst[1])[:, :, t0:t0 + S], want[1], dtype)
    assert np.all(to_np(dst[2])[:, :, :t0] == 7.0)


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
@pytest.mark.parametrize("aligned", [True, False], ids=["vec", "unaligned"])
def test_quantize_batch_matches_oracle(device, dtype, aligned):
    """qsdpa_quantize_batch: a key job and a value job of different shapes
    (D 128 and 64, 5 and 3 rows) in one launch land bit-exactly at [t0,
    t0 + S) of their own capacity-padded buffers; nothing else is written.
    A value source with rows 2-byte aligned only takes the element-wise
    load path for both jobs."""
    rng = np.random.default_rng(11)
    T = torch_dtype(dtype)
    bits, gs, t0, cap = 4, 32, 9, 24
    shapes = [(2, 3, 5, 128), (2, 3, 3, 64)]
    srcs, dsts, views = [], [], []
    for i, (B, H, S, D) in enumerate(shapes):
        w = affine.random_T(rng, (B, H, S, D), dtype, outlier_frac=0.02)
        w[0, 0, 0] = 0.0
        if aligned or i == 0:
            v = from_np(w, T, device)
        else:  # rows start one element into a D + 1 wide buffer
            base = torch.zeros((B, H, S, D + 1), dtype=T, device=device)
            base[..., 1:] = from_np(w, T, device)
            v = base[..., 1:]
        srcs.append(w)
        views.append(v)
        dsts.append((torch.full((B, H, cap, D * bits // 32), 0x5A5A, dtype=torch.int32, device=device)
                     .view(torch.uint32),
                     torch.full((B, H, cap, D // gs), 7.0, dtype=T, device=device),
                     torch.full((B, H, cap, D // gs), 7.0, dtype=T, device=device)))
    kernels.quantize_kv_into(views[0], views[1], dsts[0], dsts[1], t0, bits, gs)
    for w, dst in zip(srcs, dsts):
        S = w.shape[2]
        want = affine.quantize(w, gs, bits, dtype)
        p = to_np(dst[0])
        assert np.array_equal(p[:, :, t0:t0 + S], want[0])
        assert np.all(p[:, :, :t0] == 0x5A5A) and np.all(p[:, :, t0 + S:] == 0x5A5A)
        assert _bits_equal(to_np(dst[1])[:, :, t0:t0 + S], want[1], dtype)
        assert _bits_equal(to_np(dst[2])[:, :, t0:t0 + S], want[2], dtype)
        assert np.all(to_np(dst[1])[:, :, t0 + S:] == 7.0) and np.all(to_np(dst[2])[:, :, :t0] == 7.0)


def _scalar_T(bits_hex, dt, device):
    v = int(bits_hex, 16)
    v = v - (1 << 16) if v >= 1 << 15 else v
    return torch.tensor([[v]], dtype=torch.int16).view(dt).to(device)


@pytest.mark.parametrize("case", KAT["dequantize"], ids=lambda c: c["name"])
def test_dequantize_kernel_known_answers(device, case):
    dt = torch_dtype(case["dtype"])
    q = np.zeros((1, case["group_size"]), np.uint32)
    q[0, 0] = case["code"]
    p = torch.from_numpy(affine.pack(q, case["bits"])).to(device)
    s = _scalar_T(case["scale_bits"], dt, device)
    b = _scalar_T(case["bias_bits"], dt, device)
    v = kernels.dequantize(p, s, b, case["group_size"], case["bits"])
    assert affine.T_bits(to_np(v)[:, :1], case["dtype"])[0, 0] == int(case["value_bits"], 16)


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
@pytest.mark.parametrize("bits,gs", [(4, 32), (4, 128), (8, 64)])
def test_dequantize_kernel_matches_oracle(device, dtype, bits, gs):
    rng = np.random.default_rng(bits + gs)
    w = affine.random_T(rng, (2, 3, 100, 128), dtype)
    p, s, b = affine.quantize(w, gs, bits, dtype)
    T = torch_dtype(dtype)
    got = kernels.dequantize(torch.from_numpy(p).to(device), from_np(s, T, device),
                             from_np(b, T, device), gs, bits)
    want = affine.dequantize(p, s, b, gs, bits, dtype)
    assert _bits_equal(to_np(got), want, dtype)
    got0 = kernels.dequantize(torch.from_numpy(p).to(device), from_np(s, T, device), None, gs, bits)
    assert _bits_equal(to_np(got0), affine.dequantize(p, s, None, gs, bits, dtype), dtype)


@pytest.mark.parametrize("keep,rot", [(0, 0), (0, 5), (3, 4), (2, 9)])
def test_dequantize_ring_reorder(device, keep, rot):
    rng = np.random.default_rng(keep * 10 + rot)
    N = 12
    w = affine.random_T(rng, (1, 2, N, 64), "f16")
    p, s, b = affine.quantize(w, 32, 4, "f16")
    T = torch.float16
    got = kernels.dequantize(torch.from_numpy(p).to(device), from_np(s, T, device),
                             from_np(b, T, device), 32, 4, keep=keep, rot=rot)
    full = affine.dequantize(p, s, b, 32, 4, "f16")
    idx = [t if t < keep else keep + (t - keep + rot) % (N - keep) for t in range(N)]
    assert _bits_equal(to_np(got), full[:, :, idx], "f16")


@pytest.mark.parametrize("case", [
    # (max_size, keep, n_old, rot, S, bits, gs, dtype)
    (64, 0, 0, 0, 40, 4, 32, "f16"),      # first prompt: no old window
    (64, 0, 0, 0, 90, 8, 64, "bf16"),     # first prompt longer than the window
    (64, 4, 3, 0, 5, 4, 32, "f16"),       # fewer old tokens than sinks
    (64, 0, 64, 17, 9, 4, 64, "f16"),     # wrapped, keep = 0
    (64, 4, 64, 29, 12, 8, 32, "bf16"),   # wrapped, keep = 4 sinks
    (64, 4, 64, 59, 70, 4, 128, "f16"),   # chunk longer than the window
    (4096, 4, 4096, 1234, 512, 8, 128, "bf16"),  # C5's chunk over its wrapped window
])
def test_requant_window_matches_oracle(device, case):
    """qsdpa_requant_window (one launch, K and V) against the oracle's steps:
    dequantize the old window in temporal order, append, keep the first
    `keep` and the newest max_size - keep, quantize; bit-exact."""
    W, keep, n_old, rot, S, bits, gs, dt = case
    B, H, D = 2, 3, 128
    rng = np.random.default_rng(W + keep + n_old + rot + S)
    T = torch_dtype(dt)
    old_np, new_np, dst = [], [], []
    for _ in range(2):  # K, V
        ring = affine.quantize(affine.random_T(rng, (B, H, W, D), dt, outlier_frac=0.02), gs, bits, dt)
        old_np.append(ring)
        new_np.append(affine.random_T(rng, (B, H, S, D), dt))
        dst.append((torch.full((B, H, W, D * bits // 32), 0xDEADBEEF, dtype=torch.int64).to(torch.uint32).to(device),
                    torch.zeros((B, H, W, D // gs), dtype=T, device=device),
                    torch.zeros((B, H, W, D // gs), dtype=T, device=device)))
    old = [tuple(from_np(x, T, device) for x in o) for o in old_np]
    new = [from_np(x, T, device) for x in new_np]
    total = kernels.requant_window(tuple(old), tuple(new), tuple(dst), n_old, keep, rot, W, bits, gs)
    torch.cuda.synchronize()
    assert total == min(n_old + S, W)
    for o, x, d in zip(old_np, new_np, dst):
        allv = x
        if n_old:
            win = affine.dequantize(*(t[:, :, :n_old] for t in o), gs, bits, dt)
            idx = np.arange(n_old)
            if rot:
                idx = np.where(idx < keep, idx, keep + (idx - keep + rot) % (n_old - keep))
            allv = np.concatenate([win[:, :, idx], x], axis=2)
        n = allv.shape[2]
        if n > W:
            allv = np.concatenate([allv[:, :, :keep], allv[:, :, n - (W - keep):]], axis=2)
        want = affine.quantize(allv, gs, bits, dt)
        assert np.array_equal(to_np(d[0][:, :, :total]), want[0]), "packed words differ"
        for i in (1, 2):
            assert np.array_equal(affine.T_bits(to_np(d[i][:, :, :total]), dt), affine.T_bits(want[i], dt))
