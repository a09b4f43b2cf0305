"""Decode parity on the GPU: HIP kernels (through the C ABI) vs the oracle.

Tolerance (north star): |out - ref| <= 2e-3 + 1e-2 * |ref| with ref the
float64 dequantize + SDPA oracle on the same seeded, oracle-quantized inputs.
"""

import numpy as np
import pytest
import torch

import torch_oracle
from conftest import from_np, to_np, torch_dtype
from oracle import affine, attention

import mlx_qsdpa_amd as mq
from mlx_qsdpa_amd import kernels

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-3, 1e-2


def make_inputs(rng, B, Hq, Hkv, N, D, bits, gs, dtype="f16", outliers=0.0, symmetric=False):
    q = affine.random_T(rng, (B, Hq, 1, D), dtype)
    kw = affine.random_T(rng, (B, Hkv, N, D), dtype, outlier_frac=outliers)
    vw = affine.random_T(rng, (B, Hkv, N, D), dtype, outlier_frac=outliers)
    kp, ks, kb = affine.quantize(kw, gs, bits, dtype)
    vp, vs, vb = affine.quantize(vw, gs, bits, dtype)
    if symmetric:
        kb = vb = None
    return dict(q=q, kp=kp, vp=vp, ks=ks, vs=vs, kb=kb, vb=vb, bits=bits, gs=gs, dtype=dtype)


def to_dev(inp, device):
    t = torch_dtype(inp["dtype"])
    g = {k: (None if inp[k] is None else from_np(inp[k], t, device))
         for k in ("q", "kp", "vp", "ks", "vs", "kb", "vb")}
    return g


def oracle_out(inp, mask=None, scale=None):
    return attention.quantized_sdpa_reference(
        inp["q"], inp["kp"], inp["vp"], inp["ks"], inp["vs"], inp["kb"], inp["vb"],
        bits=inp["bits"], group_size=inp["gs"], dtype=inp["dtype"], scale=scale, mask=mask)


def run(inp, device, **kw):
    g = to_dev(inp, device)
    out = mq.quantized_sdpa(g["q"], g["kp"], g["vp"], g["ks"], g["vs"], g["kb"], g["vb"],
                            bits=inp["bits"], group_size=inp["gs"], **kw)
    torch.cuda.synchronize()
    return to_np(out)


def assert_close(got, want, ctx=""):
    err = np.abs(got - want)
    bound = ATOL + RTOL * np.abs(want)
    bad = err > bound
    assert not bad.any(), (f"{ctx}: {bad.sum()} of {bad.size} outside tolerance, "
                           f"max abs err {err.max():.3e}")
    assert np.isfinite(got).all(), ctx


# B, Hq, Hkv, N, D, bits, gs, dtype -- the reference's test shapes
# (tests/test_correctness.py, test_2pass.py, test_formats.py, test_shapes.py,
# test_long_context.py) and BASELINE configs at oracle-sized N.
CASES = [
    (1, 1, 1, 32, 128, 4, 32, "f16"),
    (1, 16, 2, 64, 256, 4, 32, "f16"),
    (1, 16, 2, 1024, 256, 4, 32, "f16"),
    (1, 4, 1, 1, 128, 4, 32, "f16"),
    (1, 16, 2, 128, 256, 8, 32, "f16"),
    (1, 16, 2, 128, 256, 4, 64, "f16"),
    (1, 16, 2, 128, 256, 4, 128, "f16"),
    (1, 4, 4, 64, 128, 4, 32, "f16"),
    (1, 4, 2, 64, 256, 4, 32, "f16"),
    (1, 4, 2, 32, 128, 4, 32, "f16"),
    (2, 4, 2, 64, 128, 4, 32, "f16"),
    (1, 16, 2, 4096, 256, 4, 32, "f16"),
    (1, 16, 2, 8192, 256, 4, 32, "f16"),
    (1, 32, 2, 64, 256, 4, 32, "f16"),
    (1, 2, 2, 64, 256, 8, 32, "f16"),
    (1, 8, 2, 4096, 128, 4, 64, "f16"),      # C1
    (1, 2, 2, 8192, 256, 8, 64, "bf16"),     # C2 (small N)
    (1, 32, 2, 16384, 256, 4, 32, "f16"),    # C3 (small N)
    (4, 32, 8, 1024, 128, 4, 64, "f16"),     # C4 shape
    (4, 16, 4, 4096, 128, 8, 128, "bf16"),   # C5 decode window
    (1, 8, 1, 300, 64, 4, 32, "bf16"),
    (3, 6, 3, 77, 64, 8, 64, "f16"),
    # head groups of 16 / 32 (MFMA kernel) across D, bits, dtypes, ragged N
    (2, 32, 2, 777, 256, 8, 64, "bf16"),
    (1, 16, 1, 300, 128, 4, 32, "bf16"),
    (1, 32, 1, 1000, 64, 8, 32, "f16"),
    (3, 16, 1, 129, 128, 8, 128, "f16"),
    (1, 32, 2, 5000, 256, 4, 64, "bf16"),
    (1, 16, 1, 31, 256, 4, 128, "f16"),
    (2, 64, 4, 2049, 64, 4, 32, "bf16"),
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: "B{}_Hq{}_Hkv{}_N{}_D{}_b{}_g{}_{}".format(*c))
def test_decode_matches_oracle(device, case):
    B, Hq, Hkv, N, D, bits, gs, dt = case
    rng = np.random.default_rng(1000 + N + D + Hq)
    inp = make_inputs(rng, B, Hq, Hkv, N, D, bits, gs, dt, outliers=0.01 if dt == "bf16" else 0)
    want = oracle_out(inp)
    for splits in (None, 1, 7):
        got = run(inp, device, num_splits=splits)
        assert_close(got, want, f"{case} splits={splits}")


@pytest.mark.parametrize("bits", [4, 8])
def test_symmetric_format(device, bits):
    rng = np.random.default_rng(7)
    inp = make_inputs(rng, 1, 16, 2, 128, 256, bits, 32, symmetric=True)
    assert_close(run(inp, device), oracle_out(inp), "symmetric")


def test_one_bias_missing_means_zero_biases(device):
    """dispatch.py:89-94: unless both biases are given, both are zero."""
    rng = np.random.default_rng(8)
    inp = make_inputs(rng, 1, 4, 2, 64, 128, 4, 32)
    g = to_dev(inp, device)
    out = mq.quantized_sdpa(g["q"], g["kp"], g["vp"], g["ks"], g["vs"], g["kb"], None)
    want = oracle_out(dict(inp, kb=None, vb=None))
    assert_close(to_np(out), want, "one bias")


def test_threshold_semantics(device):
    """tests/test_long_context.py:30-67: threshold N+1 -> single, N-1 -> split."""
    rng = np.random.default_rng(9)
    N = 4096
    inp = make_inputs(rng, 1, 16, 2, N, 256, 4, 32)
    want = oracle_out(inp)
    a = run(inp, device, threshold=N + 1)
    b = run(inp, device, threshold=N - 1)
    c = run(inp, device, threshold=0)
    for x in (a, b, c):
        assert_close(x, want, "threshold")
    assert np.abs(a - b).max() < 2e-3


def test_single_key_returns_value_row(device):
    rng = np.random.default_rng(10)
    inp = make_inputs(rng, 1, 4, 2, 1, 128, 4, 32)
    got = run(inp, device)
    v = affine.dequantize(inp["vp"], inp["vs"], inp["vb"], 32, 4, "f16")
    want = np.repeat(v[:, :, 0:1], 2, axis=1)
    assert_close(got, want, "N=1")


def test_zero_scales_no_nan(device):
    """tests/test_shapes.py:89-101."""
    rng = np.random.default_rng(11)
    inp = make_inputs(rng, 1, 4, 2, 32, 128, 4, 32)
    for k in ("ks", "vs", "kb", "vb"):
        inp[k] = np.zeros_like(inp[k])
    got = run(inp, device)
    assert np.isfinite(got).all() and np.all(got == 0)


@pytest.mark.parametrize("heads", [(8, 2), (32, 2)], ids=["G4", "G16"])
@pytest.mark.parametrize("mdtype", ["bool", "f16", "f32", "per_head"])
def test_masked_decode_in_kernel(device, mdtype, heads):
    rng = np.random.default_rng(12)
    (Hq, Hkv), B, N = heads, 2, 700
    inp = make_inputs(rng, B, Hq, Hkv, N, 128, 4, 32)
    if mdtype == "per_head":
        keep = rng.random((B, Hq, 1, N)) > 0.5
    else:
        keep = rng.random((B, 1, 1, N)) > 0.3
    keep[..., 5] = True
    if mdtype == "bool" or mdtype == "per_head":
        m_np, m_t = keep, torch.from_numpy(keep).to(device)
    else:
        add = np.where(keep, rng.standard_normal(keep.shape) * 0.5, -np.inf).astype(np.float32)
        if mdtype == "f16":
            add = add.astype(np.float16).astype(np.float32)
        m_np = add
        m_t = torch.from_numpy(add).to(device, torch.float16 if mdtype == "f16" else torch.float32)
    want = oracle_out(inp, mask=m_np)
    for splits in (None, 1, 5):
        assert_close(run(inp, device, mask=m_t, num_splits=splits), want, f"mask {mdtype}")


@pytest.mark.parametrize("heads", [(32, 8), (32, 2)], ids=["G4", "G16"])
def test_kv_start_left_padding(device, heads):
    """Keys before kv_start[b] are skipped == additive -inf mask on them (C4 semantics)."""
    rng = np.random.default_rng(13)
    (Hq, Hkv), B, N = heads, 4, 2000
    inp = make_inputs(rng, B, Hq, Hkv, N, 128, 4, 64)
    starts = np.array([0, 1500, 37, 1999])
    add = np.where(np.arange(N)[None, :] >= starts[:, None], 0.0, -np.inf)[:, None, None, :]
    want = oracle_out(inp, mask=add)
    ks = torch.tensor(starts, dtype=torch.int32, device=device)
    for splits in (None, 1, 9):
        assert_close(run(inp, device, kv_start=ks, num_splits=splits), want, "kv_start")
    m = torch.from_numpy(add.astype(np.float32)).to(device, torch.float16)
    assert_close(run(inp, device, mask=m), want, "additive left padding")


@pytest.mark.parametrize("case", [
    # (B, Hq, Hkv, N, D, gs, dtype, splits)
    (70, 8, 2, 300, 128, 64, "f16", (None, 2, 3)),    # more sequences than a wave's 64 lanes
    (5, 32, 8, 1100, 128, 32, "f16", (2, 7, 64)),
    (6, 16, 1, 700, 256, 32, "bf16", (None, 4, 16)),
    (7, 32, 2, 650, 256, 32, "f16", (None, 3, 16)),   # C3's heads (G = 16), float16
], ids=["B70", "B5-G4", "B6-D256-bf16", "B7-D256-G16-f16"])
def test_kv_start_streamk_schedule(device, case):
    """A left-padded batch runs splits * B equal units over its sequences laid
    end to end (units cross sequences): ragged lengths, empty sequences (kv_start >= N, also past N),
    negative kv_start (clamped to 0) and split counts from 2 to 64 all match
    the oracle with an additive -inf mask on the skipped keys; repeated calls
    are bitwise identical."""
    B, Hq, Hkv, N, D, gs, dtype, splits_list = case
    rng = np.random.default_rng(31 + B)
    inp = make_inputs(rng, B, Hq, Hkv, N, D, 4, gs, dtype=dtype)
    starts = rng.integers(0, N, size=B)
    starts[0] = N          # empty
    starts[1] = N + 50     # past the end: empty
    starts[2] = -7         # clamped to 0: the whole sequence
    starts[3] = N - 1      # one key
    if B > 5:
        starts[5] = N - 33  # one key past a tile
    keep_from = np.clip(starts, 0, N)
    add = np.where(np.arange(N)[None, :] >= keep_from[:, None], 0.0, -np.inf)[:, None, None, :]
    want = oracle_out(inp, mask=add)
    want[keep_from >= N] = 0.0  # no keys: zero output
    ks = torch.tensor(starts, dtype=torch.int32, device=device)
    for splits in splits_list:
        got = run(inp, device, kv_start=ks, num_splits=splits)
        assert_close(got, want, f"stream-K kv_start splits={splits}")
        assert np.all(got[keep_from >= N] == 0)
        again = run(inp, device, kv_start=ks, num_splits=splits)
        assert np.array_equal(got, again), f"splits={splits}: repeated call differs"


def _fused(inp, device, **kw):
    """The fused kernel through the C ABI (no routing, no fallback)."""
    g = to_dev(inp, device)
    D = inp["q"].shape[-1]
    out = kernels.decode(g["q"], g["kp"], g["vp"], g["ks"], g["vs"], g["kb"], g["vb"],
                         scale=D ** -0.5, bits=inp["bits"], group_size=inp["gs"], **kw)
    torch.cuda.synchronize()
    return to_np(out)


@pytest.mark.parametrize("case", [
    # (B, Hq, Hkv, N, D, bits, gs, dtype, qL, mask)
    (2, 32, 2, 300, 256, 4, 32, "f16", 4, "causal"),     # G=16: 4 row blocks of one position
    (1, 8, 2, 1000, 128, 4, 64, "f16", 3, None),        # G=4: 12 rows, one partial block
    (2, 4, 4, 513, 128, 8, 128, "bf16", 33, "causal"),  # G=1: 33 positions, 3 blocks
    (1, 16, 4, 700, 128, 8, 64, "bf16", 5, "additive"),  # per (head, position) additive mask
    (3, 8, 1, 400, 256, 4, 64, "f16", 2, "bool"),        # bool mask broadcast over heads
    (1, 16, 2, 40, 128, 4, 32, "f16", 48, "causal"),     # qL > N: the first rows see no key
    # many row blocks per kv head (>= 128 rows), partial last blocks
    (1, 16, 4, 700, 128, 8, 64, "bf16", 64, "causal"),   # 256 rows, 2 workgroups
    (2, 32, 2, 300, 256, 4, 32, "f16", 16, "causal"),    # D=256
    (1, 8, 2, 500, 128, 4, 32, "f16", 37, "additive"),   # 148 rows: last workgroup part-filled
    (2, 4, 4, 600, 256, 8, 128, "bf16", 130, "bool"),    # G=1, per-position bool mask
], ids=["G16-q4-causal", "G4-q3", "G1-q33-causal-bf16", "G4-q5-additive", "G8-q2-bool",
        "q48-over-N40-causal", "rows-G4-q64-causal-bf16", "rows-D256-G16-q16-causal",
        "rows-G4-q37-additive", "rows-G1-q130-bool-bf16"])
def test_multi_query_matches_oracle(device, case):
    """qL > 1 query positions (speculative / chunked decoding, prefill) on the
    fused kernel: rows are (position, head) pairs of a kv head; causal is
    aligned to the last key; masks index (batch, head, position, key)."""
    B, Hq, Hkv, N, D, bits, gs, dtype, qL, mk = case
    rng = np.random.default_rng(41 + qL)
    inp = make_inputs(rng, B, Hq, Hkv, N, D, bits, gs, dtype=dtype)
    inp["q"] = affine.random_T(rng, (B, Hq, qL, D), dtype)
    kw, m_np = {}, None
    if mk == "causal":
        kw["causal"], m_np = True, "causal"
    elif mk == "additive":
        add = rng.standard_normal((1, Hq, qL, N)).astype(np.float32)
        add[rng.random(add.shape) < 0.2] = -np.inf
        add = add.astype(np.float16).astype(np.float32)
        m_np, kw["mask"] = add, torch.from_numpy(add).to(device, torch.float16)
    elif mk == "bool":
        keep = rng.random((B, 1, qL, N)) < 0.7
        keep[..., 0] = True
        m_np, kw["mask"] = keep, torch.from_numpy(keep).to(device)
    want = oracle_out(inp, mask=m_np)
    for splits in (0, 1, 3):
        got = _fused(inp, device, num_splits=splits, **kw)
        assert got.shape == (B, Hq, qL, D)
        assert_close(got, want, f"qL={qL} splits={splits}")


@pytest.mark.parametrize("case", [
    # (B, Hq, Hkv, N, D, bits, gs, dtype, qL, causal, kv_start)
    (2, 32, 2, 300, 256, 4, 32, "f16", 2, True, None),        # 32 rows: 2 blocks
    (1, 16, 1, 1000, 256, 8, 64, "bf16", 3, False, None),     # 48 rows: 3 blocks, 8-bit
    (2, 8, 2, 777, 256, 4, 128, "f16", 5, True, (0, 300)),    # 20 rows: a part-filled block, kv_start
    (1, 32, 1, 500, 256, 4, 64, "bf16", 1, False, None),      # q_len 1, 32 heads per kv head
    (1, 16, 2, 40, 256, 4, 32, "f16", 4, True, None),         # 64 rows over two tiles of keys
    (3, 64, 2, 129, 256, 8, 32, "f16", 1, False, (5, 128, 129)),  # one key / no key left
], ids=["G16-q2-causal", "G16-q3-bf16-8b", "G4-q5-kvstart", "G32-q1-bf16", "G16-q4-N40", "G32-q1-kvstart"])
def test_row_blocks_match_oracle(device, case):
    """Two to four blocks of 16 query rows per kv head at D = 256 (the decode
    kernel's row blocks: several query positions, or more than 16 query
    heads per kv head), with causal masks and kv_start, against the oracle,
    at several split counts; repeated calls are bitwise identical."""
    B, Hq, Hkv, N, D, bits, gs, dtype, qL, causal, starts = case
    rng = np.random.default_rng(71 + qL + Hq)
    inp = make_inputs(rng, B, Hq, Hkv, N, D, bits, gs, dtype=dtype)
    inp["q"] = affine.random_T(rng, (B, Hq, qL, D), dtype)
    qi = np.arange(qL)[:, None] + (N - qL)
    keep = np.ones((B, 1, qL, N), dtype=bool)
    if causal:
        keep &= (qi >= np.arange(N)[None, :])[None, None]
    kw = {"causal": True} if causal else {}
    if starts is not None:
        st = np.array(starts)
        keep &= (np.arange(N)[None, :] >= np.clip(st, 0, N)[:, None])[:, None, None, :]
        kw["kv_start"] = torch.tensor(st, dtype=torch.int32, device=device)
    want = oracle_out(inp, mask=keep)
    want[~keep.any(axis=-1, keepdims=True).repeat(Hq, axis=1).repeat(D, axis=-1)] = 0.0
    for splits in (0, 1, 3, 7):
        got = _fused(inp, device, num_splits=splits, **kw)
        assert got.shape == (B, Hq, qL, D)
        assert_close(got, want, f"{case} splits={splits}")
        again = _fused(inp, device, num_splits=splits, **kw)
        assert np.array_equal(got, again), f"splits={splits}: repeated call differs"


@pytest.mark.parametrize("case", [
    # (B, Hq, Hkv, N, D, bits, gs, dtype, qL, causal, kv_start); calls with
    # 16K+ keys and 3 * 2^20 (row, key) pairs in all take this kernel at
    # D = 256, kv_start shortens the key range
    (1, 32, 2, 49200, 256, 4, 32, "f16", 2, True, None),        # 32 rows: one full block
    (2, 32, 2, 32768, 256, 4, 64, "bf16", 3, True, None),       # 48 rows: a half-filled second block
    (1, 16, 1, 33000, 256, 4, 128, "f16", 7, False, None),      # 112 rows, full attention
    (1, 2, 2, 81920, 256, 4, 32, "bf16", 20, True, (81270,)),   # G = 1: 20 positions over 650 keys
    (1, 8, 2, 45000, 256, 4, 64, "f16", 9, True, (333,)),       # 36 rows: 4 rows in block 2, kv_start
    (1, 16, 2, 40000, 256, 4, 32, "f16", 5, True, (39871,)),    # 40 rows over 129 keys
    (1, 32, 2, 32768, 256, 4, 32, "bf16", 4, True, (32765,)),   # 3 keys: the first rows see none
    (1, 16, 1, 24600, 256, 4, 32, "f16", 8, True, None),        # 128 rows over 24K keys
    # D = 128, 4- and 8-bit: 2^23 (row, key) pairs in all
    (4, 16, 4, 16400, 128, 8, 128, "bf16", 8, True, None),      # C5's heads: 32 rows
    (1, 8, 2, 131100, 128, 4, 64, "f16", 16, True, None),       # C1's heads: 64 rows over 128K keys
    (2, 16, 4, 70000, 128, 4, 32, "f16", 5, False, None),       # 20 rows, full attention
    (1, 4, 4, 140000, 128, 8, 64, "bf16", 20, True, (139300,)), # G = 1: 20 positions over 700 keys
    (1, 32, 8, 40000, 128, 4, 128, "bf16", 9, True, None),      # 36 rows: 4 in block 2
    # D = 128 left-padded batches: the stream-K schedule, an empty sequence
    (4, 16, 4, 32768, 128, 4, 64, "f16", 8, True, (0, 5000, 32000, 32768)),
    (3, 32, 8, 20000, 128, 8, 128, "bf16", 6, False, (100, 19990, 7)),
], ids=["G16-q2", "G16-q3-bf16", "G16-q7-full", "G1-q20-bf16", "G4-q9-kvstart", "G8-q5-129keys",
        "G16-q4-3keys-bf16", "G16-q8-N24K", "D128-c5-q8", "D128-c1-q16-128K", "D128-G4-q5-full",
        "D128-G1-q20-kvstart", "D128-G4-q9-bf16", "D128-streamK-q8", "D128-streamK-q6-bf16"])
def test_rows32_blocks_match_oracle(device, case):
    """More than 16 query rows per kv head over long caches, at D = 256
    with 4-bit codes and at D = 128: the 32-row kernel (both 16-row halves
    of a block from one dequantized tile, Q^T read from LDS), against the
    oracle at several split counts, with causal masks, kv_start and partial
    blocks; repeated calls are bitwise identical."""
    B, Hq, Hkv, N, D, bits, gs, dtype, qL, causal, starts = case
    rows = Hq // Hkv * qL
    enough = B * Hq * qL * N >= (1 << 23 if D == 128 else 3 << 20)
    assert 16 < rows < 128 or (D == 256 and B * Hq * qL * N < 1 << 24)  # not the prefill kernel's
    assert rows > 16 and N >= 16384 and enough
    rng = np.random.default_rng(91 + qL + Hq + N)
    inp = make_inputs(rng, B, Hq, Hkv, N, D, bits, gs, dtype=dtype)
    inp["q"] = affine.random_T(rng, (B, Hq, qL, D), dtype)
    qi = np.arange(qL)[:, None] + (N - qL)
    keep = np.ones((B, 1, qL, N), dtype=bool)
    if causal:
        keep &= (qi >= np.arange(N)[None, :])[None, None]
    kw = {"causal": True} if causal else {}
    if starts is not None:
        st = np.array(starts)
        keep &= (np.arange(N)[None, :] >= np.clip(st, 0, N)[:, None])[:, None, None, :]
        kw["kv_start"] = torch.tensor(st, dtype=torch.int32, device=device)
    want = oracle_out(inp, mask=keep)
    want[~keep.any(axis=-1, keepdims=True).repeat(Hq, axis=1).repeat(D, axis=-1)] = 0.0
    # The plan counts 32-row blocks: one workgroup per CU over B * H_kv * blocks.
    g = to_dev(inp, device)
    splits, _ = kernels.decode_plan(g["q"], g["kp"], g["vp"], g["ks"], g["vs"], g["kb"], g["vb"], scale=D ** -0.5,
                                    bits=bits, group_size=gs)
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    units = B * Hkv * ((rows + 31) // 32)
    assert splits == max(1, min(cus // units, max(1, N // 128))), splits
    for s in (0, 1, 3, 7):
        got = _fused(inp, device, num_splits=s, **kw)
        assert got.shape == (B, Hq, qL, D)
        assert_close(got, want, f"{case} splits={s}")
        again = _fused(inp, device, num_splits=s, **kw)
        assert np.array_equal(got, again), f"splits={s}: repeated call differs"


@pytest.mark.parametrize("case,mk", [
    ((4, 16, 4, 16400, 128, 8, 128, "bf16", 8), "bool"),
    ((2, 16, 4, 65600, 128, 4, 32, "f16", 8), "additive"),
    ((1, 8, 2, 120000, 128, 4, 64, "f16", 9), "bool-causal"),
], ids=["c5-q8-bool", "G4-q8-additive-per-head", "c1-q9-bool-causal"])
def test_rows32_masked_d128(device, case, mk):
    """Mask tensors on the 32-row kernel (D = 128): a bool mask broadcast
    over heads, an additive per-(head, position) mask with -inf entries, and
    a bool mask with the causal flag, against the oracle."""
    B, Hq, Hkv, N, D, bits, gs, dtype, qL = case
    assert Hq // Hkv * qL > 16 and N >= 16384 and B * Hq * qL * N >= 1 << 23
    rng = np.random.default_rng(97 + qL + N)
    inp = make_inputs(rng, B, Hq, Hkv, N, D, bits, gs, dtype=dtype)
    inp["q"] = affine.random_T(rng, (B, Hq, qL, D), dtype)
    kw = {}
    if mk.startswith("bool"):
        keep = rng.random((B, 1, qL, N)) < 0.7
        keep[..., -1] = True
        m_np, kw["mask"] = keep, torch.from_numpy(keep).to(device)
        if mk == "bool-causal":
            kw["causal"] = True
            qi = np.arange(qL)[:, None] + (N - qL)
            m_np = keep & (qi >= np.arange(N)[None, :])[None, None]
    else:
        add = (rng.standard_normal((1, Hq, qL, N)) * 2).astype(np.float32)
        add[rng.random(add.shape) < 0.2] = -np.inf
        add[..., -1] = 0.0
        add = add.astype(np.float16).astype(np.float32)
        m_np, kw["mask"] = add, torch.from_numpy(add).to(device, torch.float16)
    want = oracle_out(inp, mask=m_np)
    for s in (0, 1, 5):
        got = _fused(inp, device, num_splits=s, **kw)
        assert_close(got, want, f"{case} {mk} splits={s}")


def test_rows32_strided_views_and_symmetric(device):
    """The 32-row kernel over strided views: q and out as (B, qL, H, D)
    buffers seen as (B, H, qL, D), K / V in capacity-padded buffers, with
    and without biases (the symmetric format); bitwise equal to the same
    call on contiguous copies."""
    rng = np.random.default_rng(93)
    B, Hq, Hkv, N, cap, D, qL = 1, 32, 2, 49200, 49300, 256, 3
    assert B * Hq * qL * N >= 3 << 20
    for symmetric in (False, True):
        inp = make_inputs(rng, B, Hq, Hkv, N, D, 4, 32, symmetric=symmetric)
        inp["q"] = affine.random_T(rng, (B, Hq, qL, D), "f16")
        g = to_dev(inp, device)
        views = {}
        for k in ("kp", "vp", "ks", "vs", "kb", "vb"):
            t = g[k]
            if t is None:
                views[k] = None
                continue
            buf = torch.zeros((B, Hkv, cap, t.shape[-1]), dtype=t.dtype, device=device)
            buf[:, :, :N] = t
            views[k] = buf[:, :, :N]
        q_bshd = g["q"].transpose(1, 2).contiguous()
        q_view = q_bshd.transpose(1, 2)
        assert not q_view.is_contiguous()
        out_buf = torch.full((B, qL, Hq, D), float("nan"), dtype=torch.float16, device=device)
        out_view = out_buf.transpose(1, 2)
        kernels.decode(q_view, views["kp"], views["vp"], views["ks"], views["vs"], views["kb"], views["vb"],
                       scale=D ** -0.5, bits=4, group_size=32, causal=True, out=out_view)
        dense = kernels.decode(g["q"], g["kp"], g["vp"], g["ks"], g["vs"], g["kb"], g["vb"],
                               scale=D ** -0.5, bits=4, group_size=32, causal=True)
        torch.cuda.synchronize()
        assert torch.equal(out_view, dense), f"symmetric={symmetric}: strided call differs"
        assert_close(to_np(dense), oracle_out(inp, mask="causal"), f"rows32 symmetric={symmetric}")


@pytest.mark.parametrize("qL", [6, 40], ids=["q6", "q40-rows"])
def test_multi_query_kv_start_causal(device, qL):
    """qL > 1 with left padding and causal together (stream-K schedule when
    split; 160 rows per kv head at qL=40)."""
    rng = np.random.default_rng(47)
    B, Hq, Hkv, N, D = 4, 16, 4, 600, 128
    inp = make_inputs(rng, B, Hq, Hkv, N, D, 4, 64)
    inp["q"] = affine.random_T(rng, (B, Hq, qL, D), "f16")
    starts = np.array([0, 100, 597, 600])
    qi = np.arange(qL)[:, None] + (N - qL)
    keep = (np.arange(N)[None, None, :] >= starts[:, None, None]) & (qi >= np.arange(N)[None, :])[None]
    want = oracle_out(inp, mask=keep[:, None])
    ks = torch.tensor(starts, dtype=torch.int32, device=device)
    for splits in (0, 1, 4):
        assert_close(_fused(inp, device, kv_start=ks, num_splits=splits, causal=True), want,
                     f"kv_start causal splits={splits}")


def test_multi_query_routes_to_fused_kernel(device, monkeypatch):
    """quantized_sdpa with qL > 1 and mask="causal" runs the fused kernel
    (the dequantize + attention fallback is made to fail)."""
    from mlx_qsdpa_amd import dispatch

    def no_fallback(*a, **k):
        raise AssertionError("fallback used")

    monkeypatch.setattr(dispatch, "fallback_sdpa", no_fallback)
    rng = np.random.default_rng(48)
    inp = make_inputs(rng, 1, 8, 2, 256, 128, 4, 64)
    inp["q"] = affine.random_T(rng, (1, 8, 7, 128), "f16")
    got = run(inp, device, mask="causal")
    assert_close(got, oracle_out(inp, mask="causal"), "routed causal")


def test_fully_masked_row_is_zero(device):
    rng = np.random.default_rng(14)
    inp = make_inputs(rng, 2, 4, 2, 64, 128, 4, 32)
    keep = np.ones((2, 1, 1, 64), bool)
    keep[1] = False
    got = run(inp, device, mask=torch.from_numpy(keep).to(device))
    assert np.all(got[1] == 0) and np.isfinite(got).all()
    assert_close(got[0], oracle_out(inp, mask=keep)[0], "masked")


def test_strided_cache_views(device):
    """Views of capacity-padded buffers are read by stride (no copy)."""
    rng = np.random.default_rng(15)
    B, Hq, Hkv, N, cap, D = 2, 8, 2, 300, 512, 128
    inp = make_inputs(rng, B, Hq, Hkv, N, D, 4, 32)
    g = to_dev(inp, device)
    views = {}
    for k in ("kp", "vp", "ks", "vs", "kb", "vb"):
        t = g[k]
        buf = torch.zeros((B, Hkv, cap, t.shape[-1]), dtype=t.dtype, device=device)
        buf[:, :, :N] = t
        views[k] = buf[:, :, :N]
        assert not views[k].is_contiguous()
    out = mq.quantized_sdpa(g["q"], views["kp"], views["vp"], views["ks"], views["vs"],
                            views["kb"], views["vb"], bits=4, group_size=32)
    assert_close(to_np(out), oracle_out(inp), "strided")


def test_multi_query_through_quantized_sdpa(device):
    """qL > 1 through quantized_sdpa with aligned D = 128 inputs: the fused
    kernel, without a mask and with mask="causal".  (The dequantize +
    attention path for shapes the fused kernel does not take is covered by
    test_gpu_parity_full.py::test_multi_query_fallback_path.)"""
    rng = np.random.default_rng(16)
    inp = make_inputs(rng, 1, 4, 2, 64, 128, 4, 32)
    q = affine.random_T(rng, (1, 4, 8, 128), "f16")
    inp8 = dict(inp, q=q)
    g = to_dev(inp8, device)
    for mask in (None, "causal"):
        out = mq.quantized_sdpa(g["q"], g["kp"], g["vp"], g["ks"], g["vs"], g["kb"], g["vb"],
                                mask=mask)
        assert_close(to_np(out), oracle_out(inp8, mask=mask), f"prefill {mask}")


@pytest.mark.parametrize("N", [65536, 131072])
def test_headline_full_size_properties(device, N):
    """C3 at full N: vs the float64 oracle restated in torch (pinned to the
    numpy oracle in test_gpu_parity_full.py), split-K vs single pass, and
    invariance to a token permutation."""
    torch.manual_seed(0)
    B, Hq, Hkv, D, bits, gs = 1, 32, 2, 256, 4, 32
    T = torch.float16
    kw = torch.randn((B, Hkv, N, D), device=device).to(T)
    vw = torch.randn((B, Hkv, N, D), device=device).to(T)
    q = torch.randn((B, Hq, 1, D), device=device).to(T)
    kq = kernels.quantize(kw, gs, bits)
    vq = kernels.quantize(vw, gs, bits)
    out = mq.quantized_sdpa(q, kq[0], vq[0], kq[1], vq[1], kq[2], vq[2], bits=bits, group_size=gs)
    ref = torch_oracle.quantized_sdpa(q, kq, vq, bits=bits, group_size=gs)
    err = (out.double() - ref).abs()
    assert bool((err <= ATOL + RTOL * ref.abs()).all()), f"max err {err.max().item():.3e}"
    single = mq.quantized_sdpa(q, kq[0], vq[0], kq[1], vq[1], kq[2], vq[2], bits=bits,
                               group_size=gs, num_splits=1)
    assert (single.float() - out.float()).abs().max().item() < 2e-3
    perm = torch.randperm(N, device=device)

    def take(t):
        src = t.view(torch.int32) if t.dtype == torch.uint32 else t
        out = src.index_select(2, perm).contiguous()
        return out.view(torch.uint32) if t.dtype == torch.uint32 else out

    pq = [take(t) for t in kq], [take(t) for t in vq]
    outp = mq.quantized_sdpa(q, pq[0][0], pq[1][0], pq[0][1], pq[1][1], pq[0][2], pq[1][2],
                             bits=bits, group_size=gs)
    assert (outp.float() - out.float()).abs().max().item() < 2e-3


def test_c4_full_size_batched(device):
    """C4 at its full shape (B=16, H_q=32, H_kv=8, D=128, 4-bit gs64, lengths
    U[1K, 32K] left-padded): the stream-K decode vs the float64 oracle
    restated in torch with the padding masked, across split counts, and vs
    the same left padding given as a bool mask (uniform splits)."""
    torch.manual_seed(0)
    gen = torch.Generator(device="cpu")
    gen.manual_seed(0)
    B, Hq, Hkv, D, bits, gs = 16, 32, 8, 128, 4, 64
    lengths = torch.randint(1024, 32769, (B,), generator=gen)
    N = int(lengths.max())
    T = torch.float16
    kq = kernels.quantize(torch.randn((B, Hkv, N, D), device=device).to(T), gs, bits)
    vq = kernels.quantize(torch.randn((B, Hkv, N, D), device=device).to(T), gs, bits)
    q = torch.randn((B, Hq, 1, D), device=device).to(T)
    ks = (N - lengths).to(device=device, dtype=torch.int32)
    keep = torch.arange(N, device=device)[None, :] >= ks[:, None].long()
    ref = torch_oracle.quantized_sdpa(q, kq, vq, bits=bits, group_size=gs, mask=keep[:, None, None, :])
    outs = {}
    for splits in (None, 2, 4):
        out = mq.quantized_sdpa(q, kq[0], vq[0], kq[1], vq[1], kq[2], vq[2], bits=bits, group_size=gs,
                                kv_start=ks, num_splits=splits).double()
        err = (out - ref).abs()
        assert bool((err <= ATOL + RTOL * ref.abs()).all()), f"splits={splits}: max err {err.max().item():.3e}"
        outs[splits] = out
    masked = mq.quantized_sdpa(q, kq[0], vq[0], kq[1], vq[1], kq[2], vq[2], bits=bits, group_size=gs,
                               mask=keep[:, None, None, :]).double()
    assert (masked - outs[None]).abs().max().item() < 2e-3


@pytest.mark.parametrize("case", [(1, 32, 2, 4096, 256, 4, 32, "f16"), (2, 16, 4, 3000, 128, 8, 64, "bf16")],
                         ids=["C3_small", "B2_G4_bf16"])
def test_repeated_calls_reuse_workspace(device, case):
    """Split-K calls through one DecodePlan (one workspace, reused): every call
    gives the same output, within tolerance of the oracle."""
    B, Hq, Hkv, N, D, bits, gs, dt = case
    rng = np.random.default_rng(77)
    inp = make_inputs(rng, B, Hq, Hkv, N, D, bits, gs, dt)
    g = to_dev(inp, device)
    plan = kernels.DecodePlan(g["q"], g["kp"], g["vp"], g["ks"], g["vs"], g["kb"], g["vb"],
                              scale=D ** -0.5, bits=bits, group_size=gs, num_splits=0)
    assert plan.num_splits > 1
    outs = [plan().clone() for _ in range(4)]
    torch.cuda.synchronize()
    for o in outs[1:]:
        assert torch.equal(o, outs[0])
    assert_close(to_np(outs[0]), oracle_out(inp), f"{case}")


def test_plan_grows_in_place_with_appends(device):
    """A DecodePlan over a capacity-padded, left-padded batch cache: each step
    appends one token per sequence (qsdpa_quantize_batch, K and V in one
    launch), moves N with set_keys and decodes; every step matches the oracle
    on the first N keys with the padding masked.  N past the capacity is
    refused."""
    rng = np.random.default_rng(91)
    B, Hq, Hkv, D, bits, gs, n0, cap = 3, 8, 2, 128, 4, 64, 200, 260
    T = torch.float16
    starts = np.array([0, 150, 37])
    kw = affine.random_T(rng, (B, Hkv, cap, D), "f16")
    vw = affine.random_T(rng, (B, Hkv, cap, D), "f16")
    bufs = []
    for w in (kw, vw):
        p, s, b = (torch.zeros((B, Hkv, cap, D * bits // 32), dtype=torch.uint32, device=device),
                   torch.zeros((B, Hkv, cap, D // gs), dtype=T, device=device),
                   torch.zeros((B, Hkv, cap, D // gs), dtype=T, device=device))
        kernels.quantize_into(from_np(w[:, :, :n0], T, device), (p, s, b), 0, bits, gs)
        bufs.append((p, s, b))
    q = from_np(affine.random_T(rng, (B, Hq, 1, D), "f16"), T, device)
    ks = torch.tensor(starts, dtype=torch.int32, device=device)
    (kp, kss, kb), (vp, vs, vb) = bufs
    plan = kernels.DecodePlan(q, kp[:, :, :n0], vp[:, :, :n0], kss[:, :, :n0], vs[:, :, :n0],
                              kb[:, :, :n0], vb[:, :, :n0], scale=D ** -0.5, bits=bits, group_size=gs,
                              kv_start=ks, num_splits=3, capacity=cap)
    for n in range(n0, n0 + 3):
        kernels.quantize_kv_into(from_np(kw[:, :, n:n + 1], T, device), from_np(vw[:, :, n:n + 1], T, device),
                                 bufs[0], bufs[1], n, bits, gs)
        plan.set_keys(n + 1)
        got = to_np(plan())
        inp = dict(q=to_np(q), kp=to_np(kp[:, :, :n + 1]), vp=to_np(vp[:, :, :n + 1]),
                   ks=to_np(kss[:, :, :n + 1]), vs=to_np(vs[:, :, :n + 1]), kb=to_np(kb[:, :, :n + 1]),
                   vb=to_np(vb[:, :, :n + 1]), bits=bits, gs=gs, dtype="f16")
        add = np.where(np.arange(n + 1)[None, :] >= starts[:, None], 0.0, -np.inf)[:, None, None, :]
        assert_close(got, oracle_out(inp, mask=add), f"n={n + 1}")
    with pytest.raises(ValueError):
        plan.set_keys(cap + 1)


def test_decode_argument_cache(device):
    """kernels.decode re-launches a cached argument block for a repeated
    tensor geometry (key count free): every cached call, over a growing key
    count, with kv_start and on a second stream, equals the uncached call
    bit for bit and the oracle to tolerance."""
    rng = np.random.default_rng(61)
    B, Hq, Hkv, D, bits, gs, cap = 2, 16, 2, 128, 4, 64, 3000
    inp = make_inputs(rng, B, Hq, Hkv, cap, D, bits, gs)
    g = to_dev(inp, device)
    ks = torch.tensor([0, 37], dtype=torch.int32, device=device)
    side = torch.cuda.Stream(device)

    def call(n, kv_start, cached):
        if not cached:
            kernels._ARGS.d = {}
        v = [g[k][:, :, :n] for k in ("kp", "vp", "ks", "vs", "kb", "vb")]
        return kernels.decode(g["q"], *v, scale=D ** -0.5, bits=bits, group_size=gs, kv_start=kv_start)

    for kv_start in (None, ks):
        for n in (100, 2047, 2048, 3000, 64, 1):
            print(f"argument cache n={n} kv_start={kv_start is not None}", flush=True)
            want = call(n, kv_start, cached=False)
            got = call(n, kv_start, cached=True)       # hit (cached by the call above)
            nxt = call(min(n + 1, cap), kv_start, cached=True)  # hit with another key count
            with torch.cuda.stream(side):
                other = call(n, kv_start, cached=True)  # a new entry for the other stream
            torch.cuda.synchronize()
            assert torch.equal(got, want), f"n={n}: cached call differs"
            assert torch.equal(other, want), f"n={n}: other stream differs"
            sub = {k: (None if inp[k] is None else inp[k][:, :, :min(n + 1, cap)]) for k in inp
                   if k in ("kp", "vp", "ks", "vs", "kb", "vb")}
            ref_in = dict(inp, **sub)
            mask = None
            if kv_start is not None:
                mask = np.arange(min(n + 1, cap))[None, None, None, :] >= np.array([0, 37])[:, None, None, None]
                if min(n + 1, cap) <= 37:
                    continue  # sequence 1 has no keys: its row is all-masked
            assert_close(to_np(nxt), oracle_out(ref_in, mask=mask), f"n={n + 1} cached")


def test_argument_cache_keys_on_alignment(device):
    """A cached argument block is re-used only for views with the same
    pointer alignment: the same geometry with q, or the K scales, one
    element (2 bytes) off a 4-byte boundary takes another plan (the
    matrix-core kernel reads them as 32-bit words), and each call still
    matches the oracle, before and after the aligned block is cached."""
    rng = np.random.default_rng(62)
    B, Hq, Hkv, N, D, bits, gs = 1, 16, 2, 4000, 256, 4, 32
    inp = make_inputs(rng, B, Hq, Hkv, N, D, bits, gs)
    g = to_dev(inp, device)
    want = oracle_out(inp)

    def shifted(t):
        """t's values in a view with t's strides, 2 bytes past a 4-byte boundary."""
        wide = torch.empty(t.numel() + 1, dtype=t.dtype, device=device)
        wide[1:] = t.reshape(-1)
        v = wide[1:].view(t.shape)
        assert v.stride() == t.stride() and v.data_ptr() % 4 == 2
        return v

    kernels._ARGS.d = {}
    for name in ("q", "ks"):
        for order in ("aligned first", "shifted first"):
            print(f"alignment key: {name} {order}", flush=True)
            kernels._ARGS.d = {}
            alt = dict(g, **{name: shifted(g[name])})
            seq = (g, alt, g, alt) if order == "aligned first" else (alt, g, alt, g)
            for t in seq:
                out = mq.quantized_sdpa(t["q"], t["kp"], t["vp"], t["ks"], t["vs"], t["kb"], t["vb"],
                                        bits=bits, group_size=gs)
                torch.cuda.synchronize()
                assert_close(to_np(out), want, f"{name} {order}")
