"""The prefill kernel (many query positions per kv head, D = 128 with 64-key
tiles, D = 256 with 32-key tiles) against the float64 oracle
(tests/torch_oracle.py, pinned to the numpy oracle by
tests/test_gpu_parity_full.py).

Shapes are chosen so the library routes them to the prefill kernel: at
least one full 128-row group per kv head (H_q / H_kv x q_len), with one
pass where the groups fill the GPU and key splits (merged by the split-K
merge kernel) where they do not.  Covered: both dtypes, 4- and 8-bit codes, all
group sizes, the symmetric format, causal and full attention, kv_start
(left padding), bool and additive masks, a partial last row group, a
partial last key tile, keys that start inside a tile, key ranges of one to
three tiles, huge K scales, and the C5 chunk.
Tolerance: |out - ref| <= 2e-3 + 1e-2 |ref|.
"""

import pytest
import torch

import torch_oracle as to

from mlx_qsdpa_amd import kernels

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-3, 1e-2


def _inputs(B, Hq, Hkv, N, L, bits, gs, dtype, seed, symmetric=False, D=128):
    g = torch.Generator(device="cpu").manual_seed(seed)
    dev = torch.device("cuda:0")
    q = torch.randn(B, Hq, L, D, generator=g).to(dtype).to(dev)
    kw = torch.randn(B, Hkv, N, D, generator=g)
    kw[..., :3] *= 6.0  # a few large channels: scores with a spread
    vw = torch.randn(B, Hkv, N, D, generator=g)
    kq = kernels.quantize(kw.to(dtype).to(dev), gs, bits)
    vq = kernels.quantize(vw.to(dtype).to(dev), gs, bits)
    if symmetric:
        kq, vq = (kq[0], kq[1], None), (vq[0], vq[1], None)
    return q, kq, vq


def _check(q, kq, vq, bits, gs, ctx, mask=None, causal=False, kv_start=None):
    D = q.shape[-1]
    out = kernels.decode(q, kq[0], vq[0], kq[1], vq[1], kq[2], vq[2], scale=D ** -0.5, bits=bits,
                         group_size=gs, mask=mask, kv_start=kv_start, causal=causal)
    ref_mask = mask
    N, L = kq[0].shape[2], q.shape[2]
    keep = None
    if causal:
        keep = torch.arange(N, device=q.device)[None, :] <= (N - L) + torch.arange(L, device=q.device)[:, None]
        keep = keep[None, None]
    if kv_start is not None:
        ks = torch.arange(N, device=q.device)[None, :] >= kv_start.to(q.device).long()[:, None]
        ks = ks[:, None, None, :]
        keep = ks if keep is None else keep & ks
    if keep is not None:
        if ref_mask is None:
            ref_mask = keep
        elif ref_mask.dtype == torch.bool:
            ref_mask = ref_mask & keep
        else:
            ref_mask = ref_mask.float().masked_fill(~keep, float("-inf"))
    want = to.quantized_sdpa(q, kq, vq, bits=bits, group_size=gs, scale=D ** -0.5, mask=ref_mask)
    torch.cuda.synchronize()
    err = (out.double() - want).abs()
    bound = ATOL + RTOL * want.abs()
    bad = err > bound
    assert not bool(bad.any()), f"{ctx}: {int(bad.sum())} outside tolerance, max err {float(err.max()):.3e}"
    assert bool(torch.isfinite(out).all()), ctx


CASES = [  # (B, Hq, Hkv, N, L, bits, gs, dtype, causal, symmetric)
    (2, 32, 8, 1000, 256, 4, 64, torch.float16, True, False),
    (2, 32, 8, 777, 256, 4, 32, torch.float16, True, False),
    (2, 32, 8, 1024, 200, 8, 128, torch.bfloat16, True, False),   # last row group partial
    (4, 16, 4, 4096, 512, 8, 128, torch.bfloat16, True, False),   # the C5 chunk
    (4, 16, 4, 2111, 512, 4, 128, torch.bfloat16, False, False),
    (2, 32, 8, 700, 256, 8, 32, torch.float16, False, True),
    (1, 64, 8, 600, 512, 4, 64, torch.bfloat16, True, True),
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: "B{}_H{}x{}_N{}_L{}_b{}_g{}_{}_{}{}".format(
    *c[:7], str(c[7]).split(".")[-1], "causal" if c[8] else "full", "_sym" if c[9] else ""))
def test_prefill_matches_oracle(device, case):
    B, Hq, Hkv, N, L, bits, gs, dtype, causal, sym = case
    print(f"prefill case {case}", flush=True)
    q, kq, vq = _inputs(B, Hq, Hkv, N, L, bits, gs, dtype, seed=N + L, symmetric=sym)
    _check(q, kq, vq, bits, gs, f"case {case}", causal=causal)


SPLIT_CASES = [  # small grids: the planner gives each row group several key splits
    (1, 32, 8, 4000, 256, 4, 64, torch.float16, True, False),     # 64 groups: 4 splits
    (1, 16, 4, 3000, 128, 8, 128, torch.bfloat16, True, False),   # 16 groups: 11 splits
    (2, 16, 4, 2500, 128, 4, 32, torch.float16, False, True),     # 32 groups, full attention: 8 splits
    (2, 16, 4, 2500, 256, 8, 64, torch.bfloat16, True, False),    # 64 groups: 4 splits, bfloat16
    (1, 8, 2, 40010, 32, 4, 64, torch.float16, True, False),      # 2 groups: 128 splits, merge kernel
]


@pytest.mark.parametrize("case", SPLIT_CASES, ids=lambda c: "B{}_H{}x{}_N{}_L{}_b{}_g{}".format(*c[:7]))
def test_prefill_key_splits(device, case):
    B, Hq, Hkv, N, L, bits, gs, dtype, causal, sym = case
    q, kq, vq = _inputs(B, Hq, Hkv, N, L, bits, gs, dtype, seed=N + 7, symmetric=sym)
    splits, ws = kernels.decode_plan(q, kq[0], vq[0], kq[1], vq[1], kq[2], vq[2], scale=128 ** -0.5, bits=bits,
                                     group_size=gs)
    print(f"prefill split case {case}: {splits} splits", flush=True)
    assert splits > 1 and ws > 0
    _check(q, kq, vq, bits, gs, f"split case {case}", causal=causal)
    if causal:
        ks = torch.tensor([0, 611][:B], dtype=torch.int32, device=device)
        _check(q, kq, vq, bits, gs, f"split case {case} kv_start", causal=True, kv_start=ks)


@pytest.mark.parametrize("N", [1, 63, 64, 65, 130, 191])
def test_prefill_short_key_ranges(device, N):
    """One to three 64-key tiles (full and partial): the pipeline dequantizes
    two tiles ahead into four LDS buffers, so the first pair's stages and
    loads reach past the last tile.  Full attention and causal, where qL > N
    leaves the first positions without keys (rows of zeros)."""
    B, Hq, Hkv, L, bits, gs = 1, 16, 4, 128, 8, 128
    for dtype in (torch.bfloat16, torch.float16):
        q, kq, vq = _inputs(B, Hq, Hkv, N, L, bits, gs, dtype, seed=N)
        print(f"prefill short N={N} {dtype}", flush=True)
        _check(q, kq, vq, bits, gs, f"short N={N} {dtype}")
        _check(q, kq, vq, bits, gs, f"short N={N} {dtype} causal", causal=True)


def test_prefill_kv_start_and_masks(device):
    B, Hq, Hkv, N, L, bits, gs = 2, 32, 8, 900, 256, 4, 64
    for dtype in (torch.float16, torch.bfloat16):
        q, kq, vq = _inputs(B, Hq, Hkv, N, L, bits, gs, dtype, seed=11)
        ks = torch.tensor([37, 300], dtype=torch.int32, device=device)  # starts inside a tile
        print(f"prefill kv_start {dtype}", flush=True)
        _check(q, kq, vq, bits, gs, f"kv_start {dtype}", kv_start=ks, causal=True)
        g = torch.Generator(device="cpu").manual_seed(12)
        keep = torch.rand(B, 1, L, N, generator=g) < 0.8
        keep[..., -1] = True  # no all-masked rows
        print(f"prefill bool mask {dtype}", flush=True)
        _check(q, kq, vq, bits, gs, f"bool mask {dtype}", mask=keep.to(device), causal=True)
        add = (torch.randn(1, Hq, L, N, generator=g) * 3).to(dtype).to(device)
        print(f"prefill additive mask {dtype}", flush=True)
        _check(q, kq, vq, bits, gs, f"additive mask {dtype}", mask=add)


@pytest.mark.parametrize("case", [
    # (shape B, H_q, H_kv, N, L; V scale; scale of 4 outlier channels; tolerance)
    ((2, 32, 8, 900, 256), 1.0, 8.0, "parity"),          # max |V| ~ 40: P in two float16 terms
    ((2, 32, 8, 900, 256), 2.0e4, 40.0, "scaled"),       # max |V| ~ 3e6: V staged at 2^-6
    ((1, 16, 4, 3000, 128), 2.0e4, 40.0, "scaled"),      # the same through 11 key splits (merge kernel)
    ((2, 32, 8, 2500, 128), 2.0e4, 40.0, "scaled"),      # 4 key splits (merge_rows_kernel)
    ((2, 32, 8, 900, 256), 2.0e36, 4.0, "scaled"),       # max |V| ~ 4e37: V staged at 2^-119
], ids=["outliers", "beyond_f16", "beyond_f16_splits", "beyond_f16_4_splits", "near_bf16_max"])
def test_prefill_bf16_large_values(device, case):
    """bfloat16 V with large values.  Past max |V| = 8 the kernel feeds P to
    the P.V MFMAs as two float16 terms (22 significant bits), and past
    64000 it stages V in float16 scaled by 2^-k and scales the output (or the
    float32 partials) back by 2^k (k up to 113 for any finite bfloat16 V,
    exercised near the bfloat16 maximum).  With outlier channels the parity bar
    holds; at |V| ~ 1e6 no float P meets an absolute 2e-3 where outputs
    cancel, so the bar there is 2^-20 max|V| (22-bit P moves an output by up to
    2^-22 max|V|) plus the relative 1e-2: a wrong scale would miss it by
    orders of magnitude."""
    (B, Hq, Hkv, N, L), vmul, omul, tol = case
    g = torch.Generator(device="cpu").manual_seed(21)
    q = torch.randn(B, Hq, L, 128, generator=g).bfloat16().to(device)
    kw = torch.randn(B, Hkv, N, 128, generator=g)
    vw = torch.randn(B, Hkv, N, 128, generator=g) * vmul
    vw[..., :4] *= omul
    kq = kernels.quantize(kw.bfloat16().to(device), 64, 8)
    vq = kernels.quantize(vw.bfloat16().to(device), 64, 8)
    print(f"prefill bf16 large V {case}", flush=True)
    if tol == "parity":
        _check(q, kq, vq, 8, 64, f"large V {case}", causal=True)
        return
    out = kernels.decode(q, kq[0], vq[0], kq[1], vq[1], kq[2], vq[2], scale=128 ** -0.5, bits=8, group_size=64,
                         causal=True)
    keep = torch.arange(N, device=device)[None, :] <= (N - L) + torch.arange(L, device=device)[:, None]
    want = to.quantized_sdpa(q, kq, vq, bits=8, group_size=64, scale=128 ** -0.5, mask=keep[None, None])
    vmax = float(kernels.dequantize(vq[0], vq[1], vq[2], 64, 8).float().abs().max())
    err = (out.double() - want).abs()
    bound = 2.0 ** -20 * vmax + RTOL * want.abs()
    assert bool(torch.isfinite(out).all())
    assert bool((err <= bound).all()), f"{case}: max err {float(err.max()):.4g} (max |V| {vmax:.3g})"


@pytest.mark.parametrize("bits,gs", [(8, 64), (4, 128)])
def test_prefill_bf16_huge_k_scales(device, bits, gs):
    """bfloat16 K groups with scales of 2^101 and more.  The kernel's
    dequantization multiplies each scale by 2^24 (codes read as float16
    subnormals); a wave with a scale at or above 2^100 takes the plain
    float32 path instead, whose values are finite where the scaled one would
    overflow.  Keys 64-127 (whole waves of a tile) and every seventh key
    (most waves) carry such groups, with values near 2^109 (8-bit) or 2^105
    (4-bit); queries scaled to match keep their scores near 1, so the
    softmax mixes them and the normal keys (scores near 0): a wrong K value
    shows as a wrong output or a NaN."""
    B, Hq, Hkv, N, L = 2, 32, 8, 900, 256
    q, kq, vq = _inputs(B, Hq, Hkv, N, L, bits, gs, torch.bfloat16, seed=31)
    q = (q.float() * 2.0 ** (-108 if bits == 8 else -104)).bfloat16()
    huge = torch.zeros(N, dtype=torch.bool)
    huge[64:128] = True
    huge[::7] = True
    g = torch.Generator(device="cpu").manual_seed(32)
    ks, kb = kq[1].clone(), kq[2].clone()
    shape = (B, Hkv, int(huge.sum()), ks.shape[-1])
    s = (2.0 ** 101 * (1.0 + torch.rand(shape, generator=g))).bfloat16().to(device)
    ks[:, :, huge.to(device)] = s
    kb[:, :, huge.to(device)] = (-(2 ** (bits - 1)) * s.float()).bfloat16()
    kq = (kq[0], ks, kb)
    print(f"prefill huge K scales bits={bits} gs={gs}", flush=True)
    _check(q, kq, vq, bits, gs, f"huge K scales {bits}-bit", causal=True)


def test_prefill_repeatable(device):
    """Repeated calls give bit-identical outputs."""
    q, kq, vq = _inputs(4, 16, 4, 4096, 512, 8, 128, torch.bfloat16, seed=5)
    outs = [kernels.decode(q, kq[0], vq[0], kq[1], vq[1], kq[2], vq[2], scale=128 ** -0.5, bits=8,
                           group_size=128, causal=True) for _ in range(3)]
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1]) and torch.equal(outs[0], outs[2])


# D = 256: 32-key tiles, the same 128-row groups.  The library sends a
# D = 256 call here when its kv heads have two or more row groups (H_q /
# H_kv x q_len >= 256) and it has at least 2^24 (query row, key) pairs
# (B x H_q x q_len x N); the shapes below meet both.  (B, Hq, Hkv, N, L,
# bits, gs, dtype, causal, symmetric)
D256_PAIRS = 1 << 24
D256_CASES = [
    (1, 32, 2, 33000, 16, 4, 32, torch.float16, True, False),     # C3's heads, 2 groups: key splits
    (2, 16, 4, 8300, 64, 8, 64, torch.bfloat16, True, False),     # partial last tile
    (1, 2, 2, 16411, 512, 8, 64, torch.bfloat16, False, False),   # C2's heads (G = 1), full attention
    (2, 8, 2, 2700, 400, 4, 128, torch.float16, True, True),      # 1600 rows: partial last group
    (4, 16, 4, 2100, 128, 4, 64, torch.bfloat16, True, False),
    (1, 32, 8, 8200, 64, 8, 32, torch.float16, False, False),
    (1, 32, 2, 65611, 8, 8, 32, torch.float16, True, False),      # one group per kv head: 128 key splits
    (1, 2, 2, 65601, 128, 8, 64, torch.bfloat16, True, False),    # C2's heads, one group: 128 key splits
]


def _d256_routed(B, Hq, Hkv, N, L, bits=4):
    """The call meets the D = 256 prefill routing (unmasked): two row groups
    per kv head, or one with 8-bit codes (4-bit single groups go to the
    32-row decode kernel), and 2^24 (row, key) pairs."""
    rows = Hq // Hkv * L
    return (rows >= 256 or (rows >= 128 and bits == 8)) and B * Hq * L * N >= D256_PAIRS


@pytest.mark.parametrize("case", D256_CASES, ids=lambda c: "B{}_H{}x{}_N{}_L{}_b{}_g{}_{}_{}{}".format(
    *c[:7], str(c[7]).split(".")[-1], "causal" if c[8] else "full", "_sym" if c[9] else ""))
def test_prefill_d256_matches_oracle(device, case):
    B, Hq, Hkv, N, L, bits, gs, dtype, causal, sym = case
    assert _d256_routed(B, Hq, Hkv, N, L, bits)
    print(f"prefill D=256 case {case}", flush=True)
    q, kq, vq = _inputs(B, Hq, Hkv, N, L, bits, gs, dtype, seed=N + L + 256, symmetric=sym, D=256)
    _check(q, kq, vq, bits, gs, f"D=256 case {case}", causal=causal)


@pytest.mark.parametrize("keys", [1, 31, 32, 33, 65, 95])
def test_prefill_d256_short_key_ranges(device, keys):
    """One to three 32-key tiles at D = 256 (the pipeline's loads and stages
    reach past the last tile): a long cache whose kv_start leaves `keys`
    keys, with full attention and causal (where q_len > keys leaves the
    first positions without keys: rows of zeros)."""
    B, Hq, Hkv, N, L, bits, gs = 1, 16, 2, 33000, 32, 4, 64
    assert _d256_routed(B, Hq, Hkv, N, L)
    ks = torch.tensor([N - keys], dtype=torch.int32, device=device)
    for dtype in (torch.bfloat16, torch.float16):
        q, kq, vq = _inputs(B, Hq, Hkv, N, L, bits, gs, dtype, seed=keys + 256, D=256)
        print(f"prefill D=256 short keys={keys} {dtype}", flush=True)
        _check(q, kq, vq, bits, gs, f"D=256 short keys={keys} {dtype}", kv_start=ks)
        _check(q, kq, vq, bits, gs, f"D=256 short keys={keys} {dtype} causal", kv_start=ks, causal=True)


def test_prefill_d256_kv_start_and_masks(device):
    B, Hq, Hkv, N, L, bits, gs = 2, 16, 2, 16500, 32, 8, 32
    assert _d256_routed(B, Hq, Hkv, N, L, bits)
    for dtype in (torch.float16, torch.bfloat16):
        q, kq, vq = _inputs(B, Hq, Hkv, N, L, bits, gs, dtype, seed=13, D=256)
        ks = torch.tensor([19, 9000], dtype=torch.int32, device=device)  # starts inside a tile
        print(f"prefill D=256 kv_start {dtype}", flush=True)
        _check(q, kq, vq, bits, gs, f"D=256 kv_start {dtype}", kv_start=ks, causal=True)
        g = torch.Generator(device="cpu").manual_seed(14)
        keep = torch.rand(B, 1, L, N, generator=g) < 0.8
        keep[..., -1] = True
        print(f"prefill D=256 bool mask {dtype}", flush=True)
        _check(q, kq, vq, bits, gs, f"D=256 bool mask {dtype}", mask=keep.to(device), causal=True)
        add = (torch.randn(1, Hq, L, N, generator=g) * 3).to(dtype).to(device)
        print(f"prefill D=256 additive mask {dtype}", flush=True)
        _check(q, kq, vq, bits, gs, f"D=256 additive mask {dtype}", mask=add)


@pytest.mark.parametrize("vmul,omul,tol", [(1.0, 8.0, "parity"), (2.0e4, 40.0, "scaled")],
                         ids=["outliers", "beyond_f16"])
def test_prefill_d256_bf16_large_values(device, vmul, omul, tol):
    """bfloat16 V past max |V| = 8 (P as two float16 terms) and past 64000
    (V staged at 2^-k) at D = 256; the bars as in the D = 128 test."""
    B, Hq, Hkv, N, L = 2, 16, 2, 16500, 32
    assert _d256_routed(B, Hq, Hkv, N, L)
    g = torch.Generator(device="cpu").manual_seed(23)
    q = torch.randn(B, Hq, L, 256, generator=g).bfloat16().to(device)
    kw = torch.randn(B, Hkv, N, 256, generator=g)
    vw = torch.randn(B, Hkv, N, 256, generator=g) * vmul
    vw[..., :4] *= omul
    kq = kernels.quantize(kw.bfloat16().to(device), 64, 8)
    vq = kernels.quantize(vw.bfloat16().to(device), 64, 8)
    print(f"prefill D=256 bf16 large V {vmul} {omul}", flush=True)
    if tol == "parity":
        _check(q, kq, vq, 8, 64, "D=256 large V", causal=True)
        return
    out = kernels.decode(q, kq[0], vq[0], kq[1], vq[1], kq[2], vq[2], scale=256 ** -0.5, bits=8, group_size=64,
                         causal=True)
    keep = torch.arange(N, device=device)[None, :] <= (N - L) + torch.arange(L, device=device)[:, None]
    want = to.quantized_sdpa(q, kq, vq, bits=8, group_size=64, scale=256 ** -0.5, mask=keep[None, None])
    vmax = float(kernels.dequantize(vq[0], vq[1], vq[2], 64, 8).float().abs().max())
    err = (out.double() - want).abs()
    bound = 2.0 ** -20 * vmax + RTOL * want.abs()
    assert bool(torch.isfinite(out).all())
    assert bool((err <= bound).all()), f"D=256 large V: max err {float(err.max()):.4g} (max |V| {vmax:.3g})"


def test_prefill_d256_bf16_huge_k_scales(device):
    """K groups with scales of 2^101 and more at D = 256 (the float32
    dequantization path for the waves that hold them)."""
    B, Hq, Hkv, N, L, bits, gs = 1, 16, 2, 33000, 32, 8, 64
    assert _d256_routed(B, Hq, Hkv, N, L, bits)
    q, kq, vq = _inputs(B, Hq, Hkv, N, L, bits, gs, torch.bfloat16, seed=33, D=256)
    q = (q.float() * 2.0 ** -108).bfloat16()
    huge = torch.zeros(N, dtype=torch.bool)
    huge[32:64] = True
    huge[-64:-32] = True
    huge[::7] = True
    g = torch.Generator(device="cpu").manual_seed(34)
    ks, kb = kq[1].clone(), kq[2].clone()
    shape = (B, Hkv, int(huge.sum()), ks.shape[-1])
    s = (2.0 ** 101 * (1.0 + torch.rand(shape, generator=g))).bfloat16().to(device)
    ks[:, :, huge.to(device)] = s
    kb[:, :, huge.to(device)] = (-(2 ** (bits - 1)) * s.float()).bfloat16()
    kq = (kq[0], ks, kb)
    print("prefill D=256 huge K scales", flush=True)
    _check(q, kq, vq, bits, gs, "D=256 huge K scales", causal=True)


def test_prefill_d256_repeatable(device):
    """Repeated D = 256 calls (one pass and key splits) give bit-identical outputs."""
    for (B, Hq, Hkv, N, L) in [(4, 16, 4, 2100, 128), (1, 32, 2, 33000, 16)]:
        assert _d256_routed(B, Hq, Hkv, N, L)
        q, kq, vq = _inputs(B, Hq, Hkv, N, L, 4, 32, torch.float16, seed=6, D=256)
        outs = [kernels.decode(q, kq[0], vq[0], kq[1], vq[1], kq[2], vq[2], scale=256 ** -0.5, bits=4,
                               group_size=32, causal=True) for _ in range(3)]
        torch.cuda.synchronize()
        assert torch.equal(outs[0], outs[1]) and torch.equal(outs[0], outs[2])


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_prefill_split_merge_unaligned_out(device, dtype):
    """Key splits merged by the row merge into an output whose rows are not
    aligned (a view one element into wider rows: 16-bit stores) give the
    same bits as into a contiguous output (one store per 8 values of
    float16 partial rows, per 4 of float32 ones)."""
    B, Hq, Hkv, N, L, bits, gs = 1, 32, 8, 4000, 256, 4, 64   # 4 key splits, 8192 rows
    q, kq, vq = _inputs(B, Hq, Hkv, N, L, bits, gs, dtype, seed=77)
    args = dict(scale=128 ** -0.5, bits=bits, group_size=gs, causal=True)
    splits, _ = kernels.decode_plan(q, kq[0], vq[0], kq[1], vq[1], kq[2], vq[2], scale=128 ** -0.5, bits=bits,
                                    group_size=gs)
    assert 1 < splits <= 16
    ref = kernels.decode(q, kq[0], vq[0], kq[1], vq[1], kq[2], vq[2], **args)
    wide = torch.zeros(B, Hq, L, 128 + 2, dtype=q.dtype, device=device)
    out = wide[..., 1:129]
    kernels.decode(q, kq[0], vq[0], kq[1], vq[1], kq[2], vq[2], out=out, **args)
    torch.cuda.synchronize()
    assert torch.equal(out, ref)
    assert bool((wide[..., 0] == 0).all()) and bool((wide[..., 129] == 0).all())
