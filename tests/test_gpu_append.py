"""The one-token append folded into the decode (qsdpa_decode_args.k_new /
v_new, DecodePlan(append=...)): the cache update of a decode step
(update_and_fetch, mlx_qsdpa/cache.py:279-322) and the attention over the
updated cache in one call.

Over three steps of a capacity-padded cache (rows past the valid ones hold
garbage that the append must overwrite), after every call:

* every valid row of the caches -- codes, scales, biases -- is bit-exact
  against the numpy quantizer (oracle/affine.py) of the same T values, the
  appended row included, and rows past it are untouched;
* the output is within tolerance of the float64 oracle over the valid keys
  (kv_start masks a sequence's left padding; a sequence whose kv_start is
  past every key returns zeros).

Cases: inside the decode launch (D = 128, one row block per kv head: the
stream-K schedule of a left-padded batch, uniform splits, a single pass,
sequences without keys) and through the quantize launch that precedes the
decode where the kernel does not take it (D = 256, D = 64, two row blocks,
a mask tensor, new rows not 16-byte aligned).
"""

import numpy as np
import pytest
import torch

from conftest import from_np, to_np, torch_dtype
from oracle import affine, attention

from mlx_qsdpa_amd import kernels

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-3, 1e-2
GARBAGE = 0x5A5A5A5A


def _bits_equal(got, want, dt):
    if want.dtype == np.uint32:
        return np.array_equal(got, want)
    return np.array_equal(affine.T_bits(got, dt), affine.T_bits(want, dt))


CASES = [
    # B, H_q, H_kv, D, bits, gs, dtype, n0, kv_start, num_splits, how
    (4, 16, 4, 128, 4, 64, "f16", 300, [0, 100, 37, 250], 2, "plan"),        # stream-K, merge inside
    (3, 32, 8, 128, 8, 128, "bf16", 700, [5, 0, 690], 3, "plan"),           # stream-K, bf16 8-bit
    (3, 8, 2, 128, 4, 32, "f16", 200, [0, 10, 10 ** 6], 2, "plan"),         # a sequence with no keys
    (1, 16, 2, 128, 4, 64, "f16", 1000, None, 0, "plan"),                   # uniform splits
    (1, 4, 4, 128, 8, 64, "bf16", 150, None, 1, "plan"),                    # single pass, G = 1
    (1, 4, 1, 128, 4, 64, "f16", 90, [10 ** 6], 3, "plan"),                 # uniform, no keys in range
    (2, 32, 2, 256, 4, 32, "f16", 400, [0, 33], 2, "plan"),                 # D = 256: quantize launch
    (2, 8, 2, 64, 4, 32, "bf16", 120, None, 0, "plan"),                     # D = 64 (VALU kernel)
    (2, 64, 2, 128, 4, 64, "f16", 300, None, 0, "plan"),                    # two row blocks per kv head
    (2, 16, 4, 128, 4, 64, "f16", 260, [0, 20], 0, "mask"),                 # mask tensor
    (2, 16, 4, 128, 4, 64, "bf16", 260, [3, 0], 2, "unaligned"),            # new rows 2 bytes off
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"B{c[0]}_G{c[1] // c[2]}_D{c[3]}_{c[4]}b_gs{c[5]}_{c[6]}_"
                         f"{'ks' if c[8] else 'noks'}_s{c[9]}_{c[10]}")
def test_append_in_decode(device, case):
    B, Hq, Hkv, D, bits, gs, dt, n0, starts, splits, how = case
    T = torch_dtype(dt)
    rng = np.random.default_rng(n0 + D + bits)
    steps = 3 if how != "mask" else 1
    cap = n0 + 4
    kw = affine.random_T(rng, (B, Hkv, cap, D), dt)
    vw = affine.random_T(rng, (B, Hkv, cap, D), dt)
    kq = affine.quantize(kw, gs, bits, dt)
    vq = affine.quantize(vw, gs, bits, dt)

    def buffers(quant):
        """Device caches holding the first n0 rows of `quant`, garbage after."""
        out = []
        for x in quant:
            t = from_np(x, T, device)
            if t.dtype == torch.uint32:
                t.view(torch.int32)[:, :, n0:] = GARBAGE
            else:
                t[:, :, n0:] = float("nan")
            out.append(t)
        return out

    kbuf, vbuf = buffers(kq), buffers(vq)
    q = from_np(affine.random_T(rng, (B, Hq, 1, D), dt), T, device)
    ks = None if starts is None else torch.tensor(starts, dtype=torch.int32, device=device)
    if how == "unaligned":
        wide = [torch.empty(B * Hkv * D + 1, dtype=T, device=device) for _ in range(2)]
        new = [w[1:].view(B, Hkv, 1, D) for w in wide]
        assert new[0].data_ptr() % 16 == 2
    else:
        new = [torch.empty((B, Hkv, 1, D), dtype=T, device=device) for _ in range(2)]
    views = lambda n: [t[:, :, :n] for t in (kbuf[0], vbuf[0], kbuf[1], vbuf[1], kbuf[2], vbuf[2])]  # noqa: E731
    plan = None
    if how != "mask":
        plan = kernels.DecodePlan(q, *views(n0 + 1), scale=D ** -0.5, bits=bits, group_size=gs, kv_start=ks,
                                  num_splits=splits, capacity=cap, append=(new[0], new[1]))
    for step in range(steps):
        n = n0 + step  # the appended key
        print(f"append {case} step {step}", flush=True)
        new[0].copy_(from_np(kw[:, :, n:n + 1], T, device))
        new[1].copy_(from_np(vw[:, :, n:n + 1], T, device))
        keep = np.ones((B, 1, 1, n + 1), bool)
        if starts is not None:
            keep = np.arange(n + 1)[None, None, None, :] >= np.array(starts)[:, None, None, None]
        mask_np = keep
        if how == "mask":
            drop = rng.random((B, 1, 1, n + 1)) < 0.2
            drop[..., -1] = False
            mask_np = keep & ~drop
            add = np.where(mask_np, 0.0, -np.inf).astype(np.float32)
            out = kernels.decode(q, *views(n + 1), scale=D ** -0.5, bits=bits, group_size=gs,
                                 mask=from_np(add, T, device), append=(new[0], new[1]))
        else:
            plan.set_keys(n + 1)
            out = plan()
        torch.cuda.synchronize()
        for name, got, want in (("K", kbuf, kq), ("V", vbuf, vq)):
            for i, part in enumerate(("codes", "scales", "biases")):
                g = to_np(got[i][:, :, :n + 1])
                assert _bits_equal(g, want[i][:, :, :n + 1], dt), f"step {step}: {name} {part} differ"
                rest = got[i][:, :, n + 1:]
                if rest.numel():
                    if rest.dtype == torch.uint32:
                        assert bool((rest.view(torch.int32) == GARBAGE).all()), f"{name} {part}: rows past N written"
                    else:
                        assert bool(rest.isnan().all()), f"{name} {part}: rows past N written"
        want = attention.quantized_sdpa_reference(
            to_np(q), kq[0][:, :, :n + 1], vq[0][:, :, :n + 1], kq[1][:, :, :n + 1], vq[1][:, :, :n + 1],
            kq[2][:, :, :n + 1], vq[2][:, :, :n + 1], bits=bits, group_size=gs, dtype=dt, mask=mask_np)
        got = to_np(out)
        err = np.abs(got - want)
        assert np.isfinite(got).all() and (err <= ATOL + RTOL * np.abs(want)).all(), \
            f"step {step}: max err {err.max():.3e}"
