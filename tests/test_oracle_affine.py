"""Pins the oracle's affine quantizer / dequantizer (CPU)."""

import json

import numpy as np
import pytest

from conftest import GOLDEN
from oracle import affine

KAT = json.loads((GOLDEN / "affine_known_answers.json").read_text())


def _val(bits_hex, dtype):
    u = np.array([int(bits_hex, 16)], np.uint16)
    if dtype == "f16":
        return u.view(np.float16).astype(np.float32)
    return affine.bf16_bits_to_f32(u)


@pytest.mark.parametrize("case", KAT["quantize"], ids=lambda c: c["name"])
def test_quantize_known_answers(case):
    w = np.array(case["w"], np.float32)[None]
    assert np.array_equal(affine.to_T(w, case["dtype"]), w), "KAT input not exact in dtype"
    p, s, b = affine.quantize(w, case["group_size"], case["bits"], case["dtype"])
    assert affine.unpack(p, case["bits"])[0].tolist() == case["codes"]
    if "words" in case:
        assert p[0].tolist() == [int(x, 16) for x in case["words"]]
    sb = affine.T_bits(s, case["dtype"])[0, 0]
    bb = affine.T_bits(b, case["dtype"])[0, 0]
    assert bb == int(case["bias_bits"], 16)
    if "scale_bits" in case:
        assert sb == int(case["scale_bits"], 16)
    if "scale_range" in case:
        lo, hi = case["scale_range"]
        assert lo <= float(s[0, 0]) <= hi


@pytest.mark.parametrize("case", KAT["dequantize"], ids=lambda c: c["name"])
def test_dequantize_known_answers(case):
    q = np.zeros((1, case["group_size"]), np.uint32)
    q[0, 0] = case["code"]
    p = affine.pack(q, case["bits"])
    s = _val(case["scale_bits"], case["dtype"])[None]
    b = _val(case["bias_bits"], case["dtype"])[None]
    v = affine.dequantize(p, s, b, case["group_size"], case["bits"], case["dtype"])
    assert affine.T_bits(v[:, :1], case["dtype"])[0, 0] == int(case["value_bits"], 16)


@pytest.mark.parametrize("bits", [4, 8])
def test_pack_unpack_roundtrip(bits, rng):
    q = rng.integers(0, 1 << bits, size=(3, 5, 64), dtype=np.uint32)
    assert np.array_equal(affine.unpack(affine.pack(q, bits), bits), q)


def test_pack_order_matches_reference_shift_rule(rng):
    """Element d of a word is (word >> (d % per) * bits) & mask (kernels.py:103-105)."""
    q = rng.integers(0, 16, size=(64,), dtype=np.uint32)
    p = affine.pack(q[None], 4)[0]
    for d in range(64):
        assert (int(p[d // 8]) >> ((d % 8) * 4)) & 0xF == q[d]


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
@pytest.mark.parametrize("bits,gs", [(4, 32), (4, 64), (4, 128), (8, 32), (8, 64), (8, 128)])
def test_error_bound(dtype, bits, gs, rng):
    """MLX's own test bound: |w - dequant(quant(w))| <= |scale| (plus T rounding).

    Not |scale|/2: the snapped scale can push the far extreme past the last
    code, where it is clipped."""
    w = affine.random_T(rng, (16, 256), dtype)
    p, s, b = affine.quantize(w, gs, bits, dtype)
    w_hat = affine.dequantize(p, s, b, gs, bits, dtype)
    err = np.abs(w - w_hat).reshape(16, 256 // gs, gs)
    tol = np.abs(s)[..., None] + np.abs(w).reshape(err.shape) * (2 ** -7) + 1e-6
    assert np.all(err <= tol)


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_zero_is_on_the_grid(dtype, rng):
    """The snapped scale puts 0.0 on the grid (before T rounding of the scale)."""
    w = affine.random_T(rng, (64, 64), dtype)
    wg = w.reshape(64, 2, 32)
    scale, bias = affine.group_params(wg, 4)
    k = -bias / scale
    nz = bias != 0
    assert np.allclose(k[nz], np.rint(k[nz]), atol=1e-4)


def test_codes_in_range_and_extremes_hit(rng):
    w = affine.random_T(rng, (32, 128), "f16")
    p, s, b = affine.quantize(w, 32, 4, "f16")
    q = affine.unpack(p, 4).reshape(32, 4, 32)
    assert q.max() <= 15
    # The edge element maps to code 0, the far extreme to code 15 (+/-1 from snapping).
    assert np.all(q.min(axis=-1) == 0)
    assert np.all(q.max(axis=-1) >= 14)


def test_bf16_rounding_ties_to_even():
    x = np.array([1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, -(1.0 + 2 ** -8)], np.float32)
    # 1 + 2^-8 is halfway between bf16 1.0 and 1.0078125 -> even (1.0);
    # 1 + 3*2^-8 is halfway between 1.0078125 and 1.015625 -> even (1.015625).
    assert affine.to_T(x, "bf16").tolist() == [1.0, 1.015625, -1.0]


def test_bf16_nan_stays_nan():
    x = np.array([np.nan], np.float32)
    assert np.isnan(affine.to_T(x, "bf16")[0])
