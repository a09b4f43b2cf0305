"""Pins the oracle's float64 attention and mask helper (CPU)."""

import json
import math

import numpy as np
import pytest

from conftest import GOLDEN
from oracle import affine, attention
from oracle import caches as oc

REF = json.loads((GOLDEN / "reference_fixtures.json").read_text())


def _brute(q, k, v, scale, keep=None):
    """Pure-Python loops, one (b, h) at a time (tiny inputs only)."""
    B, Hq, L, D = q.shape
    Hkv, N = k.shape[1], k.shape[2]
    G = Hq // Hkv
    out = np.zeros((B, Hq, L, D))
    for b in range(B):
        for h in range(Hq):
            for i in range(L):
                sc = []
                for j in range(N):
                    if keep is not None and not keep[b, h, i, j]:
                        sc.append(None)
                        continue
                    sc.append(sum(float(q[b, h, i, d]) * float(k[b, h // G, j, d])
                                  for d in range(D)) * scale)
                vals = [s for s in sc if s is not None]
                if not vals:
                    continue
                mx = max(vals)
                w = [0.0 if s is None else math.exp(s - mx) for s in sc]
                tot = sum(w)
                for d in range(D):
                    out[b, h, i, d] = sum(w[j] * float(v[b, h // G, j, d]) for j in range(N)) / tot
    return out


def test_sdpa_matches_brute_force(rng):
    q = rng.standard_normal((2, 4, 3, 8))
    k = rng.standard_normal((2, 2, 5, 8))
    v = rng.standard_normal((2, 2, 5, 8))
    keep = rng.random((2, 4, 3, 5)) > 0.3
    keep[..., 0] = True
    np.testing.assert_allclose(attention.sdpa(q, k, v, 0.3), _brute(q, k, v, 0.3), atol=1e-12)
    np.testing.assert_allclose(attention.sdpa(q, k, v, 0.3, mask=keep),
                               _brute(q, k, v, 0.3, keep), atol=1e-12)


def test_single_key_returns_value_row(rng):
    q = rng.standard_normal((1, 4, 1, 16))
    k = rng.standard_normal((1, 2, 1, 16))
    v = rng.standard_normal((1, 2, 1, 16))
    o = attention.sdpa(q, k, v, 0.25)
    np.testing.assert_allclose(o[0, :2, 0], np.repeat(v[0, :1, 0], 2, 0), atol=1e-14)
    np.testing.assert_allclose(o[0, 2:, 0], np.repeat(v[0, 1:, 0], 2, 0), atol=1e-14)


def test_identical_keys_give_mean_value(rng):
    q = rng.standard_normal((1, 2, 1, 16))
    k = np.repeat(rng.standard_normal((1, 1, 1, 16)), 7, axis=2)
    v = rng.standard_normal((1, 1, 7, 16))
    o = attention.sdpa(q, k, v, 1.0)
    np.testing.assert_allclose(o[0, 0, 0], v[0, 0].mean(0), atol=1e-14)


def test_value_shift_is_additive(rng):
    """Adding c to every value adds exactly c to every output (softmax rows sum to 1)."""
    q = rng.standard_normal((1, 4, 1, 32))
    k = rng.standard_normal((1, 2, 50, 32))
    v = rng.standard_normal((1, 2, 50, 32))
    np.testing.assert_allclose(attention.sdpa(q, k, v + 0.75, 0.2) - attention.sdpa(q, k, v, 0.2),
                               0.75, atol=1e-12)


def test_reference_path_is_dequantize_then_sdpa(rng):
    B, H, N, D, gs = 1, 2, 40, 64, 32
    q = affine.random_T(rng, (B, H, 1, D), "f16")
    kp, ks, kb = affine.quantize(affine.random_T(rng, (B, H, N, D), "f16"), gs, 4, "f16")
    vp, vs, vb = affine.quantize(affine.random_T(rng, (B, H, N, D), "f16"), gs, 4, "f16")
    o = attention.quantized_sdpa_reference(q, kp, vp, ks, vs, kb, vb, bits=4, group_size=gs,
                                           dtype="f16")
    k = affine.dequantize(kp, ks, kb, gs, 4, "f16")
    v = affine.dequantize(vp, vs, vb, gs, 4, "f16")
    np.testing.assert_array_equal(o, attention.sdpa(q, k, v, D ** -0.5))
    # symmetric format: None biases are zero biases (dispatch.py:71, 76)
    o0 = attention.quantized_sdpa_reference(q, kp, vp, ks, vs, None, None, bits=4,
                                            group_size=gs, dtype="f16")
    z = np.zeros_like(ks)
    o1 = attention.quantized_sdpa_reference(q, kp, vp, ks, vs, z, z, bits=4, group_size=gs,
                                            dtype="f16")
    np.testing.assert_array_equal(o0, o1)


def test_permutation_invariance(rng):
    q = rng.standard_normal((1, 2, 1, 16))
    k = rng.standard_normal((1, 1, 9, 16))
    v = rng.standard_normal((1, 1, 9, 16))
    perm = rng.permutation(9)
    np.testing.assert_allclose(attention.sdpa(q, k, v, 0.5),
                               attention.sdpa(q, k[:, :, perm], v[:, :, perm], 0.5), atol=1e-13)


def test_fully_masked_row_is_zero(rng):
    q = rng.standard_normal((1, 1, 1, 8))
    k = rng.standard_normal((1, 1, 4, 8))
    v = rng.standard_normal((1, 1, 4, 8))
    keep = np.zeros((1, 1, 1, 4), bool)
    assert np.all(attention.sdpa(q, k, v, 1.0, mask=keep) == 0)


def test_causal_string_is_lower_right_aligned(rng):
    q = rng.standard_normal((1, 1, 3, 8))
    k = rng.standard_normal((1, 1, 5, 8))
    v = rng.standard_normal((1, 1, 5, 8))
    keep = np.array([[j <= i + 2 for j in range(5)] for i in range(3)])[None, None]
    np.testing.assert_allclose(attention.sdpa(q, k, v, 0.7, mask="causal"),
                               attention.sdpa(q, k, v, 0.7, mask=keep), atol=0)


def test_additive_mask_equals_bool_mask(rng):
    q = rng.standard_normal((1, 2, 1, 8))
    k = rng.standard_normal((1, 2, 6, 8))
    v = rng.standard_normal((1, 2, 6, 8))
    keep = rng.random((1, 2, 1, 6)) > 0.4
    keep[..., 2] = True
    add = np.where(keep, 0.0, -np.inf)
    np.testing.assert_allclose(attention.sdpa(q, k, v, 1.0, mask=keep),
                               attention.sdpa(q, k, v, 1.0, mask=add), atol=0)


@pytest.mark.parametrize("key", ["batch_mask_left_padding"])
def test_batch_mask_golden(key):
    g = REF[key]
    lengths = g["lengths"]
    lp = np.array([max(lengths) - l for l in lengths])
    offset = np.array(lengths)  # offset = -lp + max_len after merge
    mask = attention.create_causal_mask(g["N"], offset, left_padding=lp)
    assert list(mask.shape) == g["shape"]
    assert np.array_equal(mask, np.array(g["expected"]))


def test_batch_mask_golden_through_oracle_caches(rng):
    """Same golden array, produced through the oracle cache classes."""
    g = REF["batch_mask_left_padding"]
    cs = []
    for n in g["lengths"]:
        c = oc.QuantizedSDPACache(bits=4, group_size=32)
        c.update_and_fetch(affine.random_T(rng, (1, 2, n, 256), "f16"),
                           affine.random_T(rng, (1, 2, n, 256), "f16"))
        cs.append(c)
    batch = oc.BatchQuantizedSDPACache.merge(cs)
    assert np.array_equal(batch.make_mask(g["N"]), np.array(g["expected"]))
    g2 = REF["batch_rotating_mask_left_padding"]
    rs = []
    for n in g2["lengths"]:
        c = oc.QuantizedRotatingSDPACache(max_size=g2["max_size"], bits=4, group_size=32)
        for _ in range(n):
            c.update_and_fetch(affine.random_T(rng, (1, 2, 1, 64), "f16"),
                               affine.random_T(rng, (1, 2, 1, 64), "f16"))
        rs.append(c)
    rb = oc.BatchQuantizedRotatingSDPACache.merge(rs)
    assert np.array_equal(rb.make_mask(g2["N"]), np.array(g2["expected"]))


def test_decode_fp32_close_to_reference(rng):
    B, Hq, Hkv, N, D, gs = 1, 4, 2, 64, 128, 32
    q = affine.random_T(rng, (B, Hq, 1, D), "f16")
    kp, ks, kb = affine.quantize(affine.random_T(rng, (B, Hkv, N, D), "f16"), gs, 4, "f16")
    vp, vs, vb = affine.quantize(affine.random_T(rng, (B, Hkv, N, D), "f16"), gs, 4, "f16")
    ref = attention.quantized_sdpa_reference(q, kp, vp, ks, vs, kb, vb, bits=4, group_size=gs,
                                             dtype="f16")
    f32 = attention.decode_fp32(q, kp, vp, ks, vs, kb, vb, bits=4, group_size=gs)
    np.testing.assert_allclose(f32, ref, atol=2e-3)


@pytest.mark.parametrize("threads", [1, 3, 8])
def test_decode_fp32_threads_equals_single_thread(rng, threads):
    """The key-range split + log-sum-exp merge of the multi-core CPU
    baseline gives the single-pass float32 result (to float32 rounding),
    including a range whose keys all score far below another's."""
    B, Hq, Hkv, N, D, gs = 2, 8, 2, 301, 64, 32
    q = affine.random_T(rng, (B, Hq, 1, D), "f16")
    k = affine.random_T(rng, (B, Hkv, N, D), "f16")
    k[:, :, 200:] *= 6.0  # the last range dominates the softmax
    v = affine.random_T(rng, (B, Hkv, N, D), "f16")
    kp, ks, kb = affine.quantize(k, gs, 4, "f16")
    vp, vs, vb = affine.quantize(v, gs, 4, "f16")
    one = attention.decode_fp32(q, kp, vp, ks, vs, kb, vb, bits=4, group_size=gs)
    par = attention.decode_fp32_threads(q, kp, vp, ks, vs, kb, vb, bits=4, group_size=gs, threads=threads)
    np.testing.assert_allclose(par, one, rtol=2e-5, atol=2e-6)
