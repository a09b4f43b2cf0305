"""Shared test setup.

* Registers the ``gpu`` marker (tests that need an MI355X).
* Puts the repo root (for ``oracle``) and ``mlx-qsdpa_amd`` (for the
  ``mlx_qsdpa_amd`` package) on sys.path.
* ``cpu_kernels``: replaces the library's kernel wrappers with oracle-backed
  CPU versions so the cache state machines (host logic) run on CPU tensors.
  The shipped package never does this; only these tests patch it.
"""

from __future__ import annotations

import os
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
for p in (ROOT, ROOT / "mlx-qsdpa_amd"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))

import torch  # noqa: E402

from oracle import affine  # noqa: E402

GOLDEN = ROOT / "tests" / "golden"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and the built HIP library")


def has_gpu() -> bool:
    return torch.cuda.is_available()


@pytest.fixture(scope="session")
def device():
    if not has_gpu():
        pytest.skip("no ROCm GPU in this environment")
    from mlx_qsdpa_amd import _lib
    _lib.load()  # fail loudly if the HIP library is missing
    return torch.device("cuda:0")


def dtype_name(dt: torch.dtype) -> str:
    return {torch.float16: "f16", torch.bfloat16: "bf16"}[dt]


def torch_dtype(name: str) -> torch.dtype:
    return {"f16": torch.float16, "bf16": torch.bfloat16}[name]


def to_np(t: torch.Tensor) -> np.ndarray:
    """Exact host copy: uint32 stays uint32, T -> float32 values."""
    t = t.detach().cpu()
    if t.dtype == torch.uint32:
        return t.numpy()
    return t.float().numpy()


def from_np(x: np.ndarray, dtype: torch.dtype, device=None) -> torch.Tensor:
    if x.dtype == np.uint32:
        t = torch.from_numpy(np.ascontiguousarray(x))
    else:
        t = torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(dtype)
    return t if device is None else t.to(device)


# ---------------------------------------------------------------------------
# oracle-backed CPU stand-ins for the kernel wrappers (tests only)
# ---------------------------------------------------------------------------
def _cpu_quantize_into(src, dst, t0, bits, group_size):
    name = dtype_name(src.dtype)
    p, s, b = affine.quantize(to_np(src), group_size, bits, name)
    S = src.shape[2]
    dst[0][:, :, t0:t0 + S] = torch.from_numpy(p)
    dst[1][:, :, t0:t0 + S] = from_np(s, src.dtype)
    dst[2][:, :, t0:t0 + S] = from_np(b, src.dtype)


def _cpu_dequantize(packed, scales, biases=None, group_size=64, bits=4, keep=0, rot=0):
    n = packed.shape[-2]
    if not 0 <= keep <= n or rot < 0 or (rot > 0 and keep >= n):  # as kernels.dequantize_into
        raise ValueError(f"bad keep={keep} / rot={rot} for N={n}")
    name = dtype_name(scales.dtype)
    out = affine.dequantize(to_np(packed), to_np(scales),
                            None if biases is None else to_np(biases), group_size, bits, name)
    n = out.shape[-2]
    if rot:
        idx = np.arange(n)
        u = np.where(idx < keep, idx, keep + (idx - keep + rot) % (n - keep))
        out = np.take(out, u, axis=-2)
    return from_np(out, scales.dtype)


def _cpu_requant_window(old, new, dst, n_old, keep, rot, max_size, bits, group_size):
    """kernels.requant_window as its steps, with the oracle: dequantize the
    old window in temporal order, append, keep the first `keep` and the
    newest max_size - keep, quantize into rows [0, total) of dst."""
    if not (0 <= keep < max_size and 0 <= n_old <= max_size and rot >= 0 and (rot == 0 or n_old > keep)):
        raise ValueError(f"bad window: max_size={max_size} keep={keep} n_old={n_old} rot={rot}")
    total = None
    for o, x, d in zip(old, new, dst):
        if n_old and d[0].data_ptr() == o[0].data_ptr():
            raise ValueError("the destination must not be the old window")
        allv = x
        if n_old:
            win = _cpu_dequantize(o[0][:, :, :n_old], o[1][:, :, :n_old], o[2][:, :, :n_old],
                                  group_size=group_size, bits=bits, keep=keep if rot else 0, rot=rot)
            allv = torch.cat([win, x], dim=2)
        n = allv.shape[2]
        if n > max_size:
            allv = torch.cat([allv[:, :, :keep], allv[:, :, n - (max_size - keep):]], dim=2)
        total = allv.shape[2]
        _cpu_quantize_into(allv, d, 0, bits, group_size)
    return total


def _cpu_quantize_kv_into(keys, values, kdst, vdst, t0, bits, group_size):
    _cpu_quantize_into(keys, kdst, t0, bits, group_size)
    _cpu_quantize_into(values, vdst, t0, bits, group_size)


def _cpu_move_rows(moves):
    """CPU stand-in for kernels.move_rows (qsdpa_move_rows): the same
    RowMove semantics with torch slicing, plus the wrapper's bounds checks."""
    for m in moves:
        if m.tokens <= 0:
            continue
        d = m.dst
        if not (0 <= m.dst_row < d.shape[0] and 0 <= m.dst_col and m.dst_col + m.tokens <= d.shape[2]):
            raise ValueError("dst rows out of range")
        seg = d[m.dst_row, :, m.dst_col:m.dst_col + m.tokens]
        seg.zero_()
        if m.src is not None and m.copy_end > m.copy_begin:
            n = m.copy_end - m.copy_begin
            s = m.src
            if not (0 <= m.src_row < s.shape[0] and 0 <= m.src_col and m.src_col + n <= s.shape[2]):
                raise ValueError("src rows out of range")
            if s.dtype != d.dtype or s.shape[1] != d.shape[1] or s.shape[3] != d.shape[3]:
                raise ValueError("src does not match dst")
            seg[:, m.copy_begin:m.copy_end] = s[m.src_row, :, m.src_col:m.src_col + n]


@pytest.fixture
def cpu_kernels(monkeypatch):
    from mlx_qsdpa_amd import kernels
    monkeypatch.setattr(kernels, "quantize_into", _cpu_quantize_into)
    monkeypatch.setattr(kernels, "quantize_kv_into", _cpu_quantize_kv_into)
    monkeypatch.setattr(kernels, "dequantize", _cpu_dequantize)
    monkeypatch.setattr(kernels, "requant_window", _cpu_requant_window)
    monkeypatch.setattr(kernels, "move_rows", _cpu_move_rows)
    return kernels


def rand_T(rng, shape, name, **kw):
    return affine.random_T(rng, shape, name, **kw)


@pytest.fixture
def rng():
    return np.random.default_rng(42)


os.environ.setdefault("PYTHONHASHSEED", "0")
