"""The C-ABI boundary (CPU only: no kernel is launched here).

* every function include/qsdpa.h declares is exported by libqsdpa_hip.so;
* the ctypes structs of the Python binding have the header's layout
  (sizeof/offsetof printed by a gcc-compiled probe of the header);
* argument errors come back as negative codes with a message, before any
  HIP call.
"""

import ctypes
import re
import shutil
import subprocess

import pytest
import torch

from conftest import ROOT
from mlx_qsdpa_amd import _lib

HEADER = ROOT / "include" / "qsdpa.h"


def _declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(qsdpa_[a-z_]+)\s*\(", text)))


def test_header_functions_match_binding():
    assert _declared_functions() == sorted(_lib.EXPORTED_SYMBOLS)


def test_library_exports_every_symbol():
    lib = _lib.load()
    for name in _declared_functions():
        assert hasattr(lib, name), f"{name} not exported"
    assert lib.qsdpa_abi_version() == _lib.ABI_VERSION


_STRUCTS = {
    "qsdpa_view": _lib.View,
    "qsdpa_decode_args": _lib.DecodeArgs,
    "qsdpa_quantize_args": _lib.QuantizeArgs,
    "qsdpa_dequantize_args": _lib.DequantizeArgs,
    "qsdpa_requant_args": _lib.RequantArgs,
    "qsdpa_row_move": _lib.RowMove,
}


@pytest.mark.skipif(shutil.which("gcc") is None, reason="gcc not available")
def test_struct_layout_matches_header(tmp_path):
    lines = ['#include <stdio.h>', '#include <stddef.h>', f'#include "{HEADER}"', "int main(void){"]
    for cname, cls in _STRUCTS.items():
        lines.append(f'printf("{cname} size %zu\\n", sizeof({cname}));')
        for fname, _ in cls._fields_:
            lines.append(f'printf("{cname} {fname} %zu\\n", offsetof({cname}, {fname}));')
    lines.append("return 0;}")
    src = tmp_path / "probe.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "probe"
    subprocess.run(["gcc", "-std=c99", "-Wall", "-Werror", str(src), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout
    got = {}
    for line in out.splitlines():
        s, f, v = line.split()
        got[(s, f)] = int(v)
    for cname, cls in _STRUCTS.items():
        assert got[(cname, "size")] == ctypes.sizeof(cls), cname
        for fname, _ in cls._fields_:
            assert got[(cname, fname)] == getattr(cls, fname).offset, f"{cname}.{fname}"


def test_invalid_arguments_return_codes():
    lib = _lib.load()
    q = _lib.QuantizeArgs()
    q.bits = 3
    q.group_size = 32
    assert lib.qsdpa_quantize(ctypes.byref(q), None) == _lib.QSDPA_ERR_INVALID
    assert b"bits" in lib.qsdpa_last_error()
    jobs = (_lib.QuantizeArgs * 2)()
    for j in jobs:
        j.bits, j.group_size, j.D, j.B, j.H, j.S = 4, 32, 64, 1, 1, 1
    jobs[1].group_size = 64
    assert lib.qsdpa_quantize_batch(jobs, 2, None) == _lib.QSDPA_ERR_INVALID
    assert b"share" in lib.qsdpa_last_error()
    assert lib.qsdpa_quantize_batch(jobs, 5, None) == _lib.QSDPA_ERR_INVALID
    assert lib.qsdpa_quantize_batch(jobs, 0, None) == _lib.QSDPA_ERR_INVALID
    d = _lib.DequantizeArgs()
    d.bits, d.group_size, d.D = 4, 48, 96
    assert lib.qsdpa_dequantize(ctypes.byref(d), None) == _lib.QSDPA_ERR_UNSUPPORTED
    r = (_lib.RequantArgs * 2)()
    for x in r:
        x.B, x.H, x.D, x.bits, x.group_size, x.max_size, x.keep, x.n_old, x.S = 1, 1, 64, 4, 32, 8, 2, 2, 1
    r[0].rot = 1  # a rotation needs more old tokens than sinks
    assert lib.qsdpa_requant_window(r, 1, None) == _lib.QSDPA_ERR_INVALID
    assert b"bad window" in lib.qsdpa_last_error()
    r[0].rot, r[1].bits = 0, 8
    assert lib.qsdpa_requant_window(r, 2, None) == _lib.QSDPA_ERR_INVALID
    assert b"share" in lib.qsdpa_last_error()
    assert lib.qsdpa_requant_window(r, 3, None) == _lib.QSDPA_ERR_INVALID
    r[1].bits, r[1].H = 4, 2  # K and V of one cache: same batch and heads
    assert lib.qsdpa_requant_window(r, 2, None) == _lib.QSDPA_ERR_INVALID
    assert b"share B, H" in lib.qsdpa_last_error()
    if not torch.cuda.is_available():  # dummy pointers: never where a launch could reach a GPU
        r[1].H = 1
        for x in r:
            for i, v in enumerate((x.old_packed, x.old_scales, x.src, x.dst_packed, x.dst_scales, x.dst_biases)):
                v.ptr = (1 + i) << 20  # stand-in addresses, never dereferenced
                v.stride_n, v.stride_h, v.stride_b = 16, 64, 64
        r[1].old_packed.stride_n = 1 << 31  # two old rows 2^31 words apart: 32-bit offsets cannot reach
        assert lib.qsdpa_requant_window(r, 2, None) == _lib.QSDPA_ERR_UNSUPPORTED
        assert b"2^31" in lib.qsdpa_last_error()
    m = (_lib.RowMove * 2)()
    for x in m:
        x.dst, x.heads, x.tokens, x.row_bytes = 64, 2, 4, 16
    assert lib.qsdpa_move_rows(m, -1, None) == _lib.QSDPA_ERR_INVALID
    assert lib.qsdpa_move_rows(None, 1, None) == _lib.QSDPA_ERR_INVALID
    assert lib.qsdpa_move_rows(None, 0, None) == _lib.QSDPA_OK  # nothing to do: no launch
    m[1].src, m[1].copy_begin, m[1].copy_end = 128, 3, 5  # copy range past `tokens`
    assert lib.qsdpa_move_rows(m, 2, None) == _lib.QSDPA_ERR_INVALID
    assert b"copy range" in lib.qsdpa_last_error()
    m[1].copy_end, m[1].src_token_stride = 4, -16
    assert lib.qsdpa_move_rows(m, 2, None) == _lib.QSDPA_ERR_INVALID
    assert b"negative stride" in lib.qsdpa_last_error()
    m[1].src_token_stride, m[1].row_bytes = 16, 0
    assert lib.qsdpa_move_rows(m, 2, None) == _lib.QSDPA_ERR_INVALID
    m[1].row_bytes, m[1].dst = 16, None
    assert lib.qsdpa_move_rows(m, 2, None) == _lib.QSDPA_ERR_INVALID
    assert b"null dst" in lib.qsdpa_last_error()
    a = _lib.DecodeArgs()
    a.B = a.H_q = a.H_kv = a.N = 1
    a.D, a.bits, a.group_size = 100, 4, 32
    assert lib.qsdpa_decode(ctypes.byref(a), None) == _lib.QSDPA_ERR_INVALID
    assert b"multiple of 32" in lib.qsdpa_last_error()
    a.D = 128
    a.H_q, a.H_kv = 3, 2
    assert lib.qsdpa_decode_workspace_size(ctypes.byref(a), None) == _lib.QSDPA_ERR_INVALID
    assert b"divisible" in lib.qsdpa_last_error()
    a.H_q = 2
    assert lib.qsdpa_decode(ctypes.byref(a), None) == _lib.QSDPA_ERR_INVALID  # null pointers
    with pytest.raises(_lib.QsdpaError):
        _lib.check(lib.qsdpa_decode(ctypes.byref(a), None))


def test_prefill_routing_rule():
    """Calls with at least one full 128-row group per kv head (D = 128) run
    the prefill kernel: one pass where its groups fill the 256 CUs, key
    splits (a merge workspace) where they would not.  Smaller multi-query
    calls and D = 256 keep the split-K decode kernel.  (Planning only
    validates arguments; nothing is launched or read.)"""
    lib = _lib.load()

    def plan(B, Hq, Hkv, N, D, L, bits=8, gs=128):
        a = _lib.DecodeArgs()
        a.B, a.H_q, a.H_kv, a.N, a.D = B, Hq, Hkv, N, D
        a.bits, a.group_size, a.dtype, a.scale = bits, gs, _lib.QSDPA_BF16, 0.1
        a.q_len, a.causal = L, 1
        W, G = D * bits // 32, D // gs
        base = 1 << 20  # 16-byte aligned stand-in addresses (never dereferenced)
        a.q = _lib.View(base, Hq * L * D, L * D, D)
        a.out = _lib.View(base, Hq * L * D, L * D, D)
        a.k_packed = a.v_packed = _lib.View(base, Hkv * N * W, N * W, W)
        a.k_scales = a.v_scales = a.k_biases = a.v_biases = _lib.View(base, Hkv * N * G, N * G, G)
        n = ctypes.c_int32(0)
        ws = lib.qsdpa_decode_workspace_size(ctypes.byref(a), ctypes.byref(n))
        assert ws >= 0, lib.qsdpa_last_error()
        return n.value, ws

    assert plan(4, 16, 4, 4096, 128, 512) == (1, 0)       # the C5 chunk: prefill kernel, one pass
    splits, ws = plan(4, 16, 4, 4096, 128, 128)            # 64 groups: 4 key splits of 16 tiles
    assert splits == 4 and ws > 0
    assert plan(1, 64, 8, 256, 128, 16)[0] == 1             # 8 groups, 4 tiles: one split each
    splits, ws = plan(1, 16, 4, 4096, 128, 8)              # 32 rows per kv head: decode kernel
    assert splits > 1 and ws > 0
    splits, ws = plan(1, 16, 4, 4096, 256, 512)             # D = 256: decode kernel
    assert splits >= 1 and (splits == 1 or ws > 0)


@pytest.mark.skipif(shutil.which("g++") is None, reason="g++ not available")
def test_wave_split_covers_every_position_once(tmp_path):
    """The decode kernel's share of a split's tile positions among its 8
    waves (csrc/wave_split.h, compiled here for the host): for every J up
    to 1024 and both ratios, each position in [0, J) is visited by exactly
    one wave, waves 4-7 take no positions of the tail, and
    wave_split_last_owner names the wave that visits position J - 1."""
    header = HEADER.parent.parent / "mlx-qsdpa_amd" / "csrc" / "wave_split.h"
    src = tmp_path / "split.cc"
    src.write_text(f"""
#include <cstdio>
#include <vector>
#include "{header}"
int main() {{
  for (int D : {{128, 256}})
    for (int J = 0; J <= 1024; ++J) {{
      const int J8 = qsdpa::wave_split_rr_end(J, D);
      if (J8 < 0 || J8 > J) {{ std::printf("J8 %d of %d\\n", J8, J); return 1; }}
      std::vector<int> seen(J, 0);
      int last = -1;
      for (int w = 0; w < 8; ++w)
        for (int j = w; j < J; j = qsdpa::wave_split_next(j, J, J8, w)) {{
          seen[j]++;
          if (j == J - 1) last = w;
          if (w >= 4 && j >= J8) {{ std::printf("wave %d in the tail at %d (J=%d)\\n", w, j, J); return 1; }}
        }}
      if (J > 0 && last != qsdpa::wave_split_last_owner(J, D)) {{
        std::printf("D=%d J=%d last position visited by wave %d, owner %d\\n", D, J, last,
                    qsdpa::wave_split_last_owner(J, D));
        return 1;
      }}
      for (int j = 0; j < J; ++j)
        if (seen[j] != 1) {{ std::printf("D=%d J=%d position %d seen %d times\\n", D, J, j, seen[j]); return 1; }}
    }}
  std::printf("ok\\n");
  return 0;
}}
""")
    exe = tmp_path / "split"
    subprocess.run(["g++", "-std=c++17", "-O1", "-Wall", "-Werror", str(src), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True)
    assert out.returncode == 0 and out.stdout.strip() == "ok", out.stdout


def test_super_tiles_cover_every_tile_once(tmp_path):
    """The decode kernel's key-tile layout (csrc/wave_split.h, compiled here
    for the host): for every tile count T up to 600 and split count S up to
    160, uniform splits (super-tiles of up to 8 tiles, split s owning super-
    tiles s, s + S, ...) cover each tile of [0, T) exactly once, positions of
    a split visit increasing tiles, and every split keeps work whenever
    T >= S.  Stream-K segments (stride 1, at most jmax tiles from t_lo) take
    tiles t_lo, t_lo + 1, ... one by one."""
    header = HEADER.parent.parent / "mlx-qsdpa_amd" / "csrc" / "wave_split.h"
    src = tmp_path / "super.cc"
    src.write_text(f"""
#include <cstdio>
#include <vector>
#include "{header}"
int main() {{
  for (int T = 0; T <= 600; ++T)
    for (int S = 2; S <= 160; ++S) {{
      const int sh = qsdpa::super_tile_shift(T, S);
      std::vector<int> seen(T, 0);
      for (int s = 0; s < S; ++s) {{
        const int J = qsdpa::super_tile_positions(T, s, S, 0x7FFFFFFF, sh);
        if (T >= S && J == 0) {{ std::printf("T=%d S=%d split %d idle\\n", T, S, s); return 1; }}
        int prev = -1;
        for (int j = 0; j < J; ++j) {{
          const int t = qsdpa::super_tile_tile(j, s, S, sh);
          if (t < 0 || t >= T || t <= prev) {{ std::printf("T=%d S=%d split %d position %d tile %d\\n", T, S, s, j, t); return 1; }}
          prev = t;
          seen[t]++;
        }}
      }}
      for (int t = 0; t < T; ++t)
        if (seen[t] != 1) {{ std::printf("T=%d S=%d tile %d seen %d times\\n", T, S, t, seen[t]); return 1; }}
    }}
  for (int T = 0; T <= 200; ++T)
    for (int lo = 0; lo <= T; ++lo)
      for (int jmax = 1; jmax <= 40; ++jmax) {{
        const int sh = qsdpa::super_tile_shift(T, 1);
        const int J = qsdpa::super_tile_positions(T, lo, 1, jmax, sh);
        const int want = T - lo < jmax ? T - lo : jmax;
        if (sh != 0 || J != want) {{ std::printf("stream-K T=%d lo=%d jmax=%d: J %d\\n", T, lo, jmax, J); return 1; }}
        for (int j = 0; j < J; ++j)
          if (qsdpa::super_tile_tile(j, lo, 1, sh) != lo + j) {{ std::printf("stream-K tile\\n"); return 1; }}
      }}
  std::printf("ok\\n");
  return 0;
}}
""")
    exe = tmp_path / "super"
    subprocess.run(["g++", "-std=c++17", "-O1", "-Wall", "-Werror", str(src), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True)
    assert out.returncode == 0 and out.stdout.strip() == "ok", out.stdout
