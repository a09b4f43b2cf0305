"""Per-phase timeline of the matrix-core decode kernel on one GPU.

  python mlx-qsdpa_amd/timeline.py build               # here (hipcc): the probe library
  python mlx-qsdpa_amd/timeline.py run [--config c3]    # on the GPU
  python mlx-qsdpa_amd/timeline.py stream [--config c3] # on the GPU: a read-only launch of the same bytes
  python mlx-qsdpa_amd/timeline.py prefill [--qlen 512] # on the GPU: the prefill kernel's phases at C5
  python mlx-qsdpa_amd/timeline.py lds                  # on the GPU: LDS read rate of the prefill pattern
  python mlx-qsdpa_amd/timeline.py rates                # on the GPU: VALU issue interval per instruction

``build`` compiles the library with -DQSDPA_TIMELINE into
mlx_qsdpa_amd/libqsdpa_timeline.so: the same kernels, plus an s_memrealtime
stamp (100 MHz clock) per wave at fixed points, copied out by
qsdpa_debug_timeline().  ``run`` times the bench.py workload of a config
(synthetic K/V cycled over enough sets to stream from HBM) and prints, for
each point, the spread over the grid's waves in microseconds from the first
wave's entry, plus the median per wave slot (0-7) of the workgroup.

``prefill`` runs C5's causal chunk (bench.py's workload, the causal flag) on the
probe build's prefill kernel and prints, per wave slot, the mean shader-clock
cycles per tile of its three phases (start of tile to row maxima, row maxima to
end of tile, barrier); ``lds`` times the probe build's LDS read kernel (the
prefill kernel's K / V^T operand reads, one workgroup per CU); ``rates`` times
one instruction at a time (8 independent chains per lane, 8 waves per SIMD)
and prints its issue interval per SIMD, in ns and relative to v_fma_f32.

Points: entry; Q staged in LDS (after the workgroup barrier); k-th tile
done; stream end (the wave's last tile); partials merged in LDS (after the
barrier); stores issued; stores complete (after a full wait).  The last
line compares the kernel's start / stop events (bench.py's measure) with
the span of the stamps.
"""

from __future__ import annotations

import argparse
import ctypes
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent
LIB = HERE / "mlx_qsdpa_amd" / "libqsdpa_timeline.so"
WGS, WAVES, SLOTS = 2048, 8, 18
POINTS = [("entry", 0), ("Q staged", 1)] + [(f"tile {k} done", 2 + k) for k in range(12)] + [
    ("stream end", 14), ("LDS merge done", 15), ("stores issued", 16), ("stores complete", 17)]


def build() -> None:
    sys.path.insert(0, str(HERE))
    import build_lib

    build_lib.build(jobs=8, extra_flags=["-DQSDPA_TIMELINE"], out=LIB)
    print(f"built {LIB}")


def run(config: str, n: int | None, calls: int, lib_path: Path = LIB) -> None:
    for p in (ROOT, HERE):
        sys.path.insert(0, str(p))
    import numpy as np
    import torch

    import bench
    from mlx_qsdpa_amd import _lib, kernels, metric

    lib = _lib.load(lib_path)
    _lib._lib = lib  # the kernels module launches through this library
    lib.qsdpa_debug_timeline.argtypes = [ctypes.c_void_p, ctypes.c_size_t]
    lib.qsdpa_debug_timeline.restype = ctypes.c_int
    cfg = bench.CONFIGS[config]
    B, Hq, Hkv, D, bits, gs, dt, N0, _ = cfg
    N = n or N0
    set_bytes = B * N * metric.kv_bytes_per_token(Hkv, D, bits, gs)
    n_sets = max(2, int(1.2e9 // set_bytes) + 1)
    sets = bench.make_sets(cfg, N, n_sets, torch.device("cuda:0"), 0)
    plans = [kernels.DecodePlan(q, kq[0], vq[0], kq[1], vq[1], kq[2], vq[2], scale=D ** -0.5,
                                bits=bits, group_size=gs) for q, kq, vq in sets]
    nwg = plans[0].num_splits * Hkv * B * ((Hq // Hkv + 15) // 16)
    if nwg > WGS:
        raise SystemExit(f"{nwg} workgroups exceed the probe's {WGS}")
    buf = np.zeros(WGS * WAVES * SLOTS, dtype=np.uint64)
    hip = bench.HipEvents()
    ev = hip.create(2 * calls)
    for i in range(calls):
        plans[i % n_sets]((ev[2 * i], ev[2 * i + 1]))
    torch.cuda.synchronize()
    ev_us = [hip.elapsed_ms(ev[2 * i], ev[2 * i + 1]) * 1e3 for i in range(calls)]
    hip.destroy(ev)
    if lib.qsdpa_debug_timeline(buf.ctypes.data, buf.nbytes) != 0:
        raise SystemExit("qsdpa_debug_timeline failed")
    t = buf[: nwg * WAVES * SLOTS].reshape(nwg, WAVES, SLOTS).astype(np.int64)
    t0 = t[:, :, 0].min()
    rel = np.where(t > 0, (t - t0) * 0.01, np.nan)  # 10 ns ticks -> us
    print(f"# {config}: N={N}, {nwg} workgroups x {WAVES} waves, splits={plans[0].num_splits}, "
          f"last of {calls} calls; us from the first wave's entry")
    print("| point | p10 | p50 | p90 | max | median by wave 0-7 |")
    print("|---|---|---|---|---|---|")
    for name, k in POINTS:
        x = rel[:, :, k]
        if np.all(np.isnan(x)):
            continue
        by_wave = " ".join("-" if np.all(np.isnan(x[:, w])) else f"{np.nanmedian(x[:, w]):.2f}"
                           for w in range(WAVES))
        print(f"| {name} | {np.nanpercentile(x, 10):.2f} | {np.nanmedian(x):.2f} | "
              f"{np.nanpercentile(x, 90):.2f} | {np.nanmax(x):.2f} | {by_wave} |")
    span = (t[:, :, 17].max() - t0) * 0.01
    print(f"\nkernel start / stop events: {ev_us[-1]:.2f} us for this call (median of the {calls}: "
          f"{np.median(ev_us):.2f}); stamps span {span:.2f} us (first entry to last store complete)")


def stream(config: str, n: int | None, calls: int, lib_path: Path = LIB, blocks=(256, 512, 1024, 2048)) -> None:
    """Time a launch that only reads the decode's bytes (the probe library's
    stream_read kernel): the floor of one kernel moving that much from HBM,
    over the same number of distinct buffers as the decode's sets."""
    for p in (ROOT, HERE):
        sys.path.insert(0, str(p))
    import numpy as np
    import torch

    import bench
    from mlx_qsdpa_amd import _lib, metric

    lib = _lib.load(lib_path)
    lib.qsdpa_debug_stream_read.argtypes = [ctypes.c_void_p, ctypes.c_uint64, ctypes.c_void_p, ctypes.c_int,
                                            ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]
    lib.qsdpa_debug_stream_read.restype = ctypes.c_int
    cfg = bench.CONFIGS[config]
    B, Hq, Hkv, D, bits, gs, dt, N0, _ = cfg
    N = n or N0
    nbytes = metric.decode_bytes(B, Hq, Hkv, D, bits, gs, B * N) // 16 * 16
    n_sets = max(2, int(1.2e9 // nbytes) + 1)
    dev = torch.device("cuda:0")
    bufs = [torch.ones(nbytes, dtype=torch.uint8, device=dev) for _ in range(n_sets)]
    sink = torch.zeros(4096, dtype=torch.int32, device=dev)
    stream_h = torch.cuda.current_stream(dev).cuda_stream
    hip = bench.HipEvents()
    print(f"# {config}: {nbytes} bytes read per launch, {n_sets} buffers cycled")
    print("| workgroups | median us | p10 us | TB/s (median) | % of 8 TB/s |")
    print("|---|---|---|---|---|")
    for nb in blocks:
        ev = hip.create(2 * calls)
        for i in range(calls + 5):
            e = (ev[2 * (i - 5)], ev[2 * (i - 5) + 1]) if i >= 5 else (None, None)
            rc = lib.qsdpa_debug_stream_read(bufs[i % n_sets].data_ptr(), nbytes, sink.data_ptr(), nb, stream_h, *e)
            if rc != 0:
                raise SystemExit("qsdpa_debug_stream_read failed")
        torch.cuda.synchronize()
        us = np.array([hip.elapsed_ms(ev[2 * i], ev[2 * i + 1]) * 1e3 for i in range(calls)])
        hip.destroy(ev)
        med = float(np.median(us))
        print(f"| {nb} | {med:.2f} | {np.percentile(us, 10):.2f} | {nbytes / med / 1e6:.2f} | "
              f"{100 * nbytes / med / 1e6 / 8:.1f} |")


def stream_width(config: str, n: int | None, calls: int, lib_path: Path = LIB, blocks: int = 256) -> None:
    """Equal bytes in flight per thread, read with 16-, 8- or 4-byte loads
    (the probe library's stream_read_w kernel): does the read rate follow
    the bytes or the load instructions in flight?"""
    for p in (ROOT, HERE):
        sys.path.insert(0, str(p))
    import numpy as np
    import torch

    import bench
    from mlx_qsdpa_amd import _lib, metric

    lib = _lib.load(lib_path)
    f = lib.qsdpa_debug_stream_read_w
    f.argtypes = [ctypes.c_void_p, ctypes.c_uint64, ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                  ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]
    f.restype = ctypes.c_int
    cfg = bench.CONFIGS[config]
    B, Hq, Hkv, D, bits, gs, dt, N0, _ = cfg
    N = n or N0
    nbytes = metric.decode_bytes(B, Hq, Hkv, D, bits, gs, B * N) // 16 * 16
    n_sets = max(2, int(1.2e9 // nbytes) + 1)
    dev = torch.device("cuda:0")
    bufs = [torch.ones(nbytes, dtype=torch.uint8, device=dev) for _ in range(n_sets)]
    sink = torch.zeros(4096, dtype=torch.int32, device=dev)
    stream_h = torch.cuda.current_stream(dev).cuda_stream
    hip = bench.HipEvents()
    print(f"# {config}: {nbytes} bytes read per launch, {n_sets} buffers cycled, {blocks} workgroups x 512 threads")
    print("| load bytes | loads per thread in flight | KB in flight per workgroup | median us | TB/s |")
    print("|---|---|---|---|---|")
    for width, per in ((16, 4), (8, 8), (4, 16), (16, 8), (8, 16), (4, 32), (16, 16), (8, 32)):
        ev = hip.create(2 * calls)
        for i in range(calls + 5):
            e = (ev[2 * (i - 5)], ev[2 * (i - 5) + 1]) if i >= 5 else (None, None)
            if f(bufs[i % n_sets].data_ptr(), nbytes, sink.data_ptr(), blocks, width, per, stream_h, *e) != 0:
                raise SystemExit("qsdpa_debug_stream_read_w failed")
        torch.cuda.synchronize()
        us = np.array([hip.elapsed_ms(ev[2 * i], ev[2 * i + 1]) * 1e3 for i in range(calls)])
        hip.destroy(ev)
        med = float(np.median(us))
        print(f"| {width} | {per} | {512 * width * per // 1024} | {med:.2f} | {nbytes / med / 1e6:.2f} |", flush=True)


def prefill(qlen: int, calls: int, lib_path: Path = LIB) -> None:
    """Per-wave phase cycles of the prefill kernel at C5's causal chunk."""
    for p in (ROOT, HERE):
        sys.path.insert(0, str(p))
    import numpy as np
    import torch

    import bench
    from mlx_qsdpa_amd import _lib, kernels, metric

    lib = _lib.load(lib_path)
    _lib._lib = lib  # the kernels module launches through this library
    lib.qsdpa_debug_prefill_phases.argtypes = [ctypes.c_void_p, ctypes.c_size_t]
    lib.qsdpa_debug_prefill_phases.restype = ctypes.c_int
    cfg = bench.CONFIGS["c5"]
    B, Hq, Hkv, D, bits, gs, dt, N, _ = cfg
    dev = torch.device("cuda:0")
    n_sets = max(2, int(1.2e9 // (B * N * metric.kv_bytes_per_token(Hkv, D, bits, gs))) + 1)
    sets = bench.make_sets(cfg, N, n_sets, dev, 0)
    g = torch.Generator(device=dev)
    g.manual_seed(1)
    plans = [kernels.DecodePlan(torch.randn((B, Hq, qlen, D), generator=g, device=dev).bfloat16(), kq[0], vq[0],
                                kq[1], vq[1], kq[2], vq[2], scale=D ** -0.5, bits=bits, group_size=gs, causal=True)
             for _, kq, vq in sets]
    hip = bench.HipEvents()
    ev = hip.create(2 * calls)
    for i in range(calls):
        plans[i % n_sets]((ev[2 * i], ev[2 * i + 1]))
    torch.cuda.synchronize()
    ev_us = [hip.elapsed_ms(ev[2 * i], ev[2 * i + 1]) * 1e3 for i in range(calls)]
    hip.destroy(ev)
    groups = (Hq // Hkv * qlen + 127) // 128
    nwg = groups * Hkv * B * plans[0].num_splits
    buf = np.zeros(4096 * 8 * 4, dtype=np.uint64)
    if lib.qsdpa_debug_prefill_phases(buf.ctypes.data, buf.nbytes) != 0:
        raise SystemExit("qsdpa_debug_prefill_phases failed")
    t = buf[: nwg * 32].reshape(nwg, 8, 4).astype(np.float64)
    n = t[:, :, 3]
    ok = n > 1
    print(f"# c5 causal chunk qL={qlen}: {nwg} workgroups x 8 waves, last of {calls} calls; kernel "
          f"{ev_us[-1]:.1f} us (median {np.median(ev_us):.1f}); tiles per wave {n[ok].mean():.1f}")
    print("| wave | start -> row maxima | row maxima -> end | barrier | cycles per tile |")
    print("|---|---|---|---|---|")
    for w in range(8):
        m = ok[:, w]
        a = (t[m, w, 0] / n[m, w]).mean()
        c = (t[m, w, 1] / n[m, w]).mean()
        d = (t[m, w, 2] / (n[m, w] - 1)).mean()
        print(f"| {w} | {a:.0f} | {c:.0f} | {d:.0f} | {a + c + d:.0f} |")


def lds(calls: int, lib_path: Path = LIB, blocks: int = 256, iters: int = 2000) -> None:
    """LDS read rate of the prefill kernel's operand pattern."""
    for p in (ROOT, HERE):
        sys.path.insert(0, str(p))
    import numpy as np
    import torch

    import bench
    from mlx_qsdpa_amd import _lib

    lib = _lib.load(lib_path)
    f = lib.qsdpa_debug_lds_read
    f.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                  ctypes.c_void_p]
    f.restype = ctypes.c_int
    dev = torch.device("cuda:0")
    sink = torch.zeros(blocks, dtype=torch.int32, device=dev)
    cyc = torch.zeros(1, dtype=torch.int64, device=dev)
    stream_h = torch.cuda.current_stream(dev).cuda_stream
    hip = bench.HipEvents()
    ev = hip.create(2 * calls)
    for i in range(calls + 2):
        e = (ev[2 * (i - 2)], ev[2 * (i - 2) + 1]) if i >= 2 else (None, None)
        if f(blocks, iters, sink.data_ptr(), cyc.data_ptr(), stream_h, *e) != 0:
            raise SystemExit("qsdpa_debug_lds_read failed")
    torch.cuda.synchronize()
    us = float(np.median([hip.elapsed_ms(ev[2 * i], ev[2 * i + 1]) * 1e3 for i in range(calls)]))
    hip.destroy(ev)
    per_wg = iters * 8 * 32 * 1024  # bytes one workgroup reads: 8 waves x 32 KB per iteration
    cycles = int(cyc.item())
    print(f"# {blocks} workgroups x 512 threads, {iters} iterations of 32 KB per wave (16 K + 16 V^T reads of "
          f"16 B per lane)")
    print(f"median {us:.1f} us per launch: {per_wg / us / 1e3:.1f} GB/s per CU, {per_wg * blocks / us / 1e6:.1f} TB/s "
          f"chip; workgroup 0: {cycles} s_memtime cycles, {per_wg / cycles:.1f} B per cycle "
          f"({cycles / iters:.0f} cycles per 256 KB iteration)")


def rates(calls: int, lib_path: Path = LIB, blocks: int = 2048, iters: int = 2048) -> None:
    """Issue interval of the dequantization's and softmax's VALU instructions."""
    for p in (ROOT, HERE):
        sys.path.insert(0, str(p))
    import numpy as np
    import torch

    import bench
    from mlx_qsdpa_amd import _lib

    lib = _lib.load(lib_path)
    lib.qsdpa_debug_valu_rate_count.restype = ctypes.c_int
    lib.qsdpa_debug_valu_rate_name.argtypes = [ctypes.c_int]
    lib.qsdpa_debug_valu_rate_name.restype = ctypes.c_char_p
    f = lib.qsdpa_debug_valu_rate
    f.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                  ctypes.c_void_p]
    f.restype = ctypes.c_int
    dev = torch.device("cuda:0")
    sink = torch.zeros(blocks * 256, dtype=torch.int32, device=dev)
    stream_h = torch.cuda.current_stream(dev).cuda_stream
    simds = torch.cuda.get_device_properties(dev).multi_processor_count * 4
    per_simd = blocks * 4 * iters * 8 / simds  # wave instructions issued per SIMD
    hip = bench.HipEvents()
    ev = hip.create(2 * calls)
    print(f"# {blocks} workgroups x 4 waves, {iters} x 8 chained instructions per lane, {simds} SIMDs")
    print("| instruction | ns per wave instruction per SIMD | relative to v_fma_f32 |")
    print("|---|---|---|")
    base = None
    for w in range(lib.qsdpa_debug_valu_rate_count()):
        for i in range(calls + 1):
            e = (ev[2 * (i - 1)], ev[2 * (i - 1) + 1]) if i >= 1 else (None, None)
            if f(w, blocks, iters, sink.data_ptr(), stream_h, *e) != 0:
                raise SystemExit("qsdpa_debug_valu_rate failed")
        torch.cuda.synchronize()
        us = float(np.median([hip.elapsed_ms(ev[2 * i], ev[2 * i + 1]) * 1e3 for i in range(calls)]))
        ns = us * 1e3 / per_simd
        base = base or ns
        print(f"| {lib.qsdpa_debug_valu_rate_name(w).decode()} | {ns:.2f} | {ns / base:.2f} |")
    hip.destroy(ev)


def main(argv=None) -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("what", choices=["build", "run", "stream", "stream-width", "prefill", "lds", "rates"])
    ap.add_argument("--config", default="c3", choices=["c1", "c2", "c3", "c5"])
    ap.add_argument("--n", type=int, default=None)
    ap.add_argument("--calls", type=int, default=40)
    ap.add_argument("--qlen", type=int, default=512, help="prefill: query positions of the chunk")
    ap.add_argument("--lib", default=str(LIB), help="probe library to run (default: the one `build` makes)")
    a = ap.parse_args(argv)
    if a.what == "build":
        build()
    elif a.what == "stream":
        stream(a.config, a.n, a.calls, Path(a.lib))
    elif a.what == "stream-width":
        stream_width(a.config, a.n, a.calls, Path(a.lib))
    elif a.what == "prefill":
        prefill(a.qlen, a.calls, Path(a.lib))
    elif a.what == "lds":
        lds(a.calls, Path(a.lib))
    elif a.what == "rates":
        rates(min(a.calls, 5), Path(a.lib))
    else:
        run(a.config, a.n, a.calls, Path(a.lib))
    return 0


if __name__ == "__main__":
    sys.exit(main())
