#!/usr/bin/env python3
"""Decode benchmark: µs per decode step + effective HBM GB/s on one MI355X.

Default workload (BASELINE.json metric): GQA-16 decode, B=1, H_q=32, H_kv=2,
D=256, MLX-affine 4-bit gs=32, fp16, N=131072 keys.  Synthetic data: K/V and
q ~ N(0,1) (torch, seeded) quantized on the GPU by the library's own
quantize kernel; no checkpoint or dataset is involved.

A "step" is one fused decode (all its launches) over one KV set.  The timed
loop cycles over enough distinct KV sets (>= --kv-bytes, default 1.2 GB) that
the 256 MB Infinity Cache cannot hold them, so every step streams its K/V
from HBM.  Inputs are resident in HBM before timing starts.

Printed JSON line (rank 0, N=1):
  value            µs per decode step (wall time of K back-to-back steps / K,
                   with no profiling hooks in the timed region)
  roofline         achieved GB/s of the main decode kernel: algorithmic bytes
                   (q + packed K/V + scales + biases + out, the reference's
                   formula) / that kernel's mean duration over a second
                   pass of the same K steps, timed with HIP events that the
                   library attaches to the kernel's own dispatch
                   (hipExtLaunchKernel start / stop events);
                   traffic = HBM bytes per launch from the committed
                   rocprofv3 FETCH_SIZE / WRITE_SIZE summary
                   (profiles/traffic.txt) when it covers this workload;
                   kernel_us_p5_p50_p95 = percentiles of the per-step durations
  cpu_baseline     the oracle's float32 dequantize + attention (the
                   reference's CPU-capable path) on a bounded sample
"""

from __future__ import annotations

import argparse
import ctypes
import json
import math
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _p in (ROOT, ROOT / "mlx-qsdpa_amd"):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

METRIC = "µs/decode step + effective HBM GB/s (% peak), GQA-16 D=256 4-bit N=128K"
HBM_PEAK_GBPS = 8000.0
# Reference's published fused decode time for this exact config on an Apple
# M2 Ultra (README.md:89): 2431 µs at N=128K.
REFERENCE_US = {131072: 2431.0, 65536: 1438.0, 32768: 882.0, 16384: 588.0}

CONFIGS = {
    # name: (B, H_q, H_kv, D, bits, group_size, dtype, N, outlier_frac)
    "c1": (1, 8, 2, 128, 4, 64, "f16", 4096, 0.0),
    "c2": (1, 2, 2, 256, 8, 64, "bf16", 131072, 0.01),
    "c3": (1, 32, 2, 256, 4, 32, "f16", 131072, 0.0),
    "c5": (4, 16, 4, 128, 8, 128, "bf16", 4096, 0.0),
}


def parse_args(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=300)
    ap.add_argument("--warmup", type=int, default=None,
                    help="untimed steps before the timed ones (default: 2000 for the decode "
                         "configurations c1, c2, c3, c5, whose first tens of milliseconds run "
                         "below the steady clock: C3 measured 25.8-26.1 us per step after 30 "
                         "warmup steps, 23.2-23.5 after 1000 to 3000; 300 for c4, 68.3-69.4 "
                         "after 30 and 62.9-63.2 after 300; 30 for the other modes)")
    ap.add_argument("--config", default="c3", choices=sorted(CONFIGS) + ["c4"])
    ap.add_argument("--n", type=int, default=None, help="override the key count N")
    ap.add_argument("--kv-bytes", type=float, default=1.2e9,
                    help="distinct KV bytes cycled through (defeats the MALL)")
    ap.add_argument("--splits", type=int, default=0, help="0 = library heuristic")
    ap.add_argument("--qlen", type=int, default=1,
                    help="query positions per call; > 1 times causal multi-query attention "
                         "(fused vs dequantize + attention) instead of the decode step")
    ap.add_argument("--mask", default="none", choices=["none", "bool", "additive"],
                    help="with --qlen: pass the causal mask as a [B, 1, qL, N] tensor (bool, or additive "
                         "in the input type with random values on the kept keys) instead of the flag")
    ap.add_argument("--rotating-prefill", action="store_true",
                    help="time C5's prefill chunk (--qlen, default 512) through the batched rotating "
                         "cache: requant + attention")
    ap.add_argument("--crossover-sweep", action="store_true",
                    help="time one decode (qL = 1) through the fused kernel (library split count and "
                         "single pass) and through dequantize + attention (cache_sdpa's branch below "
                         "its crossover) over N, for the c1 / c3 / c5 shapes: one JSON line per point")
    ap.add_argument("--cpu-seconds", type=float, default=12.0,
                    help="time budget of the CPU baseline sample (0 = skip)")
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--calib-copy-mib", type=int, default=0,
                    help="before warmup, run one device-to-device copy of this many MiB (the "
                         "known-size reference for rocprofv3 FETCH_SIZE / WRITE_SIZE scaling)")
    return ap.parse_args(argv)


TRAFFIC_FILE = ROOT / "profiles" / "traffic.txt"


def measured_traffic(workload: str):
    """HBM bytes per launch of the main decode kernel for `workload`, from the
    committed rocprofv3 FETCH_SIZE / WRITE_SIZE summary (None if absent).

    Lines look like ``<workload> | fetch_bytes=<int> | write_bytes=<int>``.
    """
    if not TRAFFIC_FILE.exists():
        return None
    for line in TRAFFIC_FILE.read_text().splitlines():
        if line.startswith("#") or "|" not in line:
            continue
        parts = [x.strip() for x in line.split("|")]
        if parts[0] != workload:
            continue
        kv = dict(x.split("=", 1) for x in parts[1:] if "=" in x)
        return int(kv["fetch_bytes"]) + int(kv["write_bytes"])
    return None


class HipEvents:
    """hipEvent_t helpers through the HIP runtime torch already loaded."""

    def __init__(self):
        self.lib = ctypes.CDLL("libamdhip64.so.7")
        self.lib.hipEventCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
        self.lib.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p,
                                                 ctypes.c_void_p]
        self.lib.hipEventDestroy.argtypes = [ctypes.c_void_p]

    def create(self, n):
        evs = []
        for _ in range(n):
            e = ctypes.c_void_p()
            rc = self.lib.hipEventCreate(ctypes.byref(e))
            if rc != 0:
                raise RuntimeError(f"hipEventCreate failed ({rc})")
            evs.append(e.value)
        return evs

    def elapsed_ms(self, a, b):
        ms = ctypes.c_float()
        rc = self.lib.hipEventElapsedTime(ctypes.byref(ms), a, b)
        if rc != 0:
            raise RuntimeError(f"hipEventElapsedTime failed ({rc})")
        return ms.value

    def destroy(self, evs):
        for e in evs:
            self.lib.hipEventDestroy(e)


def make_sets(cfg, N, n_sets, device, seed):
    import torch

    from mlx_qsdpa_amd import kernels

    B, Hq, Hkv, D, bits, gs, dt, _, outl = cfg
    T = torch.float16 if dt == "f16" else torch.bfloat16
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    sets = []
    for _ in range(n_sets):
        kv = []
        for _ in range(2):
            w = torch.randn((B, Hkv, N, D), generator=g, device=device, dtype=torch.float32)
            if outl > 0:
                n_out = max(1, int(round(outl * D)))
                ch = torch.randperm(D, generator=g, device=device)[:n_out]
                w[..., ch] *= 8.0
            kv.append(kernels.quantize(w.to(T), gs, bits))
            del w
        q = torch.randn((B, Hq, 1, D), generator=g, device=device, dtype=torch.float32).to(T)
        sets.append((q, kv[0], kv[1]))
    torch.cuda.synchronize()
    return sets


def host_threads():
    """Host threads for the CPU baseline: the cores this process may run on
    (len(os.sched_getaffinity(0))), capped by OMP_NUM_THREADS when it is set
    lower (the GPU boxes give one GPU's job a 16-core share)."""
    cores = len(os.sched_getaffinity(0))
    cap = os.environ.get("OMP_NUM_THREADS", "")
    return (min(cores, int(cap)) if cap.isdigit() and int(cap) > 0 else cores), cores


def cpu_baseline(cfg, N, host_set, budget_s):
    """Oracle float32 decode on all host threads (key ranges split over
    threads, log-sum-exp merge) on the first KV set, repeated within budget."""
    import numpy as np

    from oracle import attention

    B, Hq, Hkv, D, bits, gs, dt, _, _ = cfg
    q, kq, vq = host_set
    threads, cores = host_threads()
    times = []
    t_end = time.perf_counter() + budget_s
    while True:
        t0 = time.perf_counter()
        attention.decode_fp32_threads(q, kq[0], vq[0], kq[1], vq[1], kq[2], vq[2], bits=bits,
                                      group_size=gs, threads=threads)
        times.append(time.perf_counter() - t0)
        if time.perf_counter() > t_end or len(times) >= 50:
            break
    us = float(np.median(times)) * 1e6
    return {"value": round(us, 1), "unit": "us/step", "cores": threads, "kind": "port",
            "sample": (f"{len(times)} full decode steps of the same workload (N={N}) on {threads} host "
                       f"threads (sched_getaffinity: {cores} cores; OMP_NUM_THREADS cap "
                       f"{os.environ.get('OMP_NUM_THREADS', 'unset')}), numpy float32 dequantize + "
                       f"attention over key ranges per thread with a log-sum-exp merge "
                       f"(oracle.attention.decode_fp32_threads), median")}


# continuous-batching decode through the batch cache's
# layout -- B sequences left-padded to the longest, each step appends one
# token per sequence (quantize-on-append into the shared column) and then
# decodes with kv_start = the left padding, so padded slots are never read.
C4 = {"B": 16, "H_q": 32, "H_kv": 8, "D": 128, "bits": 4, "group_size": 64, "dtype": "f16",
      "len_lo": 1024, "len_hi": 32768}


def _pcts(ms):
    """p5 / median / p95 of per-step kernel times (ms in, us out)."""
    import numpy as np
    return [round(float(x) * 1e3, 3) for x in np.percentile(np.asarray(ms), [5, 50, 95])]


def run_c4(args) -> int:
    import numpy as np
    import torch

    from mlx_qsdpa_amd import kernels, metric

    c = C4
    B, Hq, Hkv, D, bits, gs = c["B"], c["H_q"], c["H_kv"], c["D"], c["bits"], c["group_size"]
    device = torch.device("cuda:0")
    T = torch.float16
    gen = torch.Generator(device="cpu")
    gen.manual_seed(args.seed)
    lengths = torch.randint(c["len_lo"], c["len_hi"] + 1, (B,), generator=gen)
    lmax = int(lengths.max())
    # Every step appends a key to each sequence, warmup included: the
    # sequences start `warmup` keys shorter, so that the timed steps see the
    # drawn lengths.
    start = (lengths - args.warmup).clamp(min=1)
    total = args.warmup + 2 * args.steps
    cap = lmax + total
    W, G = D * bits // 32, D // gs
    bufs = []
    for _ in range(2):  # K, V
        bufs.append((torch.empty((B, Hkv, cap, W), dtype=torch.uint32, device=device),
                     torch.empty((B, Hkv, cap, G), dtype=T, device=device),
                     torch.empty((B, Hkv, cap, G), dtype=T, device=device)))
    g = torch.Generator(device=device)
    g.manual_seed(args.seed)
    chunk = 4096
    for t0 in range(0, lmax, chunk):  # synthetic prompt (the padded slots' content is never read)
        n = min(chunk, lmax - t0)
        for kv in bufs:
            w = torch.randn((B, Hkv, n, D), generator=g, device=device, dtype=torch.float32).to(T)
            kernels.quantize_into(w, kv, t0, bits, gs)
    q = torch.randn((B, Hq, 1, D), generator=g, device=device, dtype=torch.float32).to(T)
    new = [torch.randn((B, Hkv, 1, D), generator=g, device=device, dtype=torch.float32).to(T) for _ in range(2)]
    kv_start = (lmax - start).to(device=device, dtype=torch.int32)
    torch.cuda.synchronize()

    # Launch arguments built once: each step only moves the decode's key
    # count (the caches grow in place).  The one-token append of K and V
    # rides in the decode launch (append=): the workgroup that reads a
    # sequence's new key quantizes it into column n first.
    v0 = [t[:, :, :lmax + 1] for kv in bufs for t in kv]  # the split count is chosen for the first step
    plan = kernels.DecodePlan(q, v0[0], v0[3], v0[1], v0[4], v0[2], v0[5], scale=D ** -0.5, bits=bits,
                              group_size=gs, kv_start=kv_start, num_splits=args.splits, capacity=cap,
                              append=(new[0], new[1]))
    splits = plan.num_splits

    def step(n, ev=None):
        plan.set_keys(n + 1)  # key n is the appended one
        plan(ev)

    n = lmax
    for _ in range(args.warmup):
        step(n)
        n += 1
    torch.cuda.synchronize()
    n_first = n
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step(n)
        n += 1
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    hip = HipEvents()
    ev_b, ev_e = hip.create(args.steps), hip.create(args.steps)
    n2 = n
    for i in range(args.steps):
        step(n, (ev_b[i], ev_e[i]))
        n += 1
    torch.cuda.synchronize()
    kern_ms = [hip.elapsed_ms(ev_b[i], ev_e[i]) for i in range(args.steps)]
    kern_us = float(np.mean(kern_ms)) * 1e3
    hip.destroy(ev_b + ev_e)

    # The API path: the same batch shape through BatchQuantizedSDPACache --
    # update_and_fetch (quantize-on-append, growth by 256 slots when full)
    # then cache_sdpa with kv_start = the left padding, per step.
    import mlx_qsdpa_amd as mq

    cache = mq.BatchQuantizedSDPACache((lmax - start).tolist(), bits=bits, group_size=gs)
    for t0_ in range(0, lmax, chunk):
        n_ = min(chunk, lmax - t0_)
        kk = torch.randn((B, Hkv, n_, D), generator=g, device=device, dtype=torch.float32).to(T)
        vv = torch.randn((B, Hkv, n_, D), generator=g, device=device, dtype=torch.float32).to(T)
        cache.update_and_fetch(kk, vv)
        del kk, vv
    torch.cuda.synchronize()

    def api_step():
        kq, vq = cache.update_and_fetch(new[0], new[1])
        return mq.cache_sdpa(q, kq, vq, cache, kv_start=cache.kv_start(device))

    def cap_now():
        return cache._keys[0].shape[2]

    for _ in range(args.warmup):
        api_step()
    # The cache grows by 256 slots when full (a concatenation of every
    # buffer, as the reference's cache does).  Time the steady steps between
    # two growths, and one growing step on its own.
    cap0 = cap_now()
    for _ in range(cache.step + 1):
        if cap_now() != cap0:
            break
        api_step()
    torch.cuda.synchronize()
    api_steps = min(args.steps, cache.step - 2)
    cap1 = cap_now()
    t0 = time.perf_counter()
    for _ in range(api_steps):
        api_step()
    torch.cuda.synchronize()
    api_us = (time.perf_counter() - t0) / api_steps * 1e6
    grew = cap_now() != cap1
    growth_us = None
    for _ in range(cache.step + 1):  # on to the next growth, each step timed alone
        before = cap_now()
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        api_step()
        torch.cuda.synchronize()
        if cap_now() != before:
            growth_us = (time.perf_counter() - t1) * 1e6
            break
    del cache

    us_step = wall / args.steps * 1e6
    valid = lambda n_: int((start + (n_ + 1 - lmax)).sum())  # noqa: E731 (keys per sequence after the append)
    bytes_wall = np.mean([metric.decode_bytes(B, Hq, Hkv, D, bits, gs, valid(k))
                          for k in range(n_first, n_first + args.steps)])
    bytes_kern = np.mean([metric.decode_bytes(B, Hq, Hkv, D, bits, gs, valid(k))
                          for k in range(n2, n2 + args.steps)])
    step_gbps = bytes_wall / (us_step * 1e-6) / 1e9
    kern_gbps = bytes_kern / (kern_us * 1e-6) / 1e9
    print(f"bench: c4 {us_step:.2f} us/step wall (append + decode), decode kernel {kern_us:.2f} us "
          f"({kern_gbps:.0f} GB/s), splits={splits}; API path {api_us:.2f} us/step between cache growths, "
          f"a growing step {growth_us or 0:.0f} us", file=sys.stderr,
          flush=True)
    workload = (f"c4: batched decode B={B} H_q={Hq} H_kv={Hkv} D={D} {bits}-bit gs={gs} f16, lengths "
                f"U[{c['len_lo']},{c['len_hi']}] left-padded, append + decode per step (one launch)")
    line = {
        "metric": "µs/decode step (append + decode) + effective HBM GB/s (% peak), C4 batched",
        "value": round(us_step, 3), "unit": "us/step", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(us_step / 1e3, 6), "higher_is_better": False,
        "scaling": "weak", "vs_baseline": None, "dtype": "f16", "data": "synthetic",
        "config": {"workload": workload, "B": B, "H_q": Hq, "H_kv": Hkv, "D": D, "bits": bits,
                   "group_size": gs, "mean_valid_keys": round(bytes_wall / metric.kv_bytes_per_token(Hkv, D, bits, gs) / B, 1),
                   "num_splits": splits},
        "effective_gbps": round(step_gbps, 1),
        "pct_hbm_peak": round(100.0 * step_gbps / HBM_PEAK_GBPS, 2),
        "api_path": {"us_per_step": round(api_us, 3), "steps": api_steps, "cache_grew_in_timed_steps": grew,
                     "growth_step_us": None if growth_us is None else round(growth_us, 1),
                     "call": "BatchQuantizedSDPACache.update_and_fetch + cache_sdpa(kv_start=left padding)"},
        "roofline": {"bound": "hbm", "achieved": round(kern_gbps, 1), "peak": HBM_PEAK_GBPS,
                     "unit": "GB/s", "frac": round(kern_gbps / HBM_PEAK_GBPS, 4), "traffic": None,
                     "kernel_us": round(kern_us, 3), "kernel_us_p5_p50_p95": _pcts(kern_ms),
                     "algorithmic_bytes": int(bytes_kern)},
        "cpu_baseline": None,
    }
    print(json.dumps(line), flush=True)
    return 0


def run_multi_query(args) -> int:
    """--qlen L > 1: L causal query positions per (batch, head) over the
    config's cache (speculative or chunked decoding, prefill) on the fused
    kernel, with the reference's path for such calls -- HIP dequantize, then
    float32 attention with torch (mlx_qsdpa dispatch.py:68-83) -- timed on
    the same inputs in the same run."""
    import numpy as np
    import torch

    from mlx_qsdpa_amd import dispatch, kernels, metric

    cfg = CONFIGS[args.config]
    B, Hq, Hkv, D, bits, gs, dt, N0, _ = cfg
    N, L = args.n or N0, args.qlen
    device = torch.device("cuda:0")
    T = torch.float16 if dt == "f16" else torch.bfloat16
    kv_set_bytes = B * N * metric.kv_bytes_per_token(Hkv, D, bits, gs)
    n_sets = max(2, math.ceil(args.kv_bytes / kv_set_bytes))
    sets = make_sets(cfg, N, n_sets, device, args.seed)
    g = torch.Generator(device=device)
    g.manual_seed(args.seed + 1)
    qs = [torch.randn((B, Hq, L, D), generator=g, device=device, dtype=torch.float32).to(T)
          for _ in range(n_sets)]
    # The causal mask as a flag, or (--mask) as a tensor the kernels read per score.
    mask = None
    if args.mask != "none":
        keep = torch.arange(N, device=device)[None, :] <= (N - L) + torch.arange(L, device=device)[:, None]
        keep = keep[None, None].expand(B, 1, L, N)
        if args.mask == "bool":
            mask = keep.contiguous()
        else:
            noise = torch.randn((B, 1, L, N), generator=g, device=device, dtype=torch.float32)
            mask = torch.where(keep, noise, torch.full_like(noise, float("-inf"))).to(T)
    plans = [kernels.DecodePlan(qq, kq[0], vq[0], kq[1], vq[1], kq[2], vq[2], scale=D ** -0.5,
                                bits=bits, group_size=gs, num_splits=args.splits, mask=mask,
                                causal=mask is None)
             for qq, (_, kq, vq) in zip(qs, sets)]
    splits = plans[0].num_splits

    def fallback(i):
        _, kq, vq = sets[i]
        return dispatch.fallback_sdpa(qs[i], kq, vq, bits=bits, group_size=gs, scale=D ** -0.5,
                                      mask="causal" if mask is None else mask)

    got = plans[0]().float()
    want = fallback(0).float()
    max_diff = float((got - want).abs().max())
    for i in range(args.warmup):
        plans[i % n_sets]()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        plans[i % n_sets]()
    torch.cuda.synchronize()
    us = (time.perf_counter() - t0) / args.steps * 1e6
    hip = HipEvents()
    ev_b, ev_e = hip.create(args.steps), hip.create(args.steps)
    for i in range(args.steps):
        plans[i % n_sets]((ev_b[i], ev_e[i]))
    torch.cuda.synchronize()
    kern_ms = [hip.elapsed_ms(ev_b[i], ev_e[i]) for i in range(args.steps)]
    hip.destroy(ev_b + ev_e)
    kern_us = float(np.mean(kern_ms)) * 1e3
    fb_steps = max(5, min(args.steps, 50))
    for i in range(3):
        fallback(i % n_sets)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(fb_steps):
        fallback(i % n_sets)
    torch.cuda.synchronize()
    fb_us = (time.perf_counter() - t0) / fb_steps * 1e6

    # Causal keys per query row, summed: position i sees N - L + i + 1 keys.
    pairs = sum(max(0, min(N, N - L + i + 1)) for i in range(L))
    flops = 4.0 * B * Hq * pairs * D
    tflops = flops / (kern_us * 1e-6) / 1e12
    peak = 2500.0  # dense fp16 / bf16 MFMA
    mname = "causal" if mask is None else f"causal, {args.mask} mask tensor"
    print(f"bench: {args.config} qL={L} {mname}: fused {us:.2f} us/call wall, kernel {kern_us:.2f} us "
          f"({tflops:.1f} TFLOP/s); dequantize + attention {fb_us:.2f} us; max |diff| {max_diff:.2e}",
          file=sys.stderr, flush=True)
    workload = (f"{args.config}-q{L}: causal attention B={B} H_q={Hq} H_kv={Hkv} D={D} {bits}-bit "
                f"gs={gs} {dt} N={N} qL={L}" + ("" if mask is None else f" ({args.mask} mask tensor)"))
    line = {
        "metric": f"µs per attention call, {L} causal query positions (fused vs dequantize + attention)",
        "value": round(us, 3), "unit": "us/call", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(us / 1e3, 6), "higher_is_better": False,
        "scaling": "weak", "vs_baseline": None, "dtype": dt, "data": "synthetic",
        "config": {"workload": workload, "B": B, "H_q": Hq, "H_kv": Hkv, "D": D, "N": N, "qL": L,
                   "bits": bits, "group_size": gs, "num_splits": splits, "kv_sets": n_sets},
        "reference_path_us": round(fb_us, 3),
        "speedup_vs_reference_path": round(fb_us / us, 2),
        "max_abs_diff_vs_reference_path": max_diff,
        "roofline": {"bound": "mfma", "achieved": round(tflops, 2), "peak": peak, "unit": "TFLOP/s",
                     "frac": round(tflops / peak, 4), "traffic": None, "kernel_us": round(kern_us, 3),
                     "kernel_us_p5_p50_p95": _pcts(kern_ms), "flops": flops},
        "cpu_baseline": None,
    }
    print(json.dumps(line), flush=True)
    return 0


def run_rotating_prefill(args) -> int:
    """--rotating-prefill: C5's prefill chunk through the batched rotating
    cache.  The window (max_size = C5's N, keep = 4 sinks) is filled and
    advanced past its wrap; each step then takes one chunk of --qlen tokens
    (default 512): update_and_fetch (the requant launch: the old window in
    temporal order + the chunk, trimmed to the sinks and the newest tokens,
    quantized again into the spare buffers, K and V in one launch) and
    cache_sdpa with the causal mask (rows are unpadded, so "causal" is the
    mask make_mask would build).  Reports the wall time per chunk and, from
    torch events on the launch stream, the requant and the attention."""
    import numpy as np
    import torch

    import mlx_qsdpa_amd as mq
    from mlx_qsdpa_amd import metric

    B, Hq, Hkv, D, bits, gs, dt, W, _ = CONFIGS["c5"]
    L = args.qlen if args.qlen > 1 else 512
    keep = 4
    device = torch.device("cuda:0")
    T = torch.bfloat16
    g = torch.Generator(device=device)
    g.manual_seed(args.seed)

    def rnd(n, h=Hkv):
        return torch.randn((B, h, n, D), generator=g, device=device, dtype=torch.float32).to(T)

    cache = mq.BatchQuantizedRotatingSDPACache([0] * B, W, keep=keep, bits=bits, group_size=gs)
    for _ in range(W // 1024):
        cache.update_and_fetch(rnd(1024), rnd(1024))
    for _ in range(37):  # past the wrap: the ring is rotated
        cache.update_and_fetch(rnd(1), rnd(1))
    chunks = [(rnd(L), rnd(L), rnd(L, Hq)) for _ in range(4)]
    torch.cuda.synchronize()

    def step(i, ev=None):
        k, v, q = chunks[i % len(chunks)]
        if ev is not None:
            ev[0].record()
        kq, vq = cache.update_and_fetch(k, v)
        if ev is not None:
            ev[1].record()
        out = mq.cache_sdpa(q, kq, vq, cache, mask="causal")
        if ev is not None:
            ev[2].record()
        return out

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        step(i)
    torch.cuda.synchronize()
    us = (time.perf_counter() - t0) / args.steps * 1e6
    evs = [tuple(torch.cuda.Event(enable_timing=True) for _ in range(3)) for _ in range(args.steps)]
    for i in range(args.steps):
        step(i, evs[i])
    torch.cuda.synchronize()
    req_ms = [a.elapsed_time(b) for a, b, _ in evs]
    att_ms = [b.elapsed_time(c) for _, b, c in evs]
    req_us, att_us = float(np.mean(req_ms)) * 1e3, float(np.mean(att_ms)) * 1e3
    # Requant bytes: the old window read once (quantized), the chunk read
    # (raw T), the new window written (quantized); K and V.
    per_tok = metric.kv_bytes_per_token(Hkv, D, bits, gs)
    req_bytes = B * W * per_tok + 2 * B * Hkv * L * D * 2 + B * W * per_tok
    req_gbps = req_bytes / (req_us * 1e-6) / 1e9
    pairs = sum(max(0, min(W, W - L + i + 1)) for i in range(L))
    flops = 4.0 * B * Hq * pairs * D
    tflops = flops / (att_us * 1e-6) / 1e12
    print(f"bench: c5 rotating prefill chunk L={L}: {us:.2f} us/chunk wall; requant {req_us:.2f} us "
          f"({req_gbps:.0f} GB/s), attention {att_us:.2f} us ({tflops:.1f} TFLOP/s)", file=sys.stderr, flush=True)
    workload = (f"c5-rot-q{L}: rotating prefill chunk B={B} H_q={Hq} H_kv={Hkv} D={D} {bits}-bit gs={gs} "
                f"{dt} max_size={W} keep={keep}, wrapped window, requant + causal attention")
    line = {
        "metric": f"µs per rotating prefill chunk of {L} tokens (requant + attention), C5",
        "value": round(us, 3), "unit": "us/chunk", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(us / 1e3, 6), "higher_is_better": False,
        "scaling": "weak", "vs_baseline": None, "dtype": dt, "data": "synthetic",
        "config": {"workload": workload, "B": B, "H_q": Hq, "H_kv": Hkv, "D": D, "max_size": W,
                   "keep": keep, "qL": L, "bits": bits, "group_size": gs},
        "requant": {"us": round(req_us, 3), "us_p5_p50_p95": _pcts(req_ms), "bytes": req_bytes,
                    "achieved_gbps": round(req_gbps, 1), "frac_hbm": round(req_gbps / HBM_PEAK_GBPS, 4)},
        "roofline": {"bound": "mfma", "achieved": round(tflops, 2), "peak": 2500.0, "unit": "TFLOP/s",
                     "frac": round(tflops / 2500.0, 4), "traffic": None, "kernel_us": round(att_us, 3),
                     "kernel_us_p5_p50_p95": _pcts(att_ms), "flops": flops},
        "cpu_baseline": None,
    }
    print(json.dumps(line), flush=True)
    return 0


def run_crossover_sweep(args) -> int:
    """qL = 1 over N at the c1, c3 and c5 shapes: wall µs per call of
    quantized_sdpa (the fused kernel with the library's split count, and
    with num_splits=1: the reference's single pass, its choice for N <=
    threshold = 4096) and of fallback_sdpa (HIP dequantize + float32
    attention: cache_sdpa's branch for N < crossover).  Up to 32 KV sets are
    cycled (fewer bytes than the MALL holds at small N, as a decode loop over
    layers would see them); every point also reports the largest difference
    between the fused and the fallback outputs."""
    import torch

    import mlx_qsdpa_amd as mq
    from mlx_qsdpa_amd import metric

    device = torch.device("cuda:0")
    for name in ("c1", "c3", "c5"):
        cfg = CONFIGS[name]
        B, Hq, Hkv, D, bits, gs, dt, _, _ = cfg
        for N in (256, 1024, 4096, 16384, 65536):
            set_bytes = B * N * metric.kv_bytes_per_token(Hkv, D, bits, gs)
            n_sets = max(2, min(32, math.ceil(args.kv_bytes / set_bytes)))
            sets = make_sets(cfg, N, n_sets, device, args.seed)

            def call(i, how):
                q, kq, vq = sets[i % n_sets]
                if how == "fallback":
                    return mq.fallback_sdpa(q, kq, vq, bits=bits, group_size=gs, scale=D ** -0.5)
                return mq.quantized_sdpa(q, kq[0], vq[0], kq[1], vq[1], kq[2], vq[2], bits=bits, group_size=gs,
                                         num_splits=1 if how == "single_pass" else None)

            us = {}
            for how in ("fused", "single_pass", "fallback"):
                for i in range(args.warmup):
                    call(i, how)
                torch.cuda.synchronize()
                t0 = time.perf_counter()
                for i in range(args.steps):
                    call(i, how)
                torch.cuda.synchronize()
                us[how] = round((time.perf_counter() - t0) / args.steps * 1e6, 2)
            diff = float((call(0, "fused").float() - call(0, "fallback").float()).abs().max())
            print(json.dumps({"sweep": "crossover", "config": name, "N": N, "kv_sets": n_sets,
                              "us_per_call": us, "max_abs_diff_fused_vs_fallback": diff}), flush=True)
            del sets
            torch.cuda.empty_cache()
    return 0


def main(argv=None) -> int:
    args = parse_args(argv)
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); the decode path is "
              "single-GPU in this build (sharding by kv head and by sequence is a design only).",
              file=sys.stderr)
        return 2
    other_mode = args.crossover_sweep or args.rotating_prefill or args.config == "c4" or args.qlen > 1
    if args.warmup is None:
        # C4 (20 ms at 300 steps) starts its sequences that many keys
        # shorter, as it appends one per step.
        args.warmup = 300 if args.config == "c4" and not (args.crossover_sweep or args.rotating_prefill) \
            else 30 if other_mode else 2000
    if args.crossover_sweep:
        return run_crossover_sweep(args)
    if args.rotating_prefill:
        return run_rotating_prefill(args)
    if args.config == "c4":
        return run_c4(args)
    if args.qlen > 1:
        return run_multi_query(args)
    import numpy as np
    import torch

    from mlx_qsdpa_amd import kernels, metric

    cfg = CONFIGS[args.config]
    B, Hq, Hkv, D, bits, gs, dt, N0, _ = cfg
    N = args.n or N0
    device = torch.device("cuda:0")
    kv_set_bytes = B * N * metric.kv_bytes_per_token(Hkv, D, bits, gs)
    n_sets = max(2, math.ceil(args.kv_bytes / kv_set_bytes))
    print(f"bench: config={args.config} N={N} sets={n_sets} ({kv_set_bytes / 1e6:.1f} MB each)",
          file=sys.stderr, flush=True)
    sets = make_sets(cfg, N, n_sets, device, args.seed)
    # --mask: a [B, 1, 1, N] mask tensor the kernel reads per score (bool: 10% of the keys
    # dropped; additive: random values in the input type).
    mask = None
    if args.mask != "none":
        gm = torch.Generator(device=device)
        gm.manual_seed(args.seed + 2)
        r = torch.rand((B, 1, 1, N), generator=gm, device=device)
        T = torch.float16 if dt == "f16" else torch.bfloat16
        mask = (r >= 0.1) if args.mask == "bool" else torch.randn((B, 1, 1, N), generator=gm, device=device).to(T)
    plans = [kernels.DecodePlan(q, kq[0], vq[0], kq[1], vq[1], kq[2], vq[2], scale=D ** -0.5,
                                bits=bits, group_size=gs, num_splits=args.splits, mask=mask)
             for q, kq, vq in sets]
    splits = plans[0].num_splits

    if args.calib_copy_mib > 0:
        nbytes = args.calib_copy_mib << 20
        src = torch.ones(nbytes, dtype=torch.uint8, device=device)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        print(f"bench: calibration copy of {nbytes} bytes", file=sys.stderr, flush=True)
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    for i in range(args.warmup):
        plans[i % n_sets]()
    torch.cuda.synchronize()

    # Timed region (value): K decode steps back to back, no profiling hooks.
    t0 = time.perf_counter()
    for i in range(args.steps):
        plans[i % n_sets]()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0

    # Kernel duration (roofline): the same K steps again, each main decode
    # kernel carrying start / stop events on its own dispatch.
    hip = HipEvents()
    ev_b = hip.create(args.steps)
    ev_e = hip.create(args.steps)
    for i in range(args.steps):
        plans[i % n_sets]((ev_b[i], ev_e[i]))
    torch.cuda.synchronize()
    kern_ms = [hip.elapsed_ms(ev_b[i], ev_e[i]) for i in range(args.steps)]
    hip.destroy(ev_b + ev_e)

    # Whole step (decode kernel + split-K merge): torch events on the stream
    # both launches go to.
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(args.steps)]
    for i in range(args.steps):
        evs[i][0].record()
        plans[i % n_sets]()
        evs[i][1].record()
    torch.cuda.synchronize()
    step_ms = [a.elapsed_time(b) for a, b in evs]

    # The API path: mlx_qsdpa_amd.quantized_sdpa per step (argument blocks
    # cached per tensor geometry), same KV sets.
    import mlx_qsdpa_amd as mq

    def api(i):
        q, kq, vq = sets[i % n_sets]
        return mq.quantized_sdpa(q, kq[0], vq[0], kq[1], vq[1], kq[2], vq[2], scale=D ** -0.5,
                                 bits=bits, group_size=gs, mask=mask)

    for i in range(max(args.warmup, 2)):
        api(i)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        api(i)
    torch.cuda.synchronize()
    api_us = (time.perf_counter() - t0) / args.steps * 1e6

    us_step = wall / args.steps * 1e6
    kern_us = float(np.mean(kern_ms)) * 1e3
    alg_bytes = metric.decode_bytes(B, Hq, Hkv, D, bits, gs, B * N)
    step_gbps = alg_bytes / (us_step * 1e-6) / 1e9
    kern_gbps = alg_bytes / (kern_us * 1e-6) / 1e9
    step_us = float(np.mean(step_ms)) * 1e3
    print(f"bench: {us_step:.2f} us/step wall, main kernel {kern_us:.2f} us "
          f"({kern_gbps:.0f} GB/s), whole step {step_us:.2f} us (events), API path {api_us:.2f} us/step, "
          f"splits={splits}", file=sys.stderr, flush=True)

    cpu = None
    if args.cpu_seconds > 0 and mask is None:  # the CPU baseline times the unmasked workload
        host = tuple(x.cpu().numpy() if x.dtype == torch.uint32 else x.float().cpu().numpy()
                     for x in (sets[0][0],))
        kq = tuple(x.cpu().numpy() if x.dtype == torch.uint32 else x.float().cpu().numpy()
                   for x in sets[0][1])
        vq = tuple(x.cpu().numpy() if x.dtype == torch.uint32 else x.float().cpu().numpy()
                   for x in sets[0][2])
        cpu = cpu_baseline(cfg, N, (host[0], kq, vq), args.cpu_seconds)

    ref_us = REFERENCE_US.get(N) if args.config == "c3" and mask is None else None
    workload = f"{args.config}: decode B={B} H_q={Hq} H_kv={Hkv} D={D} {bits}-bit gs={gs} {dt} N={N}"
    if mask is not None:
        workload += f" ({args.mask} mask tensor)"
    traffic = measured_traffic(workload)
    line = {
        "metric": METRIC,
        "value": round(us_step, 3),
        "unit": "us/step",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(us_step / 1e3, 6),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": round(us_step / ref_us, 5) if ref_us else None,
        "vs_baseline_ref": (f"M2 Ultra fused decode {ref_us} us (mlx-qsdpa README.md:89)"
                            if ref_us else None),
        "dtype": dt,
        "data": "synthetic",
        "config": {
            "workload": workload,
            "B": B, "H_q": Hq, "H_kv": Hkv, "D": D, "N": N, "bits": bits, "group_size": gs,
            "kv_dtype": dt, "num_splits": splits, "kv_sets": n_sets,
        },
        "effective_gbps": round(step_gbps, 1),
        "pct_hbm_peak": round(100.0 * step_gbps / HBM_PEAK_GBPS, 2),
        "whole_step": {"us": round(step_us, 3), "us_p5_p50_p95": _pcts(step_ms),
                       "what": "decode kernel + split-K merge, torch events on the launch stream"},
        "api_path": {"us_per_step": round(api_us, 3),
                     "call": "mlx_qsdpa_amd.quantized_sdpa per step (argument block cached per geometry)"},
        "roofline": {
            "bound": "hbm",
            "achieved": round(kern_gbps, 1),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(kern_gbps / HBM_PEAK_GBPS, 4),
            "traffic": traffic,
            "kernel_us": round(kern_us, 3),
            "kernel_us_p5_p50_p95": _pcts(kern_ms),
            "algorithmic_bytes": alg_bytes,
        },
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
