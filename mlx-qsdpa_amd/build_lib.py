"""Build libqsdpa_hip.so (gfx950) in-tree with hipcc.

Usage:  python mlx-qsdpa_amd/build_lib.py [--jobs N]

Compiles every csrc/*.hip translation unit for gfx950 and links one shared
library, mlx_qsdpa_amd/libqsdpa_hip.so, that exports the C ABI declared in
include/qsdpa.h.  The library depends only on the HIP runtime.
"""

from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
PKG = HERE / "mlx_qsdpa_amd"
LIB = PKG / "libqsdpa_hip.so"
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    # Packed fp32 instructions are kept out of every kernel on this target.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-fno-gpu-rdc",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found")


def build(jobs: int = 4, verbose: bool = False, extra_flags=(), out: Path | None = None) -> Path:
    """Compile csrc/*.hip and link the library (to `out`, default in-tree)."""
    cc = hipcc()
    srcs = sorted(CSRC.glob("*.hip"))
    lib = Path(out) if out is not None else LIB
    objdir = HERE / "_build" / (lib.stem if out is not None else "default")
    objdir.mkdir(parents=True, exist_ok=True)

    def compile_one(src: Path) -> Path:
        obj = objdir / (src.stem + ".o")
        cmd = [cc, *HIPCC_FLAGS, *extra_flags, "-c", str(src), "-o", str(obj)]
        if verbose:
            print(" ".join(cmd), flush=True)
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"hipcc failed for {src.name}:\n{r.stdout}\n{r.stderr}")
        return obj

    with cf.ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        objs = list(ex.map(compile_one, srcs))
    tmp = lib.with_suffix(".so.tmp")
    cmd = [cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, lib)
    return lib


def main(argv=None) -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=4)
    ap.add_argument("-v", "--verbose", action="store_true")
    ap.add_argument("--out", default=None, help="output library path (default: in-tree)")
    ap.add_argument("-D", dest="defines", action="append", default=[],
                    help="extra preprocessor define for the kernels (NAME=VALUE)")
    args = ap.parse_args(argv)
    lib = build(args.jobs, args.verbose, [f"-D{d}" for d in args.defines], args.out)
    print(f"built {lib}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
