"""Build tests/hip/libbuffer_range.so (gfx950): test infrastructure only.

Usage: python tests/hip/build_probe.py
"""

from __future__ import annotations

import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
SRC = HERE / "buffer_range.hip"
LIB = HERE / "libbuffer_range.so"


def build() -> Path:
    sys.path.insert(0, str(HERE.parents[1] / "mlx-qsdpa_amd"))
    import build_lib

    cmd = [build_lib.hipcc(), *build_lib.HIPCC_FLAGS, "-shared", str(SRC), "-o", str(LIB)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {SRC.name}:\n{r.stdout}\n{r.stderr}")
    return LIB


if __name__ == "__main__":
    print(f"built {build()}")
