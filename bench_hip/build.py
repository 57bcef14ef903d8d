"""Build bench_hip/libpth_bench.so (the measured ceilings bench.py reports)
for gfx950 with hipcc; compiles every time it is called, no GPU needed."""

from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
LIB = HERE / "libpth_bench.so"


def build() -> Path:
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, "-std=c++17", "-O3", "--offload-arch=gfx950", "-fPIC", "-shared",
           "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
           str(HERE / "ceilings.hip"), "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"build failed: {' '.join(cmd)}\n{proc.stdout}{proc.stderr}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build())
    sys.exit(0)
