"""Build the benchmark's measurement libraries for gfx950 with hipcc (compiles
every time it is called, no GPU needed):
  bench_hip/libpth_bench.so       the measured ceilings bench.py reports;
  bench_hip/libpth_attn_clock.so  the attention library built with
                                  PA_WAVE_CLOCK: the page-row kernel records
                                  each wave's XCD and start / end time
                                  (bench.py --xcd-spread)."""

from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
LIB = HERE / "libpth_bench.so"
CLOCK_LIB = HERE / "libpth_attn_clock.so"
REPO = HERE.parent
CSRC = REPO / "pth-flash-attn_amd" / "csrc"


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


def build_clock() -> Path:
    sys.path.insert(0, str(REPO / "pth-flash-attn_amd"))
    from build import HIP_SOURCES  # the product library's sources

    tmp = CLOCK_LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, "-std=c++17", "-O3", "--offload-arch=gfx950", "-fPIC", "-shared",
           "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", "-DPA_WAVE_CLOCK",
           f"-I{REPO / 'include'}", f"-I{CSRC}", *[str(CSRC / f) for f in HIP_SOURCES],
           "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"build failed: {' '.join(cmd)}\n{proc.stdout}{proc.stderr}")
    os.replace(tmp, CLOCK_LIB)
    return CLOCK_LIB


if __name__ == "__main__":
    print(build())
    print(build_clock())
    sys.exit(0)
