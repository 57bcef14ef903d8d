"""Build the gfx950 libraries of pth-flash-attn_amd in-tree.

Outputs (next to the Python package, so they travel with the source tree):
  python/pth_flash_attn/libpth_attn.so  HIP kernels + launcher + C ABI
                                        (include/pth_attn.h); no torch.
  python/pth_flash_attn/_C.so           the torch op pth_flash_attn::pth_flash_attn_fwd
                                        (CUDA = HIP key and CPU key), linked
                                        against libpth_attn.so.

Usage: python pth-flash-attn_amd/build.py [--lib-only] [-v]
Compiles every time it is called (no staleness check); needs hipcc only, no GPU.
"""

from __future__ import annotations

import argparse
import os
import subprocess
import sys
from pathlib import Path

PKG_ROOT = Path(__file__).resolve().parent
REPO = PKG_ROOT.parent
CSRC = PKG_ROOT / "csrc"
INCLUDE = REPO / "include"
PY_PKG = PKG_ROOT / "python" / "pth_flash_attn"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

HIP_SOURCES = ("attn_fwd.hip", "attn_staged.hip", "attn_rows.hip", "attn_generic.hip", "attn_combine.hip",
               "attn_launch.hip", "attn_writer.hip")
# Packed fp32 VALU ops are disabled for all device code (they have given wrong
# results on this pool); the host pass warns that it does not know the
# feature, which is harmless.
DEVICE_FLAGS = (
    "-std=c++17",
    "-O3",
    f"--offload-arch={ARCH}",
    "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
)

LIB_NAME = "libpth_attn.so"
OP_NAME = "_C.so"


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    out = "\n".join(
        ln for ln in (proc.stdout + proc.stderr).splitlines()
        if "packed-fp32-ops' is not a recognized feature" not in ln
    )
    if proc.returncode != 0:
        raise RuntimeError(f"build failed: {' '.join(cmd)}\n{out}")
    if verbose and out.strip():
        print(out)


def build_lib(verbose: bool = False) -> Path:
    """Compile the HIP kernels and the C ABI into libpth_attn.so."""
    PY_PKG.mkdir(parents=True, exist_ok=True)
    out = PY_PKG / LIB_NAME
    tmp = out.with_suffix(".so.tmp")
    cmd = [
        HIPCC, *DEVICE_FLAGS, "-shared",
        f"-I{INCLUDE}", f"-I{CSRC}",
        *[str(CSRC / s) for s in HIP_SOURCES],
        "-o", str(tmp),
    ]
    _run(cmd, verbose)
    os.replace(tmp, out)
    return out


def build_op(verbose: bool = False) -> Path:
    """Compile the torch op library _C.so against libpth_attn.so."""
    import torch.utils.cpp_extension as ce  # only the build needs torch

    out = PY_PKG / OP_NAME
    tmp = out.with_suffix(".so.tmp")
    inc = [f"-I{p}" for p in ce.include_paths()]
    libdirs = ce.library_paths()
    abi = int(getattr(__import__("torch")._C, "_GLIBCXX_USE_CXX11_ABI", True))
    cmd = [
        HIPCC, "-std=c++17", "-O2", "-fPIC", "-shared",
        "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1",
        f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
        f"-I{INCLUDE}", f"-I{CSRC}", *inc, "-I/opt/rocm/include",
        str(CSRC / "torch_op.cpp"),
        "-o", str(tmp),
        f"-L{PY_PKG}", "-l:" + LIB_NAME, "-Wl,-rpath,$ORIGIN",
        *[f"-L{d}" for d in libdirs],
        "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_hip",
        "-L/opt/rocm/lib", "-lamdhip64",
    ]
    _run(cmd, verbose)
    os.replace(tmp, out)
    return out


def build(verbose: bool = False, lib_only: bool = False) -> list[Path]:
    outs = [build_lib(verbose)]
    if not lib_only:
        outs.append(build_op(verbose))
    return outs


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--lib-only", action="store_true")
    ap.add_argument("-v", "--verbose", action="store_true")
    a = ap.parse_args()
    for p in build(verbose=a.verbose, lib_only=a.lib_only):
        print(p)
    return 0


if __name__ == "__main__":
    sys.exit(main())
