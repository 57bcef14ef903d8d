"""The kernels' integer geometry (attn_geometry.h), compiled with g++ and
checked by brute force on the CPU: magic division, row-tile ownership,
visible key ranges against the mask definition, split partitions."""

from __future__ import annotations

import shutil
import subprocess
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parent.parent


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_geometry_header(tmp_path):
    exe = tmp_path / "test_geometry"
    subprocess.run(["g++", "-std=c++17", "-O2", "-Wall", "-Werror",
                    f"-I{REPO / 'pth-flash-attn_amd' / 'csrc'}",
                    str(REPO / "tests" / "cpp" / "test_geometry.cpp"), "-o", str(exe)],
                   check=True)
    res = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300)
    assert res.returncode == 0, res.stdout + res.stderr
    assert "ALL OK" in res.stdout
