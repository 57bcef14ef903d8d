"""pytest setup: import paths and the `gpu` marker.

`-m "not gpu"` runs everything that needs no GPU (oracle pinning, planner,
op checks on CPU tensors, C-ABI symbols); `-m gpu` runs the parity tests on a
gfx950 device through the C ABI and the torch op.
"""

from __future__ import annotations

import sys
from pathlib import Path

REPO = Path(__file__).resolve().parent.parent
for p in (REPO / "pth-flash-attn_amd" / "python", REPO):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a gfx950 GPU (MI355X)")
