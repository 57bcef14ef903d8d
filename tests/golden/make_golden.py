"""Writes the golden vectors under tests/golden/ from the reference's own
compiled CPU path (oracle/_ref/libpth_ref_host.so, built by ``make -C oracle``
from the reference's sources; reference tools/build_ref_lib.sh:41-48).

Each ``<name>.npz`` holds the inputs (the raw cache bytes with the geometry to
re-carve the K/V/scale views, the block table, lengths, queries) and the
reference's fp32 output for them. The reference tree is needed only here;
the fixtures travel with the repository and are read by tests/test_golden.py
(oracle on the CPU, HIP kernels on the GPU).

Run from the repository root: python tests/golden/make_golden.py
"""

from __future__ import annotations

import math
import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
REPO = HERE.parent.parent
sys.path[:0] = [str(REPO / "pth-flash-attn_amd" / "python"), str(REPO)]

import oracle  # noqa: E402
from pth_flash_attn import capi  # noqa: E402
from pth_flash_attn.cache import build_cache, make_queries  # noqa: E402

# name: (q_lens, seq_lens, Hq, Hkv, block_size, window, causal, layout, pad, num_splits)
CASES = {
    "config1": ([1], [1024], 4, 1, 16, 0, True, "NHD", 0, 1),
    "ragged_causal": ([1, 4, 0, 2], [300, 77, 9, 16], 8, 2, 16, 0, True, "NHD", 0, 1),
    "window_q16": ([16, 3], [400, 40], 8, 2, 16, 100, True, "NHD", 0, 1),
    "noncausal_window_hnd": ([5, 1], [180, 70], 8, 2, 32, 32, False, "HND", 64, 1),
    "noncausal_full": ([4], [150], 4, 1, 16, 0, False, "NHD", 0, 1),
    "split3_combine": ([2, 1], [500, 260], 8, 2, 16, 0, True, "NHD", 0, 3),
}
D = 128
SEED = 2024


def make(name: str, spec) -> dict[str, np.ndarray]:
    q_lens, seq_lens, Hq, Hkv, bs, W, causal, layout, pad, S = spec
    cache = build_cache(seq_lens, Hkv=Hkv, D=D, block_size=bs, seed=SEED, layout=layout,
                        pad_page_bytes=pad)
    q, qsl = make_queries(q_lens, Hq=Hq, D=D, seed=SEED + 1)
    T = q.shape[0]
    out = torch.zeros(T, Hq, D, dtype=torch.float32)
    ws_o = torch.zeros(S, T, Hq, D)
    ws_l = torch.zeros(S, T, Hq)
    scale = 1.0 / math.sqrt(D)
    a = capi.attn_args(q=q, out=out, k_cache=cache.k_cache, v_cache=cache.v_cache,
                       k_scale=cache.k_scale, v_scale=cache.v_scale,
                       block_table=cache.block_table, seq_lens=cache.seq_lens,
                       query_start_loc=qsl, bq=4, num_splits=S, softmax_scale=scale,
                       ws_o=ws_o, ws_lse=ws_l, window=W, causal=causal)
    oracle.reference_attention(a)
    if S > 1:
        c = capi.combine_args(ws_o=ws_o, ws_lse=ws_l, out=out, query_start_loc=qsl,
                              num_reqs=len(q_lens), num_splits=S)
        oracle.reference_combine(c)
    return {
        "storage": cache.storage.numpy(),
        "geometry": np.array([cache.num_blocks, bs, Hkv, D, pad, 0 if layout == "NHD" else 1],
                             dtype=np.int64),
        "block_table": cache.block_table.numpy(),
        "seq_lens": cache.seq_lens.numpy(),
        "query_start_loc": qsl.numpy(),
        "q_bf16_bits": q.view(torch.int16).numpy(),
        "window": np.array(W), "causal": np.array(int(causal)),
        "softmax_scale": np.array(scale, dtype=np.float32),
        "out": out.numpy(),
    }


def main() -> None:
    if oracle.ref_lib() is None:
        raise SystemExit("oracle/_ref/libpth_ref_host.so is not built: make -C oracle")
    for name, spec in CASES.items():
        np.savez_compressed(HERE / f"{name}.npz", **make(name, spec))
        print("wrote", name)


if __name__ == "__main__":
    main()
