"""Seeded random batches on the GPU against the fp64 oracle.

The hand-picked grid of test_attn_gpu.py covers the edges one at a time; this
sweep draws whole batches at random (request count, query and KV lengths,
GQA group, KV heads, head size, window and causality, block size, page
layout, query dtype, forced split count) so that combinations nobody thought
of meet the same gate: max abs <= 2e-3 and mean abs <= 2e-4 on the 16-bit
output, |dLSE| <= 1e-3, and the same launch with fp32 output within 1e-4
(on row-block launches, whose P is fp16, the fp16-P rounding bound of
test_attn_gpu.fp32_row_block_gate).
Sizes are kept small enough for the oracle to finish each case in well under
a second. Every case prints its parameters before it runs.
"""

from __future__ import annotations

import random

import pytest
import torch

from cases import Case
from test_attn_gpu import check_case

pytestmark = pytest.mark.gpu

N_CASES = 150


def random_case(seed: int) -> tuple[Case, int | None]:
    rng = random.Random(seed)
    D = rng.choice([128, 128, 128, 64, 256])
    Hkv = rng.choice([1, 2, 4, 8])
    G = rng.choice([1, 2, 4, 6, 8])
    R = rng.randint(1, 6)
    prefill = rng.random() < 0.25
    q_lens = [rng.randint(1, 120 if prefill else 20) for _ in range(R)]
    seq_lens = [q + rng.randint(0, 2000) for q in q_lens]
    window, causal = 0, True
    if D == 128 and rng.random() < 0.4:
        window = rng.choice([1, 7, 64, 100, 257, 1000, 2048])
        causal = rng.random() < 0.7
    block_size = rng.choice([16, 16, 32, 64, 8, 24])
    layout = rng.choice(["NHD", "HND"])
    q_dtype = rng.choice([torch.bfloat16, torch.bfloat16, torch.float16])
    S = rng.choice([None, None, 1, 3, 17])
    c = Case(f"rand{seed}", q_lens=q_lens, seq_lens=seq_lens, Hq=G * Hkv, Hkv=Hkv, D=D,
             block_size=block_size, window=window, causal=causal, layout=layout,
             q_dtype=q_dtype, seed=1000 + seed)
    return c, S


@pytest.mark.parametrize("seed", range(N_CASES))
def test_random_batch(seed):
    c, S = random_case(seed)
    print(f"random case {seed}: D={c.D} G={c.G} Hkv={c.Hkv} layout={c.layout} "
          f"q_dtype={c.q_dtype} S={S}", flush=True)
    check_case(c, num_splits=S, threads=16)


def random_rows_case(seed: int) -> Case:
    """A prefill-style batch of 65-100 requests on the row-block kernel
    (num_splits = 1, 64-row tiles): more requests than one group of 64 in the
    block walk and, with 8 KV heads, more blocks than work-groups, so the
    walk's rotated rounds wrap and its request groups are scanned again."""
    rng = random.Random(50_000 + seed)
    R = rng.randint(65, 100)
    Hkv = rng.choice([2, 4, 8, 8])
    G = rng.choice([1, 2, 4, 4, 8])
    q_lens = [rng.choice([1, 1, 1, 2, 5, 17, 40, 70, 130]) for _ in range(R)]
    q_lens[rng.randrange(R)] = 0  # a request without query tokens
    seq_lens = [q + rng.randint(0, 600) for q in q_lens]
    window = rng.choice([0, 0, 0, 64, 300])
    return Case(f"rand-rows{seed}", q_lens=q_lens, seq_lens=seq_lens, Hq=G * Hkv, Hkv=Hkv,
                block_size=rng.choice([16, 32, 64]), window=window,
                q_dtype=rng.choice([torch.bfloat16, torch.float16]), is_prefill=True,
                seed=2000 + seed)


@pytest.mark.parametrize("seed", range(8))
def test_random_row_blocks_many_requests(seed):
    c = random_rows_case(seed)
    print(f"random rows case {seed}: R={len(c.q_lens)} G={c.G} Hkv={c.Hkv} W={c.window} "
          f"q_dtype={c.q_dtype}", flush=True)
    check_case(c, num_splits=1, threads=16)
