"""Poisoned null pages: block-table entries that point at vLLM's null block.

vLLM maps the evicted pages of a sliding-window layer, and the unused tail of
every block-table row, to block 0 (its null block), whose bytes are not the
request's. The reference's test (tests/gpu/test_attn_window.py:1-20, 148-200)
points every page wholly below a request's first window position at block 0,
fills block 0 with 0xFF (int8 -1, NaN scales), and requires finite output
within the gate; a negative control reads the same cache without the window
and must see the NaNs.

Here the same is done on every kernel family that can meet such a page:

* register-load (windows <= 4096 keys, config 4's shape), split and unsplit;
* page-row (8 KV heads, NHD cells, windows > 4096 keys) at q = 1 and q = 4;
* per-wave staged (HND pages, windows > 4096 keys);
* row-block (single split, 64-row tiles: windowed prefill chunks);
* the any-block-size kernel (pages of 8 keys);
* D = 64 and D = 256 (no windows there: the null pages are the block-table
  tail past each request's last page, which the kernels address for the
  16-key groups past a request's end).

Every row-tile edge case is present: lengths that are not a multiple of 16 or
32, so a chunk's second 16-key group lies past the end, and windows whose
first key is inside a page, so a chunk's first group lies below it.
"""

from __future__ import annotations

import math

import pytest
import torch

from cases import MAX_ABS, MEAN_ABS, Case, assert_parity, compare, materialize, oracle_of

pytestmark = pytest.mark.gpu

DEV = "cuda"
NULL_BLOCK = 0


def poison_null_pages(b) -> int:
    """Rewrite the batch's block table in place as vLLM lays out a windowed
    layer's: pages wholly below the first query row's window start and
    entries past the request's last page point at block 0, whose bytes are all
    0xFF. A real page that sat in block 0 moves to a spare block first, so the
    visible data is unchanged. Returns the number of null entries."""
    c, cache = b.case, b.cache
    bt = cache.block_table.cpu()
    used = set(bt.flatten().tolist())
    spare = next(x for x in range(cache.num_blocks) if x not in used)
    page = cache.page_bytes
    base = cache.offset_bytes
    st = cache.storage
    st[base + spare * page: base + (spare + 1) * page].copy_(
        st[base + NULL_BLOCK * page: base + (NULL_BLOCK + 1) * page])
    st[base + NULL_BLOCK * page: base + (NULL_BLOCK + 1) * page].fill_(-1)
    nulls = 0
    for r, (ql, L) in enumerate(zip(c.q_lens, c.seq_lens)):
        live = math.ceil(L / c.block_size)
        row = bt[r]
        row[:live] = torch.where(row[:live] == NULL_BLOCK, torch.tensor(spare, dtype=row.dtype),
                                 row[:live])
        nulls += row.shape[0] - live
        row[live:] = NULL_BLOCK
        if c.window > 0 and ql > 0:
            lo = max(0, L - ql - c.window + 1)  # first query row's window start
            below = lo // c.block_size
            row[:below] = NULL_BLOCK
            nulls += below
    cache.block_table.copy_(bt.to(cache.block_table.device))
    return nulls


def run(b, *, num_splits: int, window: int, causal: bool) -> torch.Tensor:
    from pth_flash_attn import ops
    c = b.case
    plan = c.plan()
    S = num_splits
    out = torch.full(b.q.shape, float("nan"), dtype=b.q.dtype, device=DEV)
    ws_o = torch.empty((S, c.T, c.Hq, c.D), device=DEV) if S > 1 else torch.empty(0, device=DEV)
    ws_lse = torch.empty((S, c.T, c.Hq), device=DEV) if S > 1 else torch.empty(0, device=DEV)
    ch = b.cache
    ops.pth_flash_attn_fwd(out, b.q, ch.k_cache, ch.v_cache, ch.k_scale, ch.v_scale,
                           ch.block_table, ch.seq_lens, b.qsl, max(c.q_lens), plan.wm, S,
                           1.0 / math.sqrt(c.D), ws_o, ws_lse, window, causal)
    torch.cuda.synchronize()
    return out


# (name, case kwargs, split counts). Block tables get 4 extra columns so that
# every request has tail entries.
CASES = [
    ("reg-cfg4", dict(q_lens=[16, 16, 16], seq_lens=[9000, 12345, 8203], window=2048), (0, 1, 7)),
    ("reg-noncausal", dict(q_lens=[8, 8], seq_lens=[5003, 2100], window=2048, causal=False),
     (0, 1)),
    ("pagerows-q1", dict(q_lens=[1, 1, 1], seq_lens=[20000, 9001, 6007], window=5000), (0, 1)),
    ("pagerows-q4", dict(q_lens=[4, 4], seq_lens=[30011, 12000], window=6000), (0, 3)),
    ("staged-hnd", dict(q_lens=[1, 4], seq_lens=[15013, 9999], window=4500, layout="HND"),
     (0, 1)),
    ("staged-g8", dict(q_lens=[2, 1], seq_lens=[12007, 7005], Hq=32, Hkv=4, window=5000),
     (0, 1)),
    ("rows-prefill", dict(q_lens=[300, 77, 1], seq_lens=[4000, 3001, 2500], window=1000,
                          is_prefill=True), (1,)),
    ("generic-bs8", dict(q_lens=[4, 1], seq_lens=[3001, 2003], window=700, block_size=8),
     (0, 1)),
    ("d256-tail", dict(q_lens=[4, 1, 1], seq_lens=[5003, 1001, 17], Hq=12, Hkv=2, D=256),
     (0, 1)),
    ("d64-tail", dict(q_lens=[4, 1], seq_lens=[3001, 33], Hq=16, Hkv=4, D=64), (0, 1)),
]


@pytest.mark.parametrize("name,kw,splits", CASES, ids=[c[0] for c in CASES])
def test_null_pages_are_never_used(name, kw, splits):
    if not torch.cuda.is_available():
        pytest.fail("no GPU visible")
    c = Case(name, seed=31, **kw)
    print(f"null pages {name}: {kw}", flush=True)
    b = materialize(c, DEV)
    # Widen the block table so every request has tail entries.
    bt = b.cache.block_table
    b.cache.block_table = torch.cat(
        [bt, torch.zeros(bt.shape[0], 4, dtype=bt.dtype, device=DEV)], dim=1).contiguous()
    ref_out, ref_lse, valid = oracle_of(b)  # the clean cache
    nulls = poison_null_pages(b)
    assert nulls > 0
    for S in splits:
        S = c.plan().num_splits if S == 0 else S
        out = run(b, num_splits=S, window=c.window, causal=c.causal)
        res = compare(out, None, ref_out, ref_lse, valid)
        print(f"  S={S} nulls={nulls} -> {res}", flush=True)
        assert_parity(res, name=f"null-{name}-S{S}", strict=False)
    if c.window > 0:
        # Negative control: without the window the null pages are visible.
        out = run(b, num_splits=c.plan().num_splits, window=0, causal=True)
        rows = valid
    else:
        # Negative control: one visible page pointed at the null block.
        b.cache.block_table[0, 0] = NULL_BLOCK
        out = run(b, num_splits=c.plan().num_splits, window=0, causal=True)
        rows = valid.copy()
        rows[c.q_lens[0]:] = False
    bad = compare(out, None, ref_out, ref_lse, rows)
    print(f"  control -> {bad}", flush=True)
    # The poison is read: the output is not finite, or fails the gate the
    # clean runs above pass (a score with a NaN scale compares false against
    # every bound, so these kernels drop such a key instead of propagating
    # the NaN: the answer lacks the page's keys).
    assert not bad["finite"] or bad["max_excess"] > MAX_ABS or bad["mean_excess"] > MEAN_ABS, \
        "the poisoned pages were not read where they are visible"
