"""Caches larger than 4 GiB: pages beyond byte offset 2^32 of the pool.

The kernels form a page's address as base + (uint64) block id * page bytes
(every kernel, attn_*.hip), so the block id may address any page of a pool
of any size; a 32-bit product would wrap for pages past 4 GiB and read the
wrong page. These launches read a small set of requests whose pages are a
seeded permutation over a ~5 GB pool (about one page in seven lies beyond
4 GiB), on the page-row kernel (8 KV heads, decode with splits), the
register-load kernel (windowed verify), the row-block kernel (prefill, one
split) and the staged kernel (one KV head), each against the fp64 oracle.
"""

from __future__ import annotations

import zlib

import pytest
import torch

from cases import Batch, Case, assert_parity, compare, oracle_of
from pth_flash_attn.cache import build_cache, make_queries
from test_attn_gpu import run_capi

pytestmark = pytest.mark.gpu

DEV = "cuda"
POOL_BYTES = 5 << 30
SEQ_LENS = [3000, 5000, 700, 9000, 2100, 64, 4096, 1500]


def _pool(Hkv: int, seed: int):
    page = Hkv * 16 * 2 * (128 + 4)
    need = sum(-(-L // 16) for L in SEQ_LENS)
    cache = build_cache(SEQ_LENS, Hkv=Hkv, D=128, block_size=16, seed=seed, device=DEV,
                        spare_blocks=POOL_BYTES // page - need)
    ids = torch.cat([cache.block_table[r, :-(-L // 16)] for r, L in enumerate(SEQ_LENS)])
    beyond = int((ids.long() * page >= (1 << 32)).sum())
    print(f"pool Hkv={Hkv}: {cache.storage.numel() / 2**30:.2f} GiB, {ids.numel()} pages read, "
          f"{beyond} beyond 4 GiB", flush=True)
    assert beyond > 0
    return cache, cache.to("cpu")


@pytest.fixture(scope="module")
def pool8():
    if not torch.cuda.is_available():
        pytest.fail("no GPU visible")
    cache, host = _pool(8, seed=31)
    yield cache, host
    del cache
    torch.cuda.empty_cache()


@pytest.fixture(scope="module")
def pool1():
    if not torch.cuda.is_available():
        pytest.fail("no GPU visible")
    cache, host = _pool(1, seed=32)
    yield cache, host
    del cache
    torch.cuda.empty_cache()


def _check(name, cache, host, q_lens, Hq, Hkv, *, window=0, is_prefill=None, S=None):
    case = Case(name, q_lens=q_lens, seq_lens=SEQ_LENS, Hq=Hq, Hkv=Hkv, window=window,
                is_prefill=is_prefill)
    print(f"case {name}: q_lens={q_lens} S={case.plan().num_splits if S is None else S}",
          flush=True)
    q, qsl = make_queries(q_lens, Hq=Hq, D=128, seed=zlib.crc32(name.encode()) % 1000, device=DEV)
    out, lse = run_capi(Batch(case, cache, q, qsl), num_splits=S)
    ref_out, ref_lse, valid = oracle_of(Batch(case, host, q.cpu(), qsl.cpu()))
    res = compare(out, lse, ref_out, ref_lse, valid)
    print(f"  -> {res}", flush=True)
    assert_parity(res, name=name, strict=False)


def test_large_pool_pagerows_decode(pool8):
    _check("pool-decode", *pool8, [1] * 8, 32, 8)


def test_large_pool_register_load_window(pool8):
    _check("pool-window-q16", *pool8, [16, 16, 16, 16, 16, 16, 16, 16], 32, 8, window=512)


def test_large_pool_row_blocks(pool8):
    _check("pool-prefill", *pool8, [300, 1, 64, 1, 200, 1, 1, 1], 32, 8, is_prefill=True, S=1)


def test_large_pool_staged(pool1):
    _check("pool-staged", *pool1, [1] * 8, 4, 1)
