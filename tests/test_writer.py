"""The int8 per-token-head cache writer (pth_attn_write_kv /
torch.ops.pth_flash_attn.reshape_and_cache_int8).

The reference relies on vLLM's Triton writer and mirrors it with
quantize_rows (reference python/pth_testing/reference.py:76-103); its
known-answer vectors are test_reference.py:41-56 (round half away from zero,
scale 1.0) and :58-85 (the 1e-6 scale floor). The kernel must reproduce the
oracle's restatement (oracle_quantize_rows, fp32 step for step) byte for
byte: int8 values and fp32 scales. Cells of skipped tokens (negative slots)
are left untouched. The CPU tests check the op's argument validation; the GPU
tests check the bytes.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from pth_flash_attn import ops
from pth_flash_attn.cache import carve_views, cell_bytes

needs_op = pytest.mark.skipif(not ops.is_available(), reason="op library not built")


def _cache(num_blocks: int, block_size: int, Hkv: int, D: int, device: str, layout="NHD",
           fill: int = 0x5A):
    C = cell_bytes(D)
    storage = torch.full((num_blocks * block_size * Hkv * C,), fill, dtype=torch.uint8,
                         device=device).view(torch.int8)
    return storage, carve_views(storage, num_blocks=num_blocks, block_size=block_size, Hkv=Hkv,
                                D=D, layout=layout)


def _write(key, value, views, slots):
    kc, vc, ks, vs = views
    ops.reshape_and_cache_int8(key, value, kc, vc, ks, vs, slots)


@needs_op
def test_cpu_registration_validates_then_refuses():
    key = torch.zeros(2, 2, 128, dtype=torch.bfloat16)
    _, views = _cache(2, 16, 2, 128, "cpu")
    with pytest.raises(RuntimeError, match="computes on CUDA tensors only"):
        _write(key, key, views, torch.zeros(2, dtype=torch.int64))
    with pytest.raises(RuntimeError, match="head size must be 64, 128 or 256"):
        bad = torch.zeros(2, 2, 96, dtype=torch.bfloat16)
        _write(bad, bad, views, torch.zeros(2, dtype=torch.int64))
    with pytest.raises(RuntimeError, match="slot_mapping must be int64"):
        _write(key, key, views, torch.zeros(2, dtype=torch.int32))


def _expected(x: torch.Tensor) -> tuple[np.ndarray, np.ndarray]:
    q, s = oracle.quantize_rows(x.float().cpu().numpy().reshape(-1, x.shape[-1]))
    return q.reshape(x.shape), s.reshape(x.shape[:-1])


@pytest.mark.gpu
def test_known_answers():
    """test_reference.py:41-56 and :58-85 as cache writes."""
    D, Hkv = 128, 1
    row = torch.zeros(D)
    row[:7] = torch.tensor([127, 2.5, -2.5, 0.5, -0.5, 3.5, -126.5])
    key = torch.stack([row, torch.zeros(D)]).view(2, Hkv, D).cuda()  # fp32 source
    _, views = _cache(1, 16, Hkv, D, "cuda")
    _write(key, key, views, torch.tensor([3, 9], dtype=torch.int64, device="cuda"))
    kc, vc, ks, vs = (t.cpu() for t in views)
    assert kc[0, 3, 0, :7].tolist() == [127, 3, -3, 1, -1, 4, -127]
    assert kc[0, 3, 0, 7:].abs().sum() == 0
    assert ks[0, 3, 0].item() == 1.0 and vs[0, 3, 0].item() == 1.0
    assert ks[0, 9, 0].item() == np.float32(1e-6)  # the floor of an all-zero row
    assert kc[0, 9, 0].abs().sum() == 0


@pytest.mark.gpu
@pytest.mark.parametrize("D", [64, 128, 256])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("layout", ["NHD", "HND"])
def test_bytes_equal_the_oracle(D, dtype, layout):
    gen = torch.Generator().manual_seed(1000 + D)
    T, Hkv, BS, NB = 37, 3, 16, 5
    key = (torch.randn(T, Hkv, D, generator=gen) * 3).to(dtype)
    value = torch.randn(T, Hkv, D, generator=gen).to(dtype)
    key[5] *= 1e-9  # scale floor rows
    slots = torch.randperm(NB * BS, generator=gen)[:T]
    slots[[2, 11, 30]] = -1  # padding tokens: skipped
    storage, views = _cache(NB, BS, Hkv, D, "cuda", layout)
    before = storage.clone()
    _write(key.cuda(), value.cuda(), views, slots.cuda())
    torch.cuda.synchronize()
    kc, vc, ks, vs = (t.cpu() for t in views)
    qk, sk = _expected(key)
    qv, sv = _expected(value)
    written = torch.zeros(storage.numel(), dtype=torch.bool)
    for t in range(T):
        sl = int(slots[t])
        if sl < 0:
            continue
        b, o = divmod(sl, BS)
        assert np.array_equal(kc[b, o].numpy(), qk[t]), (t, "K")
        assert np.array_equal(vc[b, o].numpy(), qv[t]), (t, "V")
        assert np.array_equal(ks[b, o].numpy(), sk[t]), (t, "k_scale")
        assert np.array_equal(vs[b, o].numpy(), sv[t]), (t, "v_scale")
    # Every byte of a cell that belongs to no written slot is untouched.
    C = cell_bytes(D)
    cells = storage.cpu().view(NB, BS, Hkv, C) if layout == "NHD" else \
        storage.cpu().view(NB, Hkv, BS, C).transpose(1, 2)
    old = before.cpu().view(cells.shape) if layout == "NHD" else \
        before.cpu().view(NB, Hkv, BS, C).transpose(1, 2)
    used = {int(x) for x in slots if x >= 0}
    for sl in range(NB * BS):
        if sl not in used:
            b, o = divmod(sl, BS)
            assert torch.equal(cells[b, o], old[b, o]), sl


@pytest.mark.gpu
def test_written_cache_reads_back_through_attention():
    """A cache written by the kernel, then read by the attention op, equals
    the oracle over the same bytes (writer and reader agree on the cell)."""
    import math

    from cases import Batch, Case, assert_parity, compare, oracle_of
    from pth_flash_attn.cache import PagedCache
    gen = torch.Generator().manual_seed(7)
    Hq, Hkv, D, BS = 8, 2, 128, 16
    L = [300, 45]
    NB = sum((x + BS - 1) // BS for x in L) + 2
    storage, views = _cache(NB, BS, Hkv, D, "cuda")
    perm = torch.randperm(NB, generator=gen)
    bt = torch.zeros(len(L), NB, dtype=torch.int32)
    k = 0
    slots = []
    for r, n in enumerate(L):
        nb = (n + BS - 1) // BS
        bt[r, :nb] = perm[k:k + nb].to(torch.int32)
        k += nb
        slots += [int(bt[r, t // BS]) * BS + t % BS for t in range(n)]
    src_k = torch.randn(sum(L), Hkv, D, generator=gen).to(torch.bfloat16).cuda()
    src_v = torch.randn(sum(L), Hkv, D, generator=gen).to(torch.bfloat16).cuda()
    _write(src_k, src_v, views, torch.tensor(slots, dtype=torch.int64, device="cuda"))
    kc, vc, ks, vs = views
    cache = PagedCache(storage=storage, k_cache=kc, v_cache=vc, k_scale=ks, v_scale=vs,
                       block_table=bt.cuda(), seq_lens=torch.tensor(L, dtype=torch.int32).cuda(),
                       Hkv=Hkv, D=D, block_size=BS, layout="NHD",
                       page_bytes=BS * Hkv * cell_bytes(D))
    q = torch.randn(2, Hq, D, generator=gen).to(torch.bfloat16).cuda()
    qsl = torch.tensor([0, 1, 2], dtype=torch.int32, device="cuda")
    out = torch.zeros_like(q)
    ops.pth_flash_attn_fwd(out, q, kc, vc, ks, vs, cache.block_table, cache.seq_lens, qsl, 1, 1,
                           1, 1.0 / math.sqrt(D), torch.empty(0, device="cuda"),
                           torch.empty(0, device="cuda"))
    torch.cuda.synchronize()
    case = Case("writer-roundtrip", q_lens=[1, 1], seq_lens=L, Hq=Hq, Hkv=Hkv, D=D)
    ref_out, ref_lse, valid = oracle_of(Batch(case, cache, q, qsl))
    assert_parity(compare(out, None, ref_out, ref_lse, valid), name="writer round trip",
                  strict=False)
