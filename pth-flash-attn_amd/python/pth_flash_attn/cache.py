"""vLLM's ``int8_per_token_head`` paged cache: layout, views and writer mirror.

The format the op reads (reference docs/integration.md:24-91): one int8
storage of pages; per (block, slot, KV head) a cell of ``C = 2 D + 8`` bytes
laid out ``[K: D int8 | k_scale: fp32 | V: D int8 | v_scale: fp32]``, pages
NHD (``[blk, slot, head, C]``) or HND (``[blk, head, slot, C]``), optionally
padded. The op's four inputs are strided views into that storage
(reference reference.py:261-298 carves the same views).

``quantize_rows`` mirrors the writer (vLLM's
``triton_reshape_and_cache_flash_per_token_head_quant``, reference
reference.py:76-103): per (token, head), in fp32, ``scale = max(absmax / 127,
1e-6)``, ``q = x * (1 / scale)``, ``+-0.5`` away from zero, clamp to
``[-128, 127]``, truncate. ``build_cache`` fills a cache for a batch of
requests with seeded N(0, 1) sources, shuffled block ids and poisoned unused
bytes (random bytes, scale 3e4), on any torch device: the benches and GPU
tests build it on the GPU, the CPU tests on the host.
"""

from __future__ import annotations

import math
from collections.abc import Sequence
from dataclasses import dataclass

import torch

SCALE_BYTES = 4
QUANT_MAX = 127.0
SCALE_FLOOR = 1e-6
POISON_SCALE = 3.0e4
SPARE_BLOCKS = 3
LAYOUTS = ("NHD", "HND")


def cell_bytes(D: int) -> int:
    """Bytes of one (token, head) cell: 2 D + 8."""
    return 2 * (D + SCALE_BYTES)


def quantize_rows(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Writer mirror: rows ``x[..., D]`` -> (int8 values, fp32 scales)."""
    xf = x.float()
    scale = torch.clamp(xf.abs().amax(-1) / QUANT_MAX, min=SCALE_FLOOR)
    q = xf * (1.0 / scale).unsqueeze(-1)
    q = torch.where(q >= 0, q + 0.5, q - 0.5)
    q = q.clamp(-128.0, QUANT_MAX)
    return q.to(torch.int8), scale


def carve_views(
    storage: torch.Tensor,
    *,
    num_blocks: int,
    block_size: int,
    Hkv: int,
    D: int,
    layout: str = "NHD",
    pad_page_bytes: int = 0,
    offset_bytes: int = 0,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    """The op's (k_cache, v_cache, k_scale, v_scale) views of a cell storage."""
    if layout not in LAYOUTS:
        raise ValueError(f"layout must be one of {LAYOUTS}")
    if pad_page_bytes % SCALE_BYTES or offset_bytes % SCALE_BYTES:
        raise ValueError("pad_page_bytes and offset_bytes must be multiples of 4")
    C = cell_bytes(D)
    page = Hkv * block_size * C + pad_page_bytes
    if layout == "NHD":
        s_slot, s_head = Hkv * C, C
    else:
        s_slot, s_head = C, block_size * C
    size = (num_blocks, block_size, Hkv)
    # as_strided offsets are absolute within the underlying storage, so a
    # storage that is itself a view (a slice of a larger buffer) adds its own.
    base = storage.storage_offset() + offset_bytes
    k = torch.as_strided(storage, (*size, D), (page, s_slot, s_head, 1), base)
    v = torch.as_strided(storage, (*size, D), (page, s_slot, s_head, 1), base + D + 4)
    f32 = torch.tensor([], dtype=torch.float32, device=storage.device).set_(
        storage.untyped_storage()
    )
    w = SCALE_BYTES
    ks = torch.as_strided(f32, size, (page // w, s_slot // w, s_head // w), (base + D) // w)
    vs = torch.as_strided(f32, size, (page // w, s_slot // w, s_head // w), (base + 2 * D + 4) // w)
    return k, v, ks, vs


def vllm_packed_views(
    kv_packed: torch.Tensor,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    """The op's (k_cache, v_cache, k_scale, v_scale) views of vLLM's packed
    ``int8_per_token_head`` layer cache.

    vLLM keeps one int8 tensor per layer, logically ``[blocks, kv_heads,
    block_size, 2 (D + 4)]``: per (block, head, slot) the cell ``[K | k_scale |
    V | v_scale]`` (reference docs/integration.md:40-46, pth_testing/
    reference.py:268-300). The views index ``[block, slot, head]`` with the
    strides of the tensor itself (never derived from its shape), so padded or
    strided caches work; nothing is copied.
    """
    if kv_packed.dtype == torch.uint8:
        kv_packed = kv_packed.view(torch.int8)  # the same bytes
    if kv_packed.dtype != torch.int8 or kv_packed.dim() != 4:
        raise ValueError("kv_packed must be an int8 (or uint8) tensor "
                         "[blocks, kv_heads, block_size, 2 (D + 4)]")
    nb, hkv, bs, content = kv_packed.shape
    if content % 2 or content // 2 <= SCALE_BYTES:
        raise ValueError(f"cell of {content} bytes is not 2 (D + 4)")
    half = content // 2
    D = half - SCALE_BYTES
    s_blk, s_head, s_slot, s_byte = (int(x) for x in kv_packed.stride())
    if s_byte != 1:
        raise ValueError("the cell bytes of kv_packed must be contiguous")
    if any(x % SCALE_BYTES for x in (s_blk, s_head, s_slot, kv_packed.storage_offset(), D)):
        raise ValueError("kv_packed strides, offset and D must be multiples of 4 bytes")
    base = kv_packed.storage_offset()
    size = (nb, bs, hkv)
    stride = (s_blk, s_slot, s_head)
    k = torch.as_strided(kv_packed, (*size, D), (*stride, 1), base)
    v = torch.as_strided(kv_packed, (*size, D), (*stride, 1), base + half)
    f32 = torch.tensor([], dtype=torch.float32, device=kv_packed.device).set_(
        kv_packed.untyped_storage()
    )
    w = SCALE_BYTES
    stride_w = tuple(x // w for x in stride)
    ks = torch.as_strided(f32, size, stride_w, (base + D) // w)
    vs = torch.as_strided(f32, size, stride_w, (base + half + D) // w)
    return k, v, ks, vs


@dataclass
class PagedCache:
    """A filled cache plus the per-request metadata the op needs."""

    storage: torch.Tensor
    k_cache: torch.Tensor
    v_cache: torch.Tensor
    k_scale: torch.Tensor
    v_scale: torch.Tensor
    block_table: torch.Tensor
    seq_lens: torch.Tensor
    Hkv: int
    D: int
    block_size: int
    layout: str
    page_bytes: int
    pad_page_bytes: int = 0
    offset_bytes: int = 0

    @property
    def num_blocks(self) -> int:
        return int(self.k_cache.shape[0])

    def to(self, device: str | torch.device) -> "PagedCache":
        """The same bytes and metadata on another device (views re-carved)."""
        storage = self.storage.to(device)
        k, v, ks, vs = carve_views(
            storage, num_blocks=self.num_blocks, block_size=self.block_size,
            Hkv=self.Hkv, D=self.D, layout=self.layout,
            pad_page_bytes=self.pad_page_bytes, offset_bytes=self.offset_bytes,
        )
        return PagedCache(
            storage=storage, k_cache=k, v_cache=v, k_scale=ks, v_scale=vs,
            block_table=self.block_table.to(device), seq_lens=self.seq_lens.to(device),
            Hkv=self.Hkv, D=self.D, block_size=self.block_size, layout=self.layout,
            page_bytes=self.page_bytes, pad_page_bytes=self.pad_page_bytes,
            offset_bytes=self.offset_bytes,
        )

    def kv_bytes(self) -> int:
        """Bytes of K, V and both scales of every cached token (the read set)."""
        return int(self.seq_lens.sum()) * self.Hkv * cell_bytes(self.D)


def build_cache(
    seq_lens: Sequence[int],
    *,
    Hkv: int,
    D: int,
    block_size: int,
    seed: int,
    device: str | torch.device = "cpu",
    layout: str = "NHD",
    pad_page_bytes: int = 0,
    offset_bytes: int = 0,
    spare_blocks: int = SPARE_BLOCKS,
    poison: bool = True,
    chunk_tokens: int = 1 << 16,
) -> PagedCache:
    """A paged cache holding ``len(seq_lens)`` requests of seeded N(0,1) K/V.

    Block ids are a seeded permutation over the whole pool (so block tables are
    not monotone), every byte not written by the writer is random and every
    unwritten scale is 3e4, so a read outside a request's tokens shows up as a
    large error. Sources are generated and quantised ``chunk_tokens`` tokens
    at a time, so a multi-GB cache never holds its fp32 sources at once.
    """
    lens = [int(s) for s in seq_lens]
    if any(s < 0 for s in lens) or block_size < 1:
        raise ValueError("seq_lens must be >= 0 and block_size >= 1")
    dev = torch.device(device)
    C = cell_bytes(D)
    page = Hkv * block_size * C + pad_page_bytes
    nblk = [math.ceil(s / block_size) for s in lens]
    need = sum(nblk)
    num_blocks = need + spare_blocks
    gen_cpu = torch.Generator().manual_seed(seed)
    ids = torch.randperm(num_blocks, generator=gen_cpu)
    bt = torch.zeros(len(lens), max(max(nblk, default=0), 1), dtype=torch.int32)
    starts = []
    k = 0
    for r, nb in enumerate(nblk):
        starts.append(k)
        if nb:
            bt[r, :nb] = ids[k : k + nb].to(torch.int32)
        k += nb

    storage = torch.empty(offset_bytes + num_blocks * page, dtype=torch.int8, device=dev)
    gen = torch.Generator(device=dev).manual_seed(seed + 1)
    if poison:
        storage.random_(-128, 128, generator=gen)
    else:
        storage.zero_()
    kc, vc, ks, vs = carve_views(
        storage, num_blocks=num_blocks, block_size=block_size, Hkv=Hkv, D=D,
        layout=layout, pad_page_bytes=pad_page_bytes, offset_bytes=offset_bytes,
    )
    ks.fill_(POISON_SCALE if poison else 0.0)
    vs.fill_(POISON_SCALE if poison else 0.0)

    # Flat (request, position) -> (block id, slot) of every cached token.
    bt_dev = bt.to(dev)
    for r, L in enumerate(lens):
        for t0 in range(0, L, chunk_tokens):
            n = min(chunk_tokens, L - t0)
            pos = torch.arange(t0, t0 + n, device=dev)
            blk = bt_dev[r].long()[pos // block_size]
            slot = pos % block_size
            k_src = torch.randn(n, Hkv, D, generator=gen, device=dev)
            v_src = torch.randn(n, Hkv, D, generator=gen, device=dev)
            kq, kscale = quantize_rows(k_src)
            vq, vscale = quantize_rows(v_src)
            kc[blk, slot] = kq
            vc[blk, slot] = vq
            ks[blk, slot] = kscale
            vs[blk, slot] = vscale
    return PagedCache(
        storage=storage, k_cache=kc, v_cache=vc, k_scale=ks, v_scale=vs,
        block_table=bt_dev, seq_lens=torch.tensor(lens, dtype=torch.int32, device=dev),
        Hkv=Hkv, D=D, block_size=block_size, layout=layout, page_bytes=page,
        pad_page_bytes=pad_page_bytes, offset_bytes=offset_bytes,
    )


def make_queries(
    q_lens: Sequence[int], *, Hq: int, D: int, seed: int,
    dtype: torch.dtype = torch.bfloat16, device: str | torch.device = "cpu",
) -> tuple[torch.Tensor, torch.Tensor]:
    """Seeded N(0,1) queries ``[T, Hq, D]`` and ``query_start_loc`` ``[R + 1]``."""
    dev = torch.device(device)
    gen = torch.Generator(device=dev).manual_seed(seed)
    T = int(sum(q_lens))
    q = torch.randn(T, Hq, D, generator=gen, device=dev).to(dtype)
    qsl = torch.zeros(len(q_lens) + 1, dtype=torch.int32)
    qsl[1:] = torch.tensor(list(q_lens), dtype=torch.int64).cumsum(0).to(torch.int32)
    return q, qsl.to(dev)
