"""The ``pth_flash_attn_fwd`` op: library loading, fake kernel, typed wrapper.

Drop-in for the reference module ``python/pth_flash_attn/ops.py``: the same
names (``OP_SCHEMA``, ``pth_flash_attn_fwd``, ``pth_flash_attn_fwd_fake``,
``is_available``), the same schema and the same metadata checks with the same
messages, in the same order, as the C++ op (``csrc/torch_op.cpp``), so a bad
call fails identically at ``torch.compile`` trace time and at run time
(reference ops.py:125-327).

Importing this module loads ``_C.so`` (the op library, built by
``pth-flash-attn_amd/build.py`` next to this file) with
``torch.ops.load_library`` and registers the fake kernel. There is no CPU
compute path: on a GPU box the wrapper raises if the library is missing, and
the CPU registration of the op only validates its arguments.
"""

from __future__ import annotations

import math
from pathlib import Path

import torch

from pth_flash_attn.planner import (
    MAX_ROWS_PER_CTA,
    MMA_ROWS_PER_WARP,
    SUPPORTED_HEAD_SIZES,
    WINDOWED_HEAD_SIZES,
    WM_CHOICES,
)

OP_NAMESPACE = "pth_flash_attn"
OP_NAME = "pth_flash_attn_fwd"
OP_QUALNAME = f"{OP_NAMESPACE}::{OP_NAME}"
# Identical to the m.def() text of csrc/torch_op.cpp and of the reference.
OP_SCHEMA = (
    "pth_flash_attn_fwd(Tensor! out, Tensor q, Tensor k_cache, "
    "Tensor v_cache, Tensor k_scale, Tensor v_scale, Tensor block_table, "
    "Tensor seq_lens, Tensor query_start_loc, int max_query_len, int wm, "
    "int num_splits, float softmax_scale, Tensor! ws_o, Tensor! ws_lse, "
    "int window=0, bool causal=True) -> ()"
)
LIBRARY_PATH = Path(__file__).with_name("_C.so")

_DTYPE_NAMES = {
    torch.bfloat16: "bfloat16",
    torch.float16: "float16",
    torch.float32: "float32",
    torch.int8: "int8",
    torch.int32: "int32",
    torch.int64: "int64",
}


def _fail(*parts: object) -> None:
    raise RuntimeError("pth_flash_attn_fwd: " + "".join(str(p) for p in parts))


def _dtype_name(dtype: torch.dtype) -> str:
    return _DTYPE_NAMES.get(dtype, "an unsupported dtype")


def _want_dim(t: torch.Tensor, n: int, name: str) -> None:
    if t.dim() != n:
        _fail(name, " must be ", n, "-D, got ", t.dim(), "-D")


def _want_dtype(t: torch.Tensor, dtype: torch.dtype, name: str) -> None:
    if t.dtype != dtype:
        _fail(name, " must be ", _dtype_name(dtype), ", got ", _dtype_name(t.dtype))


def _want_size(t: torch.Tensor, dim: int, size: int, name: str, what: str) -> None:
    if t.size(dim) != size:
        _fail(name, ".size(", dim, ") must equal ", what, " = ", size, ", got ", t.size(dim))


def _want_inner_contiguous(t: torch.Tensor, name: str) -> None:
    if t.stride(-1) != 1:
        _fail(name, " must have stride 1 in its last dimension, got ", t.stride(-1))


def _want_device(t: torch.Tensor, q: torch.Tensor, name: str) -> None:
    if t.device != q.device:
        _fail(name, " must be on the same device as q")


def _check_metadata(
    out: torch.Tensor,
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    k_scale: torch.Tensor,
    v_scale: torch.Tensor,
    block_table: torch.Tensor,
    seq_lens: torch.Tensor,
    query_start_loc: torch.Tensor,
    max_query_len: int,
    wm: int,
    num_splits: int,
    softmax_scale: float,
    ws_o: torch.Tensor,
    ws_lse: torch.Tensor,
    window: int = 0,
    causal: bool = True,
) -> None:
    """The op's metadata checks, in the C++ order with the C++ messages."""
    _want_dim(q, 3, "q")
    if q.dtype not in (torch.bfloat16, torch.float16):
        _fail("q must be bfloat16 or float16, got ", _dtype_name(q.dtype))
    T, Hq, D = q.shape
    if D not in SUPPORTED_HEAD_SIZES:
        _fail("head size D = q.size(2) must be 64, 128 or 256, got ", D)
    _want_inner_contiguous(q, "q")

    _want_dim(out, 3, "out")
    _want_dtype(out, q.dtype, "out (same dtype as q)")
    _want_size(out, 0, T, "out", "T")
    _want_size(out, 1, Hq, "out", "Hq")
    _want_size(out, 2, D, "out", "D")
    _want_inner_contiguous(out, "out")

    _want_dim(k_cache, 4, "k_cache")
    _want_dim(v_cache, 4, "v_cache")
    _want_dtype(k_cache, torch.int8, "k_cache")
    _want_dtype(v_cache, torch.int8, "v_cache")
    NB, BS, Hkv = k_cache.shape[:3]
    _want_size(k_cache, 3, D, "k_cache", "D")
    for dim, size, what in ((0, NB, "NB"), (1, BS, "BS"), (2, Hkv, "Hkv"), (3, D, "D")):
        _want_size(v_cache, dim, size, "v_cache", what)
    _want_inner_contiguous(k_cache, "k_cache")
    _want_inner_contiguous(v_cache, "v_cache")

    _want_dim(k_scale, 3, "k_scale")
    _want_dim(v_scale, 3, "v_scale")
    _want_dtype(k_scale, torch.float32, "k_scale")
    _want_dtype(v_scale, torch.float32, "v_scale")
    for scale, name in ((k_scale, "k_scale"), (v_scale, "v_scale")):
        for dim, size, what in ((0, NB, "NB"), (1, BS, "BS"), (2, Hkv, "Hkv")):
            _want_size(scale, dim, size, name, what)

    if Hkv < 1 or Hq % Hkv != 0:
        _fail("Hq = ", Hq, " must be a positive multiple of Hkv = ", Hkv)
    G = Hq // Hkv
    if wm not in WM_CHOICES:
        _fail("wm must be 1, 2 or 4, got ", wm)
    if G > MAX_ROWS_PER_CTA:
        _fail("G = Hq/Hkv = ", G, " exceeds the supported maximum ", MAX_ROWS_PER_CTA)
    if G > MMA_ROWS_PER_WARP * wm:
        _fail("G = Hq/Hkv = ", G, " must be <= 16*wm = ", MMA_ROWS_PER_WARP * wm)

    _want_dim(block_table, 2, "block_table")
    _want_dim(seq_lens, 1, "seq_lens")
    _want_dim(query_start_loc, 1, "query_start_loc")
    for t, name in (
        (block_table, "block_table"),
        (seq_lens, "seq_lens"),
        (query_start_loc, "query_start_loc"),
    ):
        _want_dtype(t, torch.int32, name)
    for t, name in (
        (block_table, "block_table"),
        (seq_lens, "seq_lens"),
        (query_start_loc, "query_start_loc"),
    ):
        _want_inner_contiguous(t, name)
    R = seq_lens.size(0)
    _want_size(query_start_loc, 0, R + 1, "query_start_loc", "num_reqs + 1")
    if block_table.size(0) < R:
        _fail("block_table has ", block_table.size(0), " rows, fewer than num_reqs = ", R)

    if not 0 <= max_query_len <= T:
        _fail("max_query_len must be in [0, T = ", T, "], got ", max_query_len)
    if num_splits < 1:
        _fail("num_splits must be >= 1, got ", num_splits)
    if not (math.isfinite(softmax_scale) and softmax_scale > 0.0):
        # %g formats a double like C++ ostream's default (-1, not -1.0).
        _fail("softmax_scale must be finite and > 0, got ", f"{softmax_scale:g}")
    if window < 0:
        _fail("window must be >= 0, got ", window)
    if (window > 0 or not causal) and D not in WINDOWED_HEAD_SIZES:
        _fail("sliding-window and non-causal attention need head size D = 128, got ", D)

    for t, name in (
        (out, "out"),
        (k_cache, "k_cache"),
        (v_cache, "v_cache"),
        (k_scale, "k_scale"),
        (v_scale, "v_scale"),
        (block_table, "block_table"),
        (seq_lens, "seq_lens"),
        (query_start_loc, "query_start_loc"),
    ):
        _want_device(t, q, name)

    if num_splits > 1:
        _want_dim(ws_o, 4, "ws_o")
        _want_dim(ws_lse, 3, "ws_lse")
        _want_dtype(ws_o, torch.float32, "ws_o")
        _want_dtype(ws_lse, torch.float32, "ws_lse")
        if ws_o.size(0) < num_splits or ws_o.size(1) < T:
            _fail(
                "ws_o must have size(0) >= num_splits = ", num_splits,
                " and size(1) >= T = ", T,
                ", got [", ws_o.size(0), ", ", ws_o.size(1), ", ...]",
            )
        _want_size(ws_o, 2, Hq, "ws_o", "Hq")
        _want_size(ws_o, 3, D, "ws_o", "D")
        if ws_lse.size(0) < num_splits or ws_lse.size(1) < T:
            _fail(
                "ws_lse must have size(0) >= num_splits = ", num_splits,
                " and size(1) >= T = ", T,
                ", got [", ws_lse.size(0), ", ", ws_lse.size(1), ", ...]",
            )
        _want_size(ws_lse, 2, Hq, "ws_lse", "Hq")
        _want_inner_contiguous(ws_o, "ws_o")
        _want_inner_contiguous(ws_lse, "ws_lse")
        _want_device(ws_o, q, "ws_o")
        _want_device(ws_lse, q, "ws_lse")


def pth_flash_attn_fwd_fake(
    out: torch.Tensor,
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    k_scale: torch.Tensor,
    v_scale: torch.Tensor,
    block_table: torch.Tensor,
    seq_lens: torch.Tensor,
    query_start_loc: torch.Tensor,
    max_query_len: int,
    wm: int,
    num_splits: int,
    softmax_scale: float,
    ws_o: torch.Tensor,
    ws_lse: torch.Tensor,
    window: int = 0,
    causal: bool = True,
) -> None:
    """Fake kernel for torch.compile: the metadata checks, no output.

    The op is an out-variant; its in-place writes are declared by ``Tensor!``
    in the schema, so the fake has nothing to create.
    """
    _check_metadata(
        out, q, k_cache, v_cache, k_scale, v_scale, block_table, seq_lens,
        query_start_loc, max_query_len, wm, num_splits, softmax_scale, ws_o,
        ws_lse, window, causal,
    )


# The int8 cache writer registered by the same library (no counterpart in the
# reference, which relies on vLLM's Triton writer; see include/pth_attn.h).
WRITER_NAME = "reshape_and_cache_int8"
WRITER_QUALNAME = f"{OP_NAMESPACE}::{WRITER_NAME}"
WRITER_SCHEMA = (
    "reshape_and_cache_int8(Tensor key, Tensor value, Tensor! k_cache, Tensor! v_cache, "
    "Tensor! k_scale, Tensor! v_scale, Tensor slot_mapping) -> ()"
)


def reshape_and_cache_int8_fake(key: torch.Tensor, value: torch.Tensor, k_cache: torch.Tensor,
                                v_cache: torch.Tensor, k_scale: torch.Tensor,
                                v_scale: torch.Tensor, slot_mapping: torch.Tensor) -> None:
    """Fake of the writer (an in-place op: nothing to create)."""
    if key.dim() != 3 or key.shape != value.shape:
        raise RuntimeError("reshape_and_cache_int8: key and value must be 3-D [T, Hkv, D] "
                           "of the same shape")
    if slot_mapping.dim() != 1 or slot_mapping.shape[0] != key.shape[0]:
        raise RuntimeError("reshape_and_cache_int8: slot_mapping must be int64 [T]")


def _load_library() -> bool:
    if not LIBRARY_PATH.is_file():
        return False
    torch.ops.load_library(str(LIBRARY_PATH))
    torch.library.register_fake(OP_QUALNAME)(pth_flash_attn_fwd_fake)
    torch.library.register_fake(WRITER_QUALNAME)(reshape_and_cache_int8_fake)
    return True


_LIBRARY_LOADED = _load_library()


def is_available() -> bool:
    """True if the op library was built and loaded (fake registered)."""
    return _LIBRARY_LOADED


def pth_flash_attn_fwd(
    out: torch.Tensor,
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    k_scale: torch.Tensor,
    v_scale: torch.Tensor,
    block_table: torch.Tensor,
    seq_lens: torch.Tensor,
    query_start_loc: torch.Tensor,
    max_query_len: int,
    wm: int,
    num_splits: int,
    softmax_scale: float,
    ws_o: torch.Tensor,
    ws_lse: torch.Tensor,
    window: int = 0,
    causal: bool = True,
) -> None:
    """Paged int8 attention for one launch, written into ``out`` in place.

    ``wm`` and ``num_splits`` come from ``planner.plan_launch`` for this slice;
    ``ws_o`` / ``ws_lse`` are views of the load-time workspace with the plan's
    ``ws_o_shape`` / ``ws_lse_shape`` (may be empty when ``num_splits == 1``).
    The query at position p sees keys [lo, hi] with lo = max(0, p - W + 1)
    (0 when W = 0) and hi = p if causal, else min(seq_len - 1, p + W - 1)
    (seq_len - 1 when W = 0). Allocates nothing, reads no device data on the
    host, never synchronises.

    Raises:
        RuntimeError: the library is not built, an argument is invalid, or the
            tensors are CPU tensors (the CPU registration only validates).
    """
    if not _LIBRARY_LOADED:
        raise RuntimeError(
            f"pth_flash_attn_fwd: op library {LIBRARY_PATH} is not built; run "
            "python pth-flash-attn_amd/build.py"
        )
    torch.ops.pth_flash_attn.pth_flash_attn_fwd.default(
        out, q, k_cache, v_cache, k_scale, v_scale, block_table, seq_lens,
        query_start_loc, max_query_len, wm, num_splits, softmax_scale, ws_o,
        ws_lse, window, causal,
    )


def reshape_and_cache_int8(key: torch.Tensor, value: torch.Tensor, k_cache: torch.Tensor,
                           v_cache: torch.Tensor, k_scale: torch.Tensor, v_scale: torch.Tensor,
                           slot_mapping: torch.Tensor) -> None:
    """Quantise ``key`` / ``value`` [T, Hkv, D] into the int8_per_token_head cache.

    Token t goes to slot ``slot_mapping[t]`` (page ``slot // block_size``,
    in-page slot ``slot % block_size``; a negative slot skips the token). Per
    (token, head): scale = max(absmax / 127, 1e-6) in fp32 and
    int8 = trunc(clamp(x * (1 / scale) +- 0.5, -128, 127)), as vLLM's writer
    (mirrored by the reference's python/pth_testing/reference.py:76-103).
    The caches are the four views ``pth_flash_attn_fwd`` reads.
    """
    if not _LIBRARY_LOADED:
        raise RuntimeError(
            f"reshape_and_cache_int8: op library {LIBRARY_PATH} is not built; run "
            "python pth-flash-attn_amd/build.py"
        )
    torch.ops.pth_flash_attn.reshape_and_cache_int8.default(
        key, value, k_cache, v_cache, k_scale, v_scale, slot_mapping)
