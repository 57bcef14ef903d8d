"""ctypes mirror of the C ABI in include/pth_attn.h (libpth_attn.so).

The structs are field-for-field the reference's (reference
python/pth_testing/ref_capi.py:38-121 mirrors the same layout of
csrc/pth_attn/attn_args.h); the library checks ``abi_version`` and
``struct_bytes``, so a stale mirror fails loudly. ``attn_args`` builds a
``PthAttnArgs`` from torch tensors (byte strides taken from the views).

Loading the library needs no GPU; calling a launch entry point does.
"""

from __future__ import annotations

import ctypes
from pathlib import Path
from typing import Any

LIBRARY_PATH = Path(__file__).with_name("libpth_attn.so")
ABI_VERSION = 2

PTH_ATTN_F32, PTH_ATTN_F16, PTH_ATTN_BF16 = 0, 1, 2
PTH_ATTN_OK, PTH_ATTN_EINVAL, PTH_ATTN_ECUDA, PTH_ATTN_ENOCUDA = 0, -1, -2, -3

# Every symbol include/pth_attn.h declares.
EXPORTED_SYMBOLS = (
    "pth_attn_abi_version",
    "pth_attn_attn_args_bytes",
    "pth_attn_combine_args_bytes",
    "pth_attn_options_bytes",
    "pth_attn_has_cuda",
    "pth_attn_last_error",
    "pth_attn_tiling",
    "pth_attn_attention",
    "pth_attn_attention_ex",
    "pth_attn_combine",
    "pth_attn_attention_lse",
    "pth_attn_attention_kernel",
    "pth_attn_attention_lse_noalloc",
    "pth_attn_combine_kernel",
    "pth_attn_write_args_bytes",
    "pth_attn_write_kv",
)


class PthAttnStream(ctypes.Structure):
    _fields_ = [
        ("data", ctypes.c_void_p),
        ("stride_block", ctypes.c_int64),
        ("stride_slot", ctypes.c_int64),
        ("stride_head", ctypes.c_int64),
    ]


class PthAttnArgs(ctypes.Structure):
    _fields_ = [
        ("abi_version", ctypes.c_int32),
        ("struct_bytes", ctypes.c_int32),
        ("q", ctypes.c_void_p),
        ("q_dtype", ctypes.c_int32),
        ("q_stride_token", ctypes.c_int64),
        ("q_stride_head", ctypes.c_int64),
        ("out", ctypes.c_void_p),
        ("out_dtype", ctypes.c_int32),
        ("out_stride_token", ctypes.c_int64),
        ("out_stride_head", ctypes.c_int64),
        ("k_cache", PthAttnStream),
        ("v_cache", PthAttnStream),
        ("k_scale", PthAttnStream),
        ("v_scale", PthAttnStream),
        ("num_blocks", ctypes.c_int32),
        ("block_size", ctypes.c_int32),
        ("num_kv_heads", ctypes.c_int32),
        ("head_size", ctypes.c_int32),
        ("block_table", ctypes.c_void_p),
        ("block_table_row_stride", ctypes.c_int64),
        ("seq_lens", ctypes.c_void_p),
        ("query_start_loc", ctypes.c_void_p),
        ("num_reqs", ctypes.c_int32),
        ("num_tokens", ctypes.c_int32),
        ("num_q_heads", ctypes.c_int32),
        ("bq", ctypes.c_int32),
        ("num_q_tiles", ctypes.c_int32),
        ("num_splits", ctypes.c_int32),
        ("softmax_scale", ctypes.c_float),
        ("ws_o", ctypes.c_void_p),
        ("ws_o_stride_split", ctypes.c_int64),
        ("ws_o_stride_token", ctypes.c_int64),
        ("ws_o_stride_head", ctypes.c_int64),
        ("ws_lse", ctypes.c_void_p),
        ("ws_lse_stride_split", ctypes.c_int64),
        ("ws_lse_stride_token", ctypes.c_int64),
        ("ws_lse_stride_head", ctypes.c_int64),
        ("window", ctypes.c_int32),
        ("causal", ctypes.c_int32),
    ]


class PthAttnCombineArgs(ctypes.Structure):
    _fields_ = [
        ("abi_version", ctypes.c_int32),
        ("struct_bytes", ctypes.c_int32),
        ("ws_o", ctypes.c_void_p),
        ("ws_o_stride_split", ctypes.c_int64),
        ("ws_o_stride_token", ctypes.c_int64),
        ("ws_o_stride_head", ctypes.c_int64),
        ("ws_lse", ctypes.c_void_p),
        ("ws_lse_stride_split", ctypes.c_int64),
        ("ws_lse_stride_token", ctypes.c_int64),
        ("ws_lse_stride_head", ctypes.c_int64),
        ("out", ctypes.c_void_p),
        ("out_dtype", ctypes.c_int32),
        ("out_stride_token", ctypes.c_int64),
        ("out_stride_head", ctypes.c_int64),
        ("query_start_loc", ctypes.c_void_p),
        ("num_reqs", ctypes.c_int32),
        ("num_tokens", ctypes.c_int32),
        ("num_q_heads", ctypes.c_int32),
        ("head_size", ctypes.c_int32),
        ("num_splits", ctypes.c_int32),
    ]


class PthAttnWriteArgs(ctypes.Structure):
    _fields_ = [
        ("abi_version", ctypes.c_int32),
        ("struct_bytes", ctypes.c_int32),
        ("key", ctypes.c_void_p),
        ("value", ctypes.c_void_p),
        ("key_stride_token", ctypes.c_int64),
        ("key_stride_head", ctypes.c_int64),
        ("value_stride_token", ctypes.c_int64),
        ("value_stride_head", ctypes.c_int64),
        ("kv_dtype", ctypes.c_int32),
        ("num_tokens", ctypes.c_int32),
        ("num_kv_heads", ctypes.c_int32),
        ("head_size", ctypes.c_int32),
        ("slot_mapping", ctypes.c_void_p),
        ("k_cache", PthAttnStream),
        ("v_cache", PthAttnStream),
        ("k_scale", PthAttnStream),
        ("v_scale", PthAttnStream),
        ("block_size", ctypes.c_int32),
        ("num_blocks", ctypes.c_int32),
    ]


class PthAttnOptions(ctypes.Structure):
    _fields_ = [
        ("abi_version", ctypes.c_int32),
        ("struct_bytes", ctypes.c_int32),
        ("loader", ctypes.c_int32),
    ]


class AttnLib:
    """The loaded libpth_attn.so with typed entry points."""

    def __init__(self, path: Path | str = LIBRARY_PATH) -> None:
        p = Path(path)
        if not p.is_file():
            raise RuntimeError(
                f"{p} is not built; run python pth-flash-attn_amd/build.py"
            )
        self.path = p
        lib = ctypes.CDLL(str(p))
        i32, vp = ctypes.c_int32, ctypes.c_void_p
        for name in (
            "pth_attn_abi_version",
            "pth_attn_attn_args_bytes",
            "pth_attn_combine_args_bytes",
            "pth_attn_options_bytes",
            "pth_attn_has_cuda",
            "pth_attn_write_args_bytes",
        ):
            getattr(lib, name).restype = i32
            getattr(lib, name).argtypes = []
        lib.pth_attn_last_error.restype = ctypes.c_char_p
        lib.pth_attn_last_error.argtypes = []
        ip = ctypes.POINTER(i32)
        lib.pth_attn_tiling.restype = i32
        lib.pth_attn_tiling.argtypes = [i32, i32, i32, ip, ip, ip]
        lib.pth_attn_attention.restype = i32
        lib.pth_attn_attention.argtypes = [ctypes.POINTER(PthAttnArgs), vp]
        lib.pth_attn_attention_ex.restype = i32
        lib.pth_attn_attention_ex.argtypes = [
            ctypes.POINTER(PthAttnArgs), ctypes.POINTER(PthAttnOptions), vp]
        lib.pth_attn_combine.restype = i32
        lib.pth_attn_combine.argtypes = [ctypes.POINTER(PthAttnCombineArgs), vp]
        lib.pth_attn_attention_kernel.restype = i32
        lib.pth_attn_attention_kernel.argtypes = [ctypes.POINTER(PthAttnArgs), vp]
        lib.pth_attn_attention_lse.restype = i32
        lib.pth_attn_attention_lse.argtypes = [
            ctypes.POINTER(PthAttnArgs), vp, ctypes.c_int64, ctypes.c_int64, vp]
        lib.pth_attn_combine_kernel.restype = i32
        lib.pth_attn_combine_kernel.argtypes = [ctypes.POINTER(PthAttnArgs), vp]
        lib.pth_attn_attention_lse_noalloc.restype = i32
        lib.pth_attn_attention_lse_noalloc.argtypes = [
            ctypes.POINTER(PthAttnArgs), vp, ctypes.c_int64, ctypes.c_int64, vp]
        lib.pth_attn_write_kv.restype = i32
        lib.pth_attn_write_kv.argtypes = [ctypes.POINTER(PthAttnWriteArgs), vp]
        self.lib = lib

    def write_kv(self, args: PthAttnWriteArgs, stream: int | None = None) -> int:
        """The int8 cache writer (see include/pth_attn.h)."""
        return self.lib.pth_attn_write_kv(ctypes.byref(args), stream)

    def last_error(self) -> str:
        return self.lib.pth_attn_last_error().decode()

    def check(self, rc: int) -> None:
        if rc != PTH_ATTN_OK:
            raise RuntimeError(f"pth_attn status {rc}: {self.last_error()}")

    def attention(self, args: PthAttnArgs, stream: int | None = None) -> int:
        return self.lib.pth_attn_attention(ctypes.byref(args), stream)

    def attention_kernel(self, args: PthAttnArgs, stream: int | None = None) -> int:
        """The attention kernel alone, as the torch op launches it (see the header)."""
        return self.lib.pth_attn_attention_kernel(ctypes.byref(args), stream)

    def combine_kernel(self, args: PthAttnArgs, stream: int | None = None) -> int:
        """The split combine alone, as the torch op launches it (see the header)."""
        return self.lib.pth_attn_combine_kernel(ctypes.byref(args), stream)

    def attention_lse(self, args: PthAttnArgs, lse: Any, stream: int | None = None) -> int:
        """Run attention (+ combine) and write the natural-log LSE into `lse` [T, Hq] fp32."""
        es = lse.element_size()
        return self.lib.pth_attn_attention_lse(
            ctypes.byref(args), lse.data_ptr(), lse.stride(0) * es, lse.stride(1) * es, stream)

    def attention_lse_noalloc(self, args: PthAttnArgs, lse: Any = None,
                              stream: int | None = None) -> int:
        """attention_lse with the split partials in the library's static scratch
        (args.ws_o / ws_lse ignored); lse may be None."""
        if lse is None:
            return self.lib.pth_attn_attention_lse_noalloc(ctypes.byref(args), None, 0, 0, stream)
        es = lse.element_size()
        return self.lib.pth_attn_attention_lse_noalloc(
            ctypes.byref(args), lse.data_ptr(), lse.stride(0) * es, lse.stride(1) * es, stream)

    def combine(self, args: PthAttnCombineArgs, stream: int | None = None) -> int:
        return self.lib.pth_attn_combine(ctypes.byref(args), stream)

    def tiling(self, head_size: int, bq: int, group: int) -> tuple[int, int, int]:
        n, s, w = ctypes.c_int32(), ctypes.c_int32(), ctypes.c_int32()
        self.check(self.lib.pth_attn_tiling(head_size, bq, group, ctypes.byref(n),
                                            ctypes.byref(s), ctypes.byref(w)))
        return n.value, s.value, w.value


def _bstride(t: Any, dim: int) -> int:
    return int(t.stride(dim)) * int(t.element_size())


def _stream(t: Any) -> PthAttnStream:
    return PthAttnStream(t.data_ptr(), _bstride(t, 0), _bstride(t, 1), _bstride(t, 2))


def _dtype_code(dtype: Any) -> int:
    import torch

    return {torch.float32: PTH_ATTN_F32, torch.float16: PTH_ATTN_F16,
            torch.bfloat16: PTH_ATTN_BF16}[dtype]


def attn_args(
    *,
    q: Any,
    out: Any,
    k_cache: Any,
    v_cache: Any,
    k_scale: Any,
    v_scale: Any,
    block_table: Any,
    seq_lens: Any,
    query_start_loc: Any,
    bq: int,
    num_splits: int,
    softmax_scale: float,
    ws_o: Any = None,
    ws_lse: Any = None,
    window: int = 0,
    causal: bool = True,
    num_q_tiles: int = 0,
) -> PthAttnArgs:
    """PthAttnArgs over torch tensors (their data must outlive the launch)."""
    a = PthAttnArgs()
    a.abi_version = ABI_VERSION
    a.struct_bytes = ctypes.sizeof(PthAttnArgs)
    a.q = q.data_ptr()
    a.q_dtype = _dtype_code(q.dtype)
    a.q_stride_token, a.q_stride_head = _bstride(q, 0), _bstride(q, 1)
    a.out = out.data_ptr()
    a.out_dtype = _dtype_code(out.dtype)
    a.out_stride_token, a.out_stride_head = _bstride(out, 0), _bstride(out, 1)
    a.k_cache, a.v_cache = _stream(k_cache), _stream(v_cache)
    a.k_scale, a.v_scale = _stream(k_scale), _stream(v_scale)
    a.num_blocks, a.block_size, a.num_kv_heads = (int(x) for x in k_cache.shape[:3])
    a.head_size = int(q.shape[2])
    a.block_table = block_table.data_ptr()
    a.block_table_row_stride = int(block_table.stride(0))
    a.seq_lens = seq_lens.data_ptr()
    a.query_start_loc = query_start_loc.data_ptr()
    a.num_reqs = int(seq_lens.shape[0])
    a.num_tokens = int(q.shape[0])
    a.num_q_heads = int(q.shape[1])
    a.bq = bq
    a.num_q_tiles = num_q_tiles
    a.num_splits = num_splits
    a.softmax_scale = softmax_scale
    if num_splits > 1:
        a.ws_o = ws_o.data_ptr()
        a.ws_o_stride_split, a.ws_o_stride_token, a.ws_o_stride_head = (
            _bstride(ws_o, 0), _bstride(ws_o, 1), _bstride(ws_o, 2))
        a.ws_lse = ws_lse.data_ptr()
        a.ws_lse_stride_split, a.ws_lse_stride_token, a.ws_lse_stride_head = (
            _bstride(ws_lse, 0), _bstride(ws_lse, 1), _bstride(ws_lse, 2))
    a.window = window
    a.causal = 1 if causal else 0
    return a


def combine_args(*, ws_o: Any, ws_lse: Any, out: Any, query_start_loc: Any,
                 num_reqs: int, num_splits: int) -> PthAttnCombineArgs:
    """PthAttnCombineArgs over torch tensors."""
    c = PthAttnCombineArgs()
    c.abi_version = ABI_VERSION
    c.struct_bytes = ctypes.sizeof(PthAttnCombineArgs)
    c.ws_o = ws_o.data_ptr()
    c.ws_o_stride_split, c.ws_o_stride_token, c.ws_o_stride_head = (
        _bstride(ws_o, 0), _bstride(ws_o, 1), _bstride(ws_o, 2))
    c.ws_lse = ws_lse.data_ptr()
    c.ws_lse_stride_split, c.ws_lse_stride_token, c.ws_lse_stride_head = (
        _bstride(ws_lse, 0), _bstride(ws_lse, 1), _bstride(ws_lse, 2))
    c.out = out.data_ptr()
    c.out_dtype = _dtype_code(out.dtype)
    c.out_stride_token, c.out_stride_head = _bstride(out, 0), _bstride(out, 1)
    c.query_start_loc = query_start_loc.data_ptr()
    c.num_reqs = num_reqs
    c.num_tokens = int(out.shape[0])
    c.num_q_heads = int(out.shape[1])
    c.head_size = int(out.shape[2])
    c.num_splits = num_splits
    return c


def write_args(*, key: Any, value: Any, k_cache: Any, v_cache: Any, k_scale: Any, v_scale: Any,
               slot_mapping: Any) -> PthAttnWriteArgs:
    """PthAttnWriteArgs of torch tensors (raw pointers: keep the tensors alive)."""
    a = PthAttnWriteArgs()
    a.abi_version = ABI_VERSION
    a.struct_bytes = ctypes.sizeof(PthAttnWriteArgs)
    a.key, a.value = key.data_ptr(), value.data_ptr()
    a.key_stride_token, a.key_stride_head = _bstride(key, 0), _bstride(key, 1)
    a.value_stride_token, a.value_stride_head = _bstride(value, 0), _bstride(value, 1)
    import torch
    a.kv_dtype = {torch.float32: PTH_ATTN_F32, torch.float16: PTH_ATTN_F16,
                  torch.bfloat16: PTH_ATTN_BF16}[key.dtype]
    a.num_tokens, a.num_kv_heads, a.head_size = (int(x) for x in key.shape)
    a.slot_mapping = slot_mapping.data_ptr()
    a.k_cache, a.v_cache = _stream(k_cache), _stream(v_cache)
    a.k_scale, a.v_scale = _stream(k_scale), _stream(v_scale)
    a.num_blocks, a.block_size = int(k_cache.shape[0]), int(k_cache.shape[1])
    return a
