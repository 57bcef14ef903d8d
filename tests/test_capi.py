"""The C ABI library on the CPU: it loads, exports exactly what
include/pth_attn.h declares, has the reference's struct layout, and rejects
invalid arguments with EINVAL and a message before touching a device.

Struct sizes are the reference's (csrc/pth_attn/attn_args.h, ABI v2:
sizeof(PthAttnArgs) = 352, sizeof(PthAttnCombineArgs) = 136), so a caller
built against the reference's header passes the library's checks.
"""

from __future__ import annotations

import ctypes
import re
import shutil
import subprocess
from pathlib import Path

import pytest
import torch

from pth_flash_attn import capi

REPO = Path(__file__).resolve().parent.parent
HEADER = REPO / "include" / "pth_attn.h"

needs_lib = pytest.mark.skipif(not capi.LIBRARY_PATH.is_file(), reason="libpth_attn.so not built")


def header_functions() -> set[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return set(re.findall(r"^\s*(?:const\s+)?\w+\*?\s+\*?(pth_attn_\w+)\s*\(", text, flags=re.M))


@pytest.fixture(scope="module")
def lib() -> capi.AttnLib:
    return capi.AttnLib()


def test_exported_symbols_list_is_the_header():
    assert header_functions() == set(capi.EXPORTED_SYMBOLS)


@needs_lib
def test_library_exports_every_symbol(lib):
    for name in capi.EXPORTED_SYMBOLS:
        assert hasattr(lib.lib, name), name
    if shutil.which("nm"):
        out = subprocess.run(["nm", "-D", "--defined-only", str(capi.LIBRARY_PATH)],
                             capture_output=True, text=True, check=True).stdout
        exported = {ln.split()[-1] for ln in out.splitlines() if " T " in ln}
        ours = {s for s in exported if s.startswith("pth_attn_")}
        assert ours == set(capi.EXPORTED_SYMBOLS)


@needs_lib
def test_identity_and_struct_sizes(lib):
    L = lib.lib
    assert L.pth_attn_abi_version() == capi.ABI_VERSION == 2
    assert L.pth_attn_attn_args_bytes() == ctypes.sizeof(capi.PthAttnArgs) == 352
    assert L.pth_attn_combine_args_bytes() == ctypes.sizeof(capi.PthAttnCombineArgs) == 136
    assert L.pth_attn_options_bytes() == ctypes.sizeof(capi.PthAttnOptions) == 12
    assert L.pth_attn_write_args_bytes() == ctypes.sizeof(capi.PthAttnWriteArgs)
    assert L.pth_attn_has_cuda() == 1


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
@pytest.mark.parametrize("struct", [capi.PthAttnArgs, capi.PthAttnCombineArgs, capi.PthAttnOptions,
                                    capi.PthAttnWriteArgs])
def test_ctypes_mirror_matches_the_header(struct, tmp_path):
    """Every field offset of the ctypes mirror equals offsetof() in the C header."""
    name = struct.__name__
    fields = [f[0] for f in struct._fields_]
    src = tmp_path / "off.c"
    src.write_text("#include <stddef.h>\n#include <stdio.h>\n#include \"pth_attn.h\"\n"
                   "int main(void) {\n" + "".join(
                       f'  printf("%zu\\n", offsetof({name}, {f}));\n' for f in fields)
                   + f'  printf("%zu\\n", sizeof({name}));\n  return 0;\n}}\n')
    exe = tmp_path / "off"
    subprocess.run(["gcc", "-std=c11", f"-I{REPO / 'include'}", str(src), "-o", str(exe)],
                   check=True)
    got = [int(x) for x in subprocess.run([str(exe)], capture_output=True, text=True,
                                          check=True).stdout.split()]
    want = [getattr(struct, f).offset for f in fields] + [ctypes.sizeof(struct)]
    assert got == want


def test_reference_cpu_path_agrees_on_the_struct_size():
    import oracle
    R = oracle.ref_lib()
    if R is None:
        pytest.skip("oracle/_ref not built")
    assert R.pth_ref_attn_args_bytes() == ctypes.sizeof(capi.PthAttnArgs)


def _valid_args(D: int = 128, splits: int = 1):
    T, Hq, Hkv, NB, BS = 2, 8, 2, 3, 16
    cell = torch.zeros(NB, BS, Hkv, 2 * D + 8, dtype=torch.int8)
    q = torch.zeros(T, Hq, D, dtype=torch.bfloat16)
    out = torch.zeros_like(q)
    ws_o = torch.zeros(max(splits, 1), T, Hq, D)
    ws_l = torch.zeros(max(splits, 1), T, Hq)
    keep = (cell, q, out, ws_o, ws_l, torch.zeros(2, NB, dtype=torch.int32),
            torch.ones(2, dtype=torch.int32), torch.tensor([0, 1, 2], dtype=torch.int32))
    a = capi.attn_args(q=q, out=out, k_cache=cell[..., :D], v_cache=cell[..., D + 4:2 * D + 4],
                       k_scale=cell[..., D:D + 4].view(torch.float32)[..., 0],
                       v_scale=cell[..., 2 * D + 4:].view(torch.float32)[..., 0],
                       block_table=keep[5], seq_lens=keep[6], query_start_loc=keep[7],
                       bq=4, num_splits=splits, softmax_scale=D ** -0.5, ws_o=ws_o, ws_lse=ws_l)
    return a, keep


@needs_lib
@pytest.mark.parametrize(("mutate", "msg"), [
    (lambda a: setattr(a, "abi_version", 1), "abi_version 1 != library ABI 2"),
    (lambda a: setattr(a, "struct_bytes", 344), "struct_bytes 344 != sizeof(PthAttnArgs) 352"),
    (lambda a: (setattr(a, "head_size", 64), setattr(a, "window", 16)), "need head size D = 128"),
    (lambda a: (setattr(a, "head_size", 256), setattr(a, "causal", 0)), "need head size D = 128"),
    (lambda a: setattr(a, "head_size", 96), "head_size"),
    (lambda a: setattr(a, "num_splits", 0), "num_splits must be >= 1"),
    (lambda a: setattr(a, "softmax_scale", float("nan")), "softmax_scale"),
    (lambda a: setattr(a, "causal", 2), "causal must be 0 or 1"),
    (lambda a: setattr(a, "window", -1), "window must be >= 0"),
    (lambda a: setattr(a, "q", None), "non-NULL"),
    (lambda a: setattr(a, "q", a.q + 2), "q"),
    (lambda a: setattr(a, "bq", 17), "bq * G"),
])
def test_attention_rejects_invalid_arguments(lib, mutate, msg):
    a, keep = _valid_args()
    mutate(a)
    assert lib.attention(a) == capi.PTH_ATTN_EINVAL
    assert msg in lib.last_error(), lib.last_error()


@needs_lib
def test_null_and_option_errors(lib):
    L = lib.lib
    assert L.pth_attn_attention(None, None) == capi.PTH_ATTN_EINVAL
    assert "args is NULL" in lib.last_error()
    assert L.pth_attn_combine(None, None) == capi.PTH_ATTN_EINVAL
    a, keep = _valid_args()
    opt = capi.PthAttnOptions(capi.ABI_VERSION, ctypes.sizeof(capi.PthAttnOptions), 2)
    assert L.pth_attn_attention_ex(ctypes.byref(a), ctypes.byref(opt), None) == capi.PTH_ATTN_EINVAL
    assert "loader" in lib.last_error()
    opt = capi.PthAttnOptions(capi.ABI_VERSION, 4, 0)
    assert L.pth_attn_attention_ex(ctypes.byref(a), ctypes.byref(opt), None) == capi.PTH_ATTN_EINVAL
    assert "options" in lib.last_error()
    assert L.pth_attn_attention_lse(ctypes.byref(a), None, 0, 0, None) == capi.PTH_ATTN_EINVAL
    assert "lse must be non-NULL" in lib.last_error()


@needs_lib
def test_split_launch_needs_workspace(lib):
    a, keep = _valid_args(splits=4)
    a.ws_o = None
    assert lib.attention(a) == capi.PTH_ATTN_EINVAL
    assert "ws_o" in lib.last_error()


@needs_lib
def test_combine_rejects_invalid_arguments(lib):
    T, Hq, D, S = 2, 8, 128, 3
    ws_o, ws_l = torch.zeros(S, T, Hq, D), torch.zeros(S, T, Hq)
    out = torch.zeros(T, Hq, D, dtype=torch.bfloat16)
    qsl = torch.tensor([0, 1, 2], dtype=torch.int32)
    c = capi.combine_args(ws_o=ws_o, ws_lse=ws_l, out=out, query_start_loc=qsl, num_reqs=2,
                          num_splits=S)
    c.head_size = 96
    assert lib.combine(c) == capi.PTH_ATTN_EINVAL
    assert "head_size" in lib.last_error()
    c.head_size = 128
    c.num_splits = 0
    assert lib.combine(c) == capi.PTH_ATTN_EINVAL
    c.num_splits = S
    c.struct_bytes = 8
    assert lib.combine(c) == capi.PTH_ATTN_EINVAL
    assert "mismatch" in lib.last_error()


@needs_lib
def test_tiling(lib):
    assert lib.tiling(128, 4, 4) == (64, 32, 1)
    assert lib.tiling(128, 16, 4) == (64, 32, 4)
    assert lib.tiling(128, 10, 6) == (64, 32, 4)
    assert lib.tiling(64, 4, 4) == (64, 32, 1)
    assert lib.tiling(256, 16, 4) == (64, 32, 4)
    with pytest.raises(RuntimeError, match="head_size"):
        lib.tiling(96, 1, 4)
    with pytest.raises(RuntimeError, match="64 rows"):
        lib.tiling(128, 17, 4)


@needs_lib
def test_error_is_cleared_by_a_success(lib):
    a, keep = _valid_args()
    a.causal = 5
    assert lib.attention(a) == capi.PTH_ATTN_EINVAL
    lib.tiling(128, 4, 4)
    assert lib.last_error() == ""


@needs_lib
def test_writer_rejects_invalid_arguments(lib):
    key = torch.zeros(2, 2, 128, dtype=torch.bfloat16)
    cell = torch.zeros(3, 16, 2, 264, dtype=torch.int8)
    sm = torch.zeros(2, dtype=torch.int64)
    w = capi.write_args(key=key, value=key, k_cache=cell[..., :128], v_cache=cell[..., 132:260],
                        k_scale=cell[..., 128:132].view(torch.float32)[..., 0],
                        v_scale=cell[..., 260:].view(torch.float32)[..., 0], slot_mapping=sm)
    w.head_size = 96
    assert lib.write_kv(w) == capi.PTH_ATTN_EINVAL
    assert "head_size" in lib.last_error()
    w.head_size = 128
    w.kv_dtype = 7
    assert lib.write_kv(w) == capi.PTH_ATTN_EINVAL
    assert "kv_dtype" in lib.last_error()
    w.kv_dtype = capi.PTH_ATTN_BF16
    w.struct_bytes = 8
    assert lib.write_kv(w) == capi.PTH_ATTN_EINVAL
    assert "sizeof(PthAttnWriteArgs)" in lib.last_error()
    assert lib.lib.pth_attn_write_kv(None, None) == capi.PTH_ATTN_EINVAL
