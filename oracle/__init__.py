"""CPU oracle for the paged int8 attention path -- TEST INFRASTRUCTURE ONLY.

Imported only by tests/, by ``__graft_entry__.smoke()`` (as the checker) and
by ``bench.py``'s ``cpu_baseline`` leg. The product path never imports it.

Two CPU implementations live here:
  * ``liboracle.so`` (oracle.c): this repository's restatement of the
    reference's fp64 reference (reference python/pth_testing/reference.py:
    76-103 quantize_rows, 553-671 visible_mask / ref_attention, and
    csrc/pth_attn/combine_kernel.cuh:255-300 combine_row);
  * ``_ref/libpth_ref_host.so`` (optional): the reference's own scalar CPU
    path, compiled by ``make -C oracle`` from the reference's sources where
    they lie (reference tools/build_ref_lib.sh:41-48), used to pin the
    restatement. It takes the same ``PthAttnArgs`` struct (same ABI).

``attention_numpy`` is a third, deliberately plain per-row numpy loop for tiny
cases (no shared code with oracle.c), the brute-force check of the C oracle.

Parity status of each function is recorded in tests/test_oracle.py.
"""

from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

ORACLE_DIR = Path(__file__).resolve().parent
LIB_PATH = ORACLE_DIR / "liboracle.so"
REF_LIB_PATH = ORACLE_DIR / "_ref" / "libpth_ref_host.so"

_lib = None
_ref = None


def build() -> None:
    """Compile liboracle.so (and _ref when the reference tree is present)."""
    subprocess.run(["make", "-s", "-B", "-C", str(ORACLE_DIR)], check=True)


def lib() -> ctypes.CDLL:
    """The loaded liboracle.so (built on first use if missing)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.is_file():
            build()
        L = ctypes.CDLL(str(LIB_PATH))
        L.oracle_quantize_rows.restype = None
        L.oracle_quantize_rows.argtypes = [
            ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32, ctypes.c_void_p, ctypes.c_void_p]
        L.oracle_attention.restype = ctypes.c_int
        L.oracle_attention.argtypes = [
            ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
            ctypes.c_int32, ctypes.c_int64, ctypes.c_int64]
        L.oracle_combine.restype = None
        L.oracle_combine.argtypes = [
            ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int32, ctypes.c_int32,
            ctypes.c_int32, ctypes.c_int32, ctypes.c_void_p, ctypes.c_void_p]
        _lib = L
    return _lib


def ref_lib() -> ctypes.CDLL | None:
    """The reference's own CPU path, or None when _ref was not built."""
    global _ref
    if _ref is None and REF_LIB_PATH.is_file():
        R = ctypes.CDLL(str(REF_LIB_PATH))
        for n in ("pth_ref_attention_host", "pth_ref_combine_host"):
            getattr(R, n).restype = ctypes.c_int32
            getattr(R, n).argtypes = [ctypes.c_void_p]
        R.pth_ref_last_error.restype = ctypes.c_char_p
        R.pth_ref_attn_args_bytes.restype = ctypes.c_int32
        _ref = R
    return _ref


def quantize_rows(x: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Writer mirror on fp32 rows ``x[..., D]`` -> (int8, fp32 scale)."""
    xf = np.ascontiguousarray(x, dtype=np.float32)
    D = xf.shape[-1]
    rows = xf.size // D
    q = np.empty(xf.shape, dtype=np.int8)
    s = np.empty(xf.shape[:-1], dtype=np.float32)
    lib().oracle_quantize_rows(xf.ctypes.data, rows, D, q.ctypes.data, s.ctypes.data)
    return q, s


def attention(args: ctypes.Structure, *, threads: int = 0,
              rows: tuple[int, int] | None = None) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """fp64 reference attention over a PthAttnArgs with HOST pointers.

    Returns (out [T, Hq, D] fp64, lse [T, Hq] fp64 natural log, valid [T] bool).
    Rows of tokens outside every request stay (0, -inf, False). ``rows``
    restricts the computation to tokens [begin, end).
    """
    T, Hq, D = args.num_tokens, args.num_q_heads, args.head_size
    out = np.zeros((T, Hq, D), dtype=np.float64)
    lse = np.full((T, Hq), -np.inf, dtype=np.float64)
    valid = np.zeros(T, dtype=np.uint8)
    b, e = rows if rows is not None else (0, 0)
    rc = lib().oracle_attention(ctypes.addressof(args), out.ctypes.data, lse.ctypes.data,
                                valid.ctypes.data, threads, b, e)
    if rc != 0:
        raise ValueError("oracle_attention: a request has q_len > seq_len")
    return out, lse, valid.astype(bool)


def combine(ws_o: np.ndarray, ws_lse: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """fp64 combine of dense fp32 partials [S, T, Hq, D] / [S, T, Hq] (log2)."""
    o = np.ascontiguousarray(ws_o, dtype=np.float32)
    l2 = np.ascontiguousarray(ws_lse, dtype=np.float32)
    S, T, Hq, D = o.shape
    out = np.zeros((T, Hq, D), dtype=np.float64)
    lse = np.zeros((T, Hq), dtype=np.float64)
    lib().oracle_combine(o.ctypes.data, l2.ctypes.data, S, T, Hq, D, out.ctypes.data,
                         lse.ctypes.data)
    return out, lse


def reference_attention(args: ctypes.Structure) -> None:
    """Run the reference's own CPU scalar path on ``args`` (host pointers).

    Writes ``args.out`` (or the split partials when num_splits > 1) exactly as
    the reference's kernels would. Raises if _ref is not built.
    """
    R = ref_lib()
    if R is None:
        raise RuntimeError("oracle/_ref/libpth_ref_host.so is not built (make -C oracle)")
    rc = R.pth_ref_attention_host(ctypes.addressof(args))
    if rc != 0:
        raise RuntimeError(f"pth_ref_attention_host: {rc}: {R.pth_ref_last_error().decode()}")


def reference_combine(cargs: ctypes.Structure) -> None:
    """Run the reference's own CPU combine on ``cargs`` (host pointers)."""
    R = ref_lib()
    if R is None:
        raise RuntimeError("oracle/_ref/libpth_ref_host.so is not built (make -C oracle)")
    rc = R.pth_ref_combine_host(ctypes.addressof(cargs))
    if rc != 0:
        raise RuntimeError(f"pth_ref_combine_host: {rc}: {R.pth_ref_last_error().decode()}")


def attention_numpy(q: np.ndarray, k: list[np.ndarray], v: list[np.ndarray],
                    qsl: list[int], seq_lens: list[int], scale: float, *,
                    window: int = 0, causal: bool = True) -> tuple[np.ndarray, np.ndarray]:
    """Plain per-(token, head) loop over dense dequantised K/V (tiny cases).

    q [T, Hq, D] float; k[r], v[r] [L_r, Hkv, D] float64 dequantised values.
    Returns (out fp64, lse natural log fp64); rows outside requests are 0 / -inf.
    """
    T, Hq, D = q.shape
    out = np.zeros((T, Hq, D))
    lse = np.full((T, Hq), -np.inf)
    for r, L in enumerate(seq_lens):
        ql = qsl[r + 1] - qsl[r]
        Hkv = k[r].shape[1]
        G = Hq // Hkv
        for i in range(ql):
            p = L - ql + i
            lo = max(0, p - window + 1) if window > 0 else 0
            hi = p if causal else (min(L - 1, p + window - 1) if window > 0 else L - 1)
            for h in range(Hq):
                kk = k[r][lo:hi + 1, h // G].astype(np.float64)
                vv = v[r][lo:hi + 1, h // G].astype(np.float64)
                s = kk @ q[qsl[r] + i, h].astype(np.float64) * scale
                m = s.max()
                w = np.exp(s - m)
                out[qsl[r] + i, h] = (w / w.sum()) @ vv
                lse[qsl[r] + i, h] = m + np.log(w.sum())
    return out, lse
