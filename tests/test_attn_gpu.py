"""GPU parity of the gfx950 kernels against the CPU oracle.

Every test here runs the HIP path (through the C ABI of libpth_attn.so or the
torch op of _C.so) on seeded inputs and compares with the fp64 oracle on the
same bytes, at the path's tolerance (max abs <= 2e-3, mean abs <= 2e-4 on bf16
outputs, |dLSE| <= 1e-3). The five configurations of the path's benchmark are
covered at full size (config 5 on sampled rows), plus a grid of edge cases the
reference's tests cover: padded rows, ragged lengths, block sizes that do not
divide 16, HND pages, padded pages, unaligned bases, fp16 queries, fp32/fp16
outputs, windows and non-causal attention.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from cases import (
    LSE_ABS, Case, Batch, abs_v_batch, assert_parity, compare, launch_args, materialize, oracle_of,
    tile_tokens, uniform_lengths,
)

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _lib():
    from pth_flash_attn import capi
    return capi.AttnLib()


def _require_gpu():
    if not torch.cuda.is_available():
        pytest.fail("no GPU visible: the gpu tests need a gfx950 device")


def run_capi(b: Batch, *, num_splits: int | None = None, out_dtype=None, with_lse=True):
    """Run attention (+ combine) through the C ABI test entry; returns (out, lse)."""
    _require_gpu()
    c = b.case
    plan = c.plan()
    S = plan.num_splits if num_splits is None else num_splits
    bq = tile_tokens(plan.wm, c.G, max(c.q_lens))
    out = torch.full(b.q.shape, float("nan"), dtype=out_dtype or b.q.dtype, device=DEV)
    ws_o = torch.full((S, c.T, c.Hq, c.D), float("nan"), device=DEV) if S > 1 else None
    ws_lse = torch.full((S, c.T, c.Hq), float("nan"), device=DEV) if S > 1 else None
    lse = torch.full((c.T, c.Hq), float("nan"), device=DEV)
    args = launch_args(b, out, num_splits=S, bq=bq, ws_o=ws_o, ws_lse=ws_lse)
    lib = _lib()
    stream = torch.cuda.current_stream().cuda_stream
    if with_lse:
        lib.check(lib.attention_lse(args, lse, stream))
    else:
        # The plain entry points, as an engine would call them: attention,
        # then (S > 1) the public combine over all S splits.
        lib.check(lib.attention(args, stream))
        if S > 1:
            from pth_flash_attn import capi
            cargs = capi.combine_args(ws_o=ws_o, ws_lse=ws_lse, out=out, query_start_loc=b.qsl,
                                      num_reqs=len(c.q_lens), num_splits=S)
            lib.check(lib.combine(cargs, stream))
    torch.cuda.synchronize()
    return out, lse


def run_op(b: Batch, *, num_splits: int | None = None):
    """Run the torch op with the planner's plan; returns out."""
    _require_gpu()
    from pth_flash_attn import ops
    c = b.case
    plan = c.plan()
    S = plan.num_splits if num_splits is None else num_splits
    out = torch.full(b.q.shape, float("nan"), dtype=b.q.dtype, device=DEV)
    ws_o = torch.empty((S, c.T, c.Hq, c.D), device=DEV) if S > 1 else torch.empty(0, device=DEV)
    ws_lse = torch.empty((S, c.T, c.Hq), device=DEV) if S > 1 else torch.empty(0, device=DEV)
    ch = b.cache
    ops.pth_flash_attn_fwd(out, b.q, ch.k_cache, ch.v_cache, ch.k_scale, ch.v_scale,
                           ch.block_table, ch.seq_lens, b.qsl, max(c.q_lens), plan.wm, S,
                           1.0 / math.sqrt(c.D), ws_o, ws_lse, c.window, c.causal)
    torch.cuda.synchronize()
    return out


# fp32 outputs carry no storage rounding: the kernel's own arithmetic (exact
# int8 K/V and q in bf16, fp32 scores, fp32 accumulation) must stay within
# these of the fp64 oracle. The decode kernels keep P as a 16-bit hi + lo
# pair: 1e-4 everywhere.
F32_MAX_ABS = 1e-4
# The row-block kernel (single-split launches with 64-row tiles: prefill,
# wide verify) keeps P in fp16 with the V scale folded in, the reference's
# precision class: each term p_i v_i of a row's sum carries one fp16 rounding
# (relative error <= 2^-11, 11 significant bits), every other operation is
# fp32. So element d of a row is within 2^-11 (sum_i p_i |v_id|) / l of the
# exact value, plus fp32 noise: the oracle run on |V| gives that sum
# exactly, and every element must meet the bound (F32_ROWS_SLACK covers the
# fp32 part). The bound takes every rounding at its largest, u = 2^-11 of its
# term; round-to-nearest errs by u/2 on average (|delta| uniform on [0, u]), so
# the mean error over a launch is at most half the mean bound in expectation,
# which F32_ROWS_MEAN_RATIO gates (a kernel whose rounding error doubled
# would exceed it; random row-block launches measure 0.2-0.37).
F32_ROWS_UNIT = 2.0 ** -11
F32_ROWS_SLACK = 2e-5
F32_ROWS_MEAN_RATIO = 0.5


def fp32_row_block_gate(b: Batch, out32: torch.Tensor, ref_out: np.ndarray,
                        valid: np.ndarray, *, threads: int = 16) -> dict:
    """The row-block kernel's fp32-output check (see F32_ROWS_UNIT): returns
    the worst element's error over its bound and the mean-error ratio."""
    ab = abs_v_batch(b)
    abs_out, _, _ = oracle_of(ab, threads=threads)
    bound = F32_ROWS_UNIT * abs_out[valid] + F32_ROWS_SLACK
    err = np.abs(out32.float().cpu().numpy()[valid].astype(np.float64) - ref_out[valid])
    return {"max_over_bound": float((err / bound).max()) if err.size else 0.0,
            "mean_ratio": float(err.mean() / (F32_ROWS_UNIT * abs_out[valid]).mean())
            if err.size else 0.0,
            "max_abs": float(err.max()) if err.size else 0.0}


def row_block_launch(c: Case, S: int) -> bool:
    """Whether the launcher takes the row-block kernel (attn_launch.hip:
    D = 128, one split, pages of a multiple of 16 keys, bq * G >= 64)."""
    plan = c.plan()
    bq = tile_tokens(plan.wm, c.G, max(c.q_lens))
    return c.D == 128 and S == 1 and c.block_size % 16 == 0 and bq * c.G >= 64


def check_case(c: Case, *, num_splits=None, out_dtype=None, threads=16, strict=False):
    print(f"case {c.name}: q_lens={c.q_lens[:8]} seq_lens={c.seq_lens[:8]} "
          f"Hq={c.Hq} Hkv={c.Hkv} BS={c.block_size} W={c.window} causal={c.causal} "
          f"S={num_splits}", flush=True)
    b = materialize(c, DEV)
    out, lse = run_capi(b, num_splits=num_splits, out_dtype=out_dtype)
    ref_out, ref_lse, valid = oracle_of(b, threads=threads)
    res = compare(out, lse, ref_out, ref_lse, valid)
    print(f"  -> {res}", flush=True)
    assert_parity(res, name=c.name, strict=strict)
    # Rows of padding tokens (beyond qsl[R]) are never written.
    if c.pad_tokens:
        assert torch.isnan(out[sum(c.q_lens):].float()).all(), "padding rows were written"
    # The same launch with fp32 output: the arithmetic alone.
    out32, _ = run_capi(b, num_splits=num_splits, out_dtype=torch.float32)
    r32 = compare(out32, None, ref_out, ref_lse, valid)
    S = c.plan().num_splits if num_splits is None else num_splits
    if row_block_launch(c, S):
        g = fp32_row_block_gate(b, out32, ref_out, valid, threads=threads)
        print(f"  fp32 out (row blocks) -> max abs {g['max_abs']:.3g} mean abs "
              f"{r32['mean_abs']:.3g}, worst error / bound {g['max_over_bound']:.3g}, "
              f"mean error / mean bound {g['mean_ratio']:.3g}", flush=True)
        assert g["max_over_bound"] <= 1.0, f"{c.name}: fp32 error beyond the fp16-P bound ({g})"
        assert g["mean_ratio"] <= F32_ROWS_MEAN_RATIO, f"{c.name}: fp32 mean error ({g})"
    else:
        print(f"  fp32 out -> max abs {r32['max_abs']:.3g} mean abs {r32['mean_abs']:.3g} "
              f"(gate {F32_MAX_ABS:g})", flush=True)
        assert r32["max_abs"] <= F32_MAX_ABS, f"{c.name}: fp32 max abs {r32['max_abs']:.3g}"
    return b, out, lse


# ---------------------------------------------------------------- config 1
@pytest.mark.parametrize("S", [1, 2, 7, 64])
def test_config1_decode_plumbing(S):
    """Config 1: 1 seq, q=1, 4q/1kv, L=1024, BS 16, shuffled blocks."""
    check_case(Case("cfg1", q_lens=[1], seq_lens=[1024], Hq=4, Hkv=1, seed=11), num_splits=S,
               strict=True)


def test_config1_planner_split():
    check_case(Case("cfg1-plan", q_lens=[1], seq_lens=[1024], Hq=4, Hkv=1, seed=12), strict=True)


# ---------------------------------------------------------------- edge grid
GRID = [
    Case("ragged-decode", q_lens=[1, 1, 1, 1], seq_lens=[1, 17, 300, 2049], Hq=8, Hkv=2, seed=1),
    Case("mtp-verify-q4", q_lens=[4, 4, 2], seq_lens=[4, 700, 129], seed=2),
    Case("g1", q_lens=[1, 3], seq_lens=[100, 65], Hq=4, Hkv=4, seed=3),
    Case("g16", q_lens=[1, 1], seq_lens=[100, 65], Hq=32, Hkv=2, seed=4),
    Case("g64", q_lens=[1], seq_lens=[333], Hq=64, Hkv=1, seed=5),
    Case("bs1", q_lens=[2, 1], seq_lens=[40, 77], Hq=8, Hkv=2, block_size=1, seed=6),
    Case("bs7", q_lens=[3, 1], seq_lens=[100, 9], Hq=8, Hkv=2, block_size=7, seed=7),
    Case("bs64", q_lens=[1, 1], seq_lens=[1000, 64], Hq=8, Hkv=2, block_size=64, seed=8),
    Case("bs528", q_lens=[5], seq_lens=[1200], Hq=8, Hkv=2, block_size=528, seed=9),
    Case("hnd", q_lens=[1, 4], seq_lens=[513, 90], layout="HND", seed=10),
    Case("pad-pages", q_lens=[2, 1], seq_lens=[300, 31], Hq=8, Hkv=2, pad_page_bytes=72, seed=11),
    Case("unaligned-base", q_lens=[1, 2], seq_lens=[200, 45], Hq=8, Hkv=2, offset_bytes=4, seed=12),
    Case("padded-rows", q_lens=[1, 1, 3], seq_lens=[50, 2, 400], Hq=8, Hkv=2, pad_tokens=5, seed=13),
    Case("fp16-q", q_lens=[1, 4], seq_lens=[300, 65], q_dtype=torch.float16, seed=14),
    Case("prefill-small", q_lens=[37, 64, 5], seq_lens=[37, 200, 5], Hq=8, Hkv=2, seed=15),
    Case("prefill-g4", q_lens=[100], seq_lens=[1000], seed=16),
    Case("window-causal", q_lens=[16, 16], seq_lens=[3000, 500], window=256, seed=17),
    Case("window-noncausal", q_lens=[8, 3], seq_lens=[2000, 40], window=100, causal=False, seed=18),
    Case("noncausal", q_lens=[4, 1], seq_lens=[300, 77], causal=False, seed=19),
    Case("window-1", q_lens=[4], seq_lens=[100], window=1, seed=20),
    Case("window-prefill", q_lens=[200], seq_lens=[900], Hq=8, Hkv=2, window=64, seed=21),
]


@pytest.mark.parametrize("case", GRID, ids=lambda c: c.name)
def test_grid(case):
    check_case(case)


@pytest.mark.parametrize("case", GRID[:4] + GRID[13:17], ids=lambda c: c.name)
def test_grid_forced_splits(case):
    check_case(case, num_splits=5)


# Single-split launches with 64-row tiles run the row-block kernel (8 waves
# share each key chunk; blocks of 256 / G tokens; short requests split their
# keys over the waves and merge). These cases cover every row-set / key-part
# shape (1 x 8, 2 x 4, 4 x 2, 8 x 1), GQA groups that do not divide a block's
# 32-row wave sets, windows, non-causal rows, fp16 q and other page shapes.
GRID_ROWS = [
    Case("rows-mixed", q_lens=[1, 3, 10, 20, 64, 100, 300, 1],
         seq_lens=[5000, 40, 900, 20, 64, 3000, 1500, 33], seed=50),
    Case("rows-g1", q_lens=[300, 1, 50], seq_lens=[2000, 700, 50], Hq=8, Hkv=8, seed=51),
    Case("rows-g8", q_lens=[70, 2, 33], seq_lens=[500, 4000, 33], Hq=16, Hkv=2, seed=52),
    Case("rows-g6", q_lens=[90, 5], seq_lens=[700, 2500], Hq=12, Hkv=2, seed=53),
    Case("rows-window", q_lens=[200, 7, 40], seq_lens=[900, 3000, 1200], window=64, seed=54),
    Case("rows-window-long", q_lens=[130, 17], seq_lens=[5000, 800], window=1000, seed=55),
    Case("rows-noncausal", q_lens=[100, 2], seq_lens=[400, 50], causal=False, seed=56),
    Case("rows-window-noncausal", q_lens=[80, 4], seq_lens=[2000, 300], window=100,
         causal=False, seed=57),
    Case("rows-fp16q", q_lens=[65, 1], seq_lens=[800, 1000], q_dtype=torch.float16, seed=58),
    Case("rows-bs64", q_lens=[48, 1], seq_lens=[1000, 3333], block_size=64, seed=59),
    Case("rows-bs528", q_lens=[40], seq_lens=[1200], Hq=8, Hkv=2, block_size=528, seed=60),
    Case("rows-hnd", q_lens=[33, 1], seq_lens=[600, 90], layout="HND", seed=61),
    Case("rows-padded", q_lens=[20, 1], seq_lens=[20, 70], pad_tokens=7, seed=62),
    Case("rows-short", q_lens=[17, 1], seq_lens=[17, 1], seed=63),
    # 100 requests: the block walk orders the requests of each group of 64 by
    # their work (two groups here), with runs of equal work (ties broken by
    # request index) and requests without query tokens.
    Case("rows-many-requests",
         q_lens=[40, 1, 0, 70] + [1] * 60 + [33] + [1] * 35,
         seq_lens=[300, 500, 7, 70] + [200 + 40 * (i % 7) for i in range(60)] + [900]
                  + [650] * 20 + [64 + 97 * i for i in range(15)], Hq=8, Hkv=2, seed=65),
    # More blocks than work-groups and more than 64 requests: the walk counts
    # the blocks over both request groups, every work-group starts at a
    # rotated round and wraps around (scanning the groups again), and the 8
    # KV heads of a row tile go to work-groups of one XCD.
    Case("rows-many-requests-rounds",
         q_lens=[1] * 90 + [20, 65, 130, 1, 0, 3, 40, 1, 9, 70],
         seq_lens=[100 + 37 * (i % 11) for i in range(90)]
                  + [400, 65, 900, 2000, 5, 3, 300, 1, 1200, 70],
         Hq=32, Hkv=8, seed=66),
]


@pytest.mark.parametrize("case", GRID_ROWS, ids=lambda c: c.name)
def test_row_blocks(case):
    check_case(case, num_splits=1)


@pytest.mark.parametrize("big", [2.0 ** 12, 2.0 ** 40])
def test_row_blocks_large_v_scales(big):
    """The row-block kernel's fp16 P folds the V scales in under a running
    exponent C: V scales far beyond fp16's range (V values up to 127 * 2^40),
    growing mid-stream (keys [100, 200) scaled by `big`, keys [400, 410) by
    big^2 in the second request), must neither overflow nor lose the small
    rows' precision. Checked relative to each row's largest output."""
    c = Case("rows-bigv", q_lens=[96, 70], seq_lens=[300, 620], seed=70)
    assert row_block_launch(c, 1)
    b = materialize(c, DEV)
    ch = b.cache
    bt = ch.block_table.cpu()
    for r, (lo, hi, f) in enumerate([(100, 200, big), (400, 410, big * big)]):
        for t in range(lo, min(hi, c.seq_lens[r])):
            blk, slot = int(bt[r, t // c.block_size]), t % c.block_size
            ch.v_scale[blk, slot] *= f
    torch.cuda.synchronize()
    ref_out, ref_lse, valid = oracle_of(b)
    out32, lse = run_capi(b, num_splits=1, out_dtype=torch.float32)
    o = out32.cpu().numpy()[valid].astype(np.float64)
    r = ref_out[valid]
    rowmax = np.abs(r).max(axis=-1, keepdims=True)
    rel = np.abs(o - r) / rowmax
    print(f"  big={big:g}: max rel {rel.max():.3g}, rows {valid.sum()}", flush=True)
    assert np.isfinite(o).all()
    assert rel.max() <= 2e-3, rel.max()
    le = np.abs(lse.cpu().numpy()[valid] - ref_lse[valid])
    assert le.max() <= 1e-3, le.max()


def test_row_blocks_deterministic_and_op():
    c = Case("rows-op", q_lens=[100, 1, 9], seq_lens=[2000, 5000, 300], seed=64,
             num_splits=1)
    b = materialize(c, DEV)
    o1, l1 = run_capi(b)
    o2, l2 = run_capi(b)
    assert torch.equal(o1.view(torch.int16), o2.view(torch.int16))
    assert torch.equal(l1, l2)
    o_op = run_op(b)
    o_capi, _ = run_capi(b, with_lse=False)
    assert torch.equal(o_op.view(torch.int16), o_capi.view(torch.int16))


# Head sizes 64 and 256 (the reference op's other instantiations): the
# register-load kernel and the combine at D / 64 columns per lane. Causal
# only, as in the reference (windows and non-causal need D = 128).
GRID_D = [
    Case("d64-decode", q_lens=[1, 1, 1], seq_lens=[1, 300, 2049], Hq=8, Hkv=2, D=64, seed=70),
    Case("d64-verify", q_lens=[4, 2], seq_lens=[700, 129], D=64, seed=71),
    Case("d64-prefill", q_lens=[37, 100], seq_lens=[37, 500], Hq=8, Hkv=2, D=64, seed=72),
    Case("d64-hnd", q_lens=[1, 4], seq_lens=[513, 90], D=64, layout="HND", seed=73),
    Case("d64-padded", q_lens=[1, 3], seq_lens=[50, 400], Hq=8, Hkv=2, D=64, pad_tokens=3,
         seed=74),
    Case("d256-decode-g6", q_lens=[1, 1], seq_lens=[5000, 17], Hq=12, Hkv=2, D=256, seed=75),
    Case("d256-verify-g6", q_lens=[5, 3], seq_lens=[2000, 99], Hq=12, Hkv=2, D=256, seed=76),
    Case("d256-prefill", q_lens=[64, 10], seq_lens=[300, 10], Hq=12, Hkv=2, D=256, seed=77),
    Case("d256-bs7", q_lens=[3, 1], seq_lens=[100, 9], Hq=8, Hkv=2, D=256, block_size=7, seed=78),
    Case("d256-fp16q", q_lens=[1, 4], seq_lens=[300, 65], Hq=8, Hkv=2, D=256,
         q_dtype=torch.float16, seed=79),
    # D = 256 on cell caches with pages of a multiple of 16 keys: the
    # direct-to-LDS kernel with 256-byte swizzled key rows.
    Case("d256-hnd", q_lens=[1, 4], seq_lens=[513, 90], Hq=12, Hkv=2, D=256, layout="HND",
         seed=81),
    Case("d256-bs64", q_lens=[1, 2, 1], seq_lens=[1000, 3333, 64], Hq=12, Hkv=2, D=256,
         block_size=64, seed=82),
    Case("d256-padded", q_lens=[1, 3], seq_lens=[50, 400], Hq=12, Hkv=2, D=256, pad_tokens=3,
         seed=83),
    Case("d256-long-ragged", q_lens=[1, 1, 1, 1, 2, 1], seq_lens=[131072, 7, 31, 33, 20000, 1],
         Hq=12, Hkv=2, D=256, seed=84),
    Case("d256-8kv", q_lens=[1, 3], seq_lens=[4000, 700], Hq=16, Hkv=8, D=256, seed=85),
]


@pytest.mark.parametrize("case", GRID_D, ids=lambda c: c.name)
def test_head_sizes(case):
    check_case(case)


@pytest.mark.parametrize("case", [GRID_D[0], GRID_D[2], GRID_D[5], GRID_D[7]],
                         ids=lambda c: c.name)
@pytest.mark.parametrize("S", [1, 5])
def test_head_sizes_forced_splits(case, S):
    check_case(case, num_splits=S)


# More than 256 splits on few rows: the shared combine with 32-split blocks
# per wave (one speculative round of LSE loads for up to 512 splits).
@pytest.mark.parametrize("case,S", [
    (Case("many-splits-d256", q_lens=[1], seq_lens=[131072], Hq=12, Hkv=2, D=256, seed=86), 512),
    (Case("many-splits-d128", q_lens=[1, 1], seq_lens=[65536, 3000], seed=87), 400),
    (Case("many-splits-verify", q_lens=[4], seq_lens=[40000], seed=88), 300),
], ids=lambda x: x.name if isinstance(x, Case) else str(x))
def test_combine_many_splits(case, S):
    check_case(case, num_splits=S)
    # The op path: the combine reads each row's split count from the marker.
    b = materialize(case, DEV)
    out = run_op(b, num_splits=S)
    ref_out, ref_lse, valid = oracle_of(b)
    assert_parity(compare(out, None, ref_out, ref_lse, valid), name=case.name + "-op",
                  strict=False)


@pytest.mark.parametrize("D", [64, 256])
def test_head_sizes_op_equals_capi(D):
    c = Case(f"op-d{D}", q_lens=[1, 4, 1], seq_lens=[3000, 400, 77], Hq=8, Hkv=2, D=D, seed=80)
    b = materialize(c, DEV)
    o_op = run_op(b)
    o_capi, _ = run_capi(b, with_lse=False)
    assert torch.equal(o_op.view(torch.int16), o_capi.view(torch.int16))


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_out_dtypes(dtype):
    c = Case("out-" + str(dtype), q_lens=[1, 2], seq_lens=[500, 70], Hq=8, Hkv=2, seed=30)
    b = materialize(c, DEV)
    for S in (1, 3):
        out, lse = run_capi(b, num_splits=S, out_dtype=dtype)
        ref_out, ref_lse, valid = oracle_of(b)
        assert_parity(compare(out, lse, ref_out, ref_lse, valid), name=c.name, strict=False)


# The column-split combine (few rows, 65 to 512 splits: a work-group per row
# and 32 columns) for every head size and output dtype, with the LSE.
@pytest.mark.parametrize("D", [64, 128, 256])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("S", [200, 480])
def test_combine_column_parts(D, dtype, S):
    Hq, Hkv = (12, 2) if D == 256 else (8, 2)
    c = Case(f"cols-d{D}", q_lens=[1, 2], seq_lens=[40000, 3000], Hq=Hq, Hkv=Hkv, D=D, seed=31)
    b = materialize(c, DEV)
    out, lse = run_capi(b, num_splits=S, out_dtype=dtype)
    ref_out, ref_lse, valid = oracle_of(b)
    res = compare(out, lse, ref_out, ref_lse, valid)
    print(f"  D={D} {dtype} S={S} -> {res}", flush=True)
    assert_parity(res, name=f"cols D={D} {dtype} S={S}", strict=False)


# ---------------------------------------------------------------- op surface
def test_op_equals_capi_bitwise():
    """The torch op and the C ABI run the same launcher: identical bytes."""
    c = Case("op-vs-capi", q_lens=[1, 4, 1], seq_lens=[3000, 400, 77], seed=40)
    b = materialize(c, DEV)
    o_op = run_op(b)
    o_capi, _ = run_capi(b, with_lse=False)
    assert torch.equal(o_op.view(torch.int16), o_capi.view(torch.int16))


def test_deterministic():
    c = Case("determinism", q_lens=[1] * 8, seq_lens=uniform_lengths(8, 100, 5000, 41), seed=41)
    b = materialize(c, DEV)
    o1, l1 = run_capi(b)
    o2, l2 = run_capi(b)
    assert torch.equal(o1.view(torch.int16), o2.view(torch.int16))
    assert torch.equal(l1, l2)


@pytest.mark.parametrize("S", [7, 64, 256])
def test_public_entry_points_combine_all_splits(S):
    """pth_attn_attention then pth_attn_combine over ALL S splits (the
    reference's launch contract): requests that use fewer splits than S must
    leave -inf in their unused log2-LSE slots, which the workspace starts
    without (it is filled with NaN)."""
    c = Case("public-all-S", q_lens=[1, 4, 1, 2], seq_lens=[100, 3000, 17, 700], Hq=8, Hkv=2,
             seed=21)
    b = materialize(c, DEV)
    out, _ = run_capi(b, num_splits=S, with_lse=False)
    ref_out, ref_lse, valid = oracle_of(b)
    res = compare(out, None, ref_out, ref_lse, valid)
    print(f"  S={S} -> {res}", flush=True)
    assert_parity(res, name=f"public S={S}", strict=False)


@pytest.mark.parametrize("S", [5, 34])
@pytest.mark.parametrize("causal", [True, False])
def test_public_entry_points_windowed_verify(S, causal):
    """As above for windowed verify rows of more than 16 rows per KV head
    (the work units of 32 rows): the unused-split fill and the combine must
    use the attention launch's partition."""
    c = Case("public-window", q_lens=[16, 8, 3], seq_lens=[3000, 700, 40], window=512,
             causal=causal, seed=22)
    b = materialize(c, DEV)
    out, _ = run_capi(b, num_splits=S, with_lse=False)
    ref_out, ref_lse, valid = oracle_of(b)
    res = compare(out, None, ref_out, ref_lse, valid)
    print(f"  S={S} causal={causal} -> {res}", flush=True)
    assert_parity(res, name=f"public window S={S}", strict=False)


# ------------------------------------- split launches of more than 64 requests
# The split partition reads the requests 64 at a time (one lane each): with
# more than 64 the partition is sized over several windows, a wave's stream
# lies in a later window than the first (the cursor refills), and the combine
# and the unused-split fill locate their rows the same way. Every kernel
# family that splits: page-row decode and verify (8 KV heads), the staged
# kernel (2 KV heads), the register-load kernel (windowed verify), and the
# D = 256 / D = 64 kernels.
GRID_MANY = [
    Case("many-decode", q_lens=[1] * 150, seq_lens=uniform_lengths(150, 1, 3000, 7), seed=80),
    Case("many-decode-g4", q_lens=[1] * 200, seq_lens=uniform_lengths(200, 1, 1200, 8),
         Hq=8, Hkv=2, seed=81),
    Case("many-verify-q4", q_lens=[4] * 130, seq_lens=uniform_lengths(130, 4, 2500, 9), seed=82),
    Case("many-window-q16", q_lens=[16] * 100, seq_lens=uniform_lengths(100, 16, 5000, 10),
         window=256, seed=83),
    Case("many-ragged", q_lens=[1, 3, 1, 2] * 33, seq_lens=uniform_lengths(132, 3, 1500, 13),
         Hq=16, Hkv=4, block_size=32, layout="HND", seed=84),
    Case("many-d256", q_lens=[1] * 90, seq_lens=uniform_lengths(90, 1, 2000, 11), Hq=16, Hkv=2,
         D=256, seed=85),
    Case("many-d64", q_lens=[1] * 90, seq_lens=uniform_lengths(90, 1, 2000, 12), Hq=16, Hkv=2,
         D=64, seed=86),
]


@pytest.mark.parametrize("case", GRID_MANY, ids=lambda c: c.name)
def test_many_requests_split(case):
    assert len(case.q_lens) > 64 and case.plan().num_splits > 1
    check_case(case)


@pytest.mark.parametrize("S", [3, 37])
@pytest.mark.parametrize("idx", [0, 2, 3], ids=["decode", "verify", "window"])
def test_many_requests_public_entry_points(idx, S):
    """More than 64 requests through pth_attn_attention then pth_attn_combine
    over all S splits: the unused-split fill must cover every request window."""
    c = GRID_MANY[idx]
    b = materialize(c, DEV)
    out, _ = run_capi(b, num_splits=S, with_lse=False)
    ref_out, ref_lse, valid = oracle_of(b)
    res = compare(out, None, ref_out, ref_lse, valid)
    print(f"  {c.name} S={S} -> {res}", flush=True)
    assert_parity(res, name=f"{c.name} public S={S}", strict=False)


# ------------------------------------------------- page-row integer QK
@pytest.mark.parametrize("q_dtype", [torch.bfloat16, torch.float16], ids=["bf16", "f16"])
@pytest.mark.parametrize("S", [1, None], ids=["S1", "plan"])
def test_pagerows_query_dynamic_range(q_dtype, S):
    """The page-row kernel's integer QK scales each query row by its own power
    of two and splits it into three int8 digits: rows whose magnitudes span
    2^-12 .. 2^12 within one unit, and elements 2^-18 below their row's
    largest (rounded to 2^-20 of it), must match the fp64 oracle beyond the
    output's own rounding and meet the decode kernels' 1e-4 fp32-output
    check."""
    c = Case("pagerows-qrange", q_lens=[1, 1, 4, 1], seq_lens=[700, 2049, 4100, 33],
             q_dtype=q_dtype, seed=31, num_splits=S)
    print(f"case {c.name} {q_dtype} S={S}", flush=True)
    b = materialize(c, DEV)
    gen = torch.Generator(device="cpu").manual_seed(77)
    T, Hq, D = b.q.shape
    row = torch.pow(2.0, torch.randint(-12, 13, (T, Hq, 1), generator=gen).float())
    small = torch.where(torch.rand(T, Hq, D, generator=gen) < 0.2,
                        torch.tensor(2.0 ** -18), torch.tensor(1.0))
    if q_dtype == torch.float16:
        row = row.clamp(max=2.0 ** 8)  # |q| within fp16's range
    b.q.copy_((b.q.float().cpu() * row * small).to(q_dtype).to(DEV))
    out, lse = run_capi(b)
    ref_out, ref_lse, valid = oracle_of(b, threads=16)
    res = compare(out, None, ref_out, ref_lse, valid)
    print(f"  -> {res}", flush=True)
    # Rows scaled by 2^12 have scores of order 10^4 and near one-hot softmax:
    # outputs of order |v| (bf16 storage alone rounds them by up to 8e-3), so
    # the gate is on the error beyond that rounding; the log-sum-exp, of
    # order 10^4, is checked relative to its size (fp32 keeps 24 bits).
    assert_parity(res, name=c.name, strict=False)
    le = np.abs(lse.float().cpu().numpy()[valid] - ref_lse[valid])
    lim = LSE_ABS + 2.0 ** -20 * np.abs(ref_lse[valid])
    print(f"  lse max abs {le.max():.3g}, worst error / limit {(le / lim).max():.3g}", flush=True)
    assert (le <= lim).all()
    out32, _ = run_capi(b, out_dtype=torch.float32)
    r32 = compare(out32, None, ref_out, ref_lse, valid)
    print(f"  fp32 out -> max abs {r32['max_abs']:.3g} (gate {F32_MAX_ABS:g})", flush=True)
    assert r32["max_abs"] <= F32_MAX_ABS


def test_pagerows_nonfinite_query_row():
    """A non-finite query element (NaN or inf) makes its own row's output
    non-finite, as a float QK product would, and leaves the other rows of the
    same unit exact (the integer QK scales each row on its own)."""
    c = Case("pagerows-nonfinite-q", q_lens=[1, 4], seq_lens=[900, 3000], seed=41)
    b = materialize(c, DEV)
    bad = [(0, 5, 17, float("nan")), (2, 9, 100, float("inf"))]  # (token, head, column, value)
    for tok, head, col, val in bad:
        b.q[tok, head, col] = val
    out, _ = run_capi(b, num_splits=1)
    o = out.float().cpu().numpy()
    for tok, head, _, _ in bad:
        assert not np.isfinite(o[tok, head]).any(), (tok, head)
    hb = Batch(c, b.cache.to("cpu"), b.q.cpu(), b.qsl.cpu())
    q_ok = hb.q.clone()
    for tok, head, col, _ in bad:
        q_ok[tok, head, col] = 0.0
    ref_out, ref_lse, valid = oracle_of(Batch(c, hb.cache, q_ok, hb.qsl), threads=16)
    keep = np.repeat(valid[:, None], c.Hq, axis=1)  # (token, head) rows to compare
    for tok, head, _, _ in bad:
        keep[tok, head] = False
    err = np.abs(o[keep].astype(np.float64) - ref_out[keep])
    print(f"  other rows -> max abs {err.max():.3g}, mean abs {err.mean():.3g}", flush=True)
    assert err.max() <= 2e-3 and err.mean() <= 2e-4


# ---------------------------------------------------------------- configs 2-5
def test_config2_batched_decode():
    """Config 2: 64 seqs, q=1, 32q/8kv, L ~ U[1k, 32k], BS 16."""
    lens = uniform_lengths(64, 1024, 32768, seed=2024)
    check_case(Case("cfg2", q_lens=[1] * 64, seq_lens=lens, seed=2), strict=True)


@pytest.mark.parametrize("q", [1, 4])
def test_config3_long_context(q):
    """Config 3: 1 seq, L = 131072, q = 1 (decode) and 4 (MTP verify, causal)."""
    check_case(Case(f"cfg3-q{q}", q_lens=[q], seq_lens=[131072], seed=3 + q), strict=True)


def test_config4_windowed_verify():
    """Config 4: 8 seqs, q=16 causal, window 2048, L ~ U[8k, 64k]."""
    lens = uniform_lengths(8, 8192, 65536, seed=4044)
    check_case(Case("cfg4", q_lens=[16] * 8, seq_lens=lens, window=2048, seed=4), strict=True)


def test_config5_mixed_sampled():
    """Config 5: 4 prefill chunks of 2048 at offsets U[0, 30k] of a 32k context
    plus 60 decodes with L ~ U[2k, 64k], in ONE launch; the oracle checks every
    decode row and 32 sampled prefill row tiles (fp64 over the whole batch
    would take minutes), all on the plain gate."""
    rng = np.random.default_rng(5055)
    offs = [int(x) for x in rng.integers(0, 30 * 1024 + 1, size=4)]
    dec = uniform_lengths(60, 2048, 65536, seed=5056)
    q_lens = [2048] * 4 + [1] * 60
    seq_lens = [o + 2048 for o in offs] + dec
    c = Case("cfg5", q_lens=q_lens, seq_lens=seq_lens, seed=5, is_prefill=True)
    print(f"case cfg5: offsets {offs}", flush=True)
    b = materialize(c, DEV)
    out, lse = run_capi(b)
    hb = Batch(c, b.cache.to("cpu"), b.q.cpu(), b.qsl.cpu())
    import oracle
    dummy = torch.empty(hb.q.shape, dtype=torch.float32)
    args = launch_args(hb, dummy, num_splits=1, bq=1)
    T = c.T
    # 8 row tiles of 16 rows per prefill chunk (its first and last 16 rows and
    # six spread between): 32 tiles, 512 prefill rows, plus every decode row.
    sample = []
    for ch in range(4):
        for t0 in (0, 272, 544, 816, 1088, 1360, 1632, 2032):
            sample.append((2048 * ch + t0, 2048 * ch + t0 + 16))
    sample.append((8192, T))
    assert sum(hi - lo for lo, hi in sample[:-1]) == 512
    for lo, hi in sample:
        ref_out, ref_lse, valid = oracle.attention(args, threads=16, rows=(lo, hi))
        v = np.zeros(T, dtype=bool)
        v[lo:hi] = valid[lo:hi]
        res = compare(out, lse, ref_out, ref_lse, v)
        print(f"  rows [{lo}, {hi}) -> {res}", flush=True)
        assert_parity(res, name=f"cfg5 rows {lo}:{hi}", strict=True)


# ------------------------------------------------- long prefill chunks
# The reference's prefill tests (tests/gpu/test_attn_prefill.py) run q = 2048
# and q = 8192 behind a prefix and check sampled windows of whole row tiles
# (fp64 over a whole 8192-token request would take minutes) plus finiteness
# of the whole output. Same here, on the row-block kernel (D = 128) and the
# D = 256 kernels.
LONG_PREFILL = [
    Case("prefill-8192-prefix", q_lens=[8192, 1], seq_lens=[16384, 5000], is_prefill=True,
         seed=70),
    Case("prefill-8192-window", q_lens=[8192], seq_lens=[12000], window=4096, is_prefill=True,
         seed=71),
    Case("prefill-4096-d256", q_lens=[4096, 3], seq_lens=[6000, 3], Hq=12, Hkv=2, D=256,
         is_prefill=True, seed=72),
]


@pytest.mark.parametrize("case", LONG_PREFILL, ids=lambda c: c.name)
def test_long_prefill_sampled(case):
    import oracle
    print(f"case {case.name}: S={case.plan().num_splits} wm={case.plan().wm}", flush=True)
    b = materialize(case, DEV)
    out, lse = run_capi(b)
    q0 = case.q_lens[0]
    assert torch.isfinite(out[:sum(case.q_lens)].float()).all(), "non-finite output"
    hb = Batch(case, b.cache.to("cpu"), b.q.cpu(), b.qsl.cpu())
    args = launch_args(hb, torch.empty(hb.q.shape, dtype=torch.float32), num_splits=1, bq=1)
    T = case.T
    # 16-row tiles at the chunk's start, its end and six points between, then
    # the other requests' rows.
    sample = [(t, t + 16) for t in np.linspace(0, q0 - 16, 8).astype(int).tolist()]
    if T > q0:
        sample.append((q0, T))
    for lo, hi in sample:
        ref_out, ref_lse, valid = oracle.attention(args, threads=16, rows=(lo, hi))
        v = np.zeros(T, dtype=bool)
        v[lo:hi] = valid[lo:hi]
        res = compare(out, lse, ref_out, ref_lse, v)
        print(f"  rows [{lo}, {hi}) -> {res}", flush=True)
        assert_parity(res, name=f"{case.name} rows {lo}:{hi}", strict=False)
