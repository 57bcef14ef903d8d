#!/usr/bin/env python3
"""Benchmark of the hot path: int8 paged attention, D = 128, on one MI355X.

Headline workload ("config 2"): 64 decode sequences, 1
query token each, 32 q / 8 KV heads, D = 128, context lengths uniform in
[1k, 32k] (seeded), vLLM block size 16 with a shuffled block table over one
shared pool, int8 K/V with inline fp32 per-token-head scales, bf16 queries
~ N(0, 1). A step is one layer call: the torch op pth_flash_attn_fwd
(attention kernel + split combine) with the planner's plan, inputs resident
in HBM.

Printed (one JSON line on stdout):
  value / ms_per_step  the headline layer call: algorithmic bytes / time over
                       exactly K eager steps after W warm-up steps (HIP events
                       on the launch stream, synchronised on both sides);
  roofline             the attention kernel alone: the median of 5 blocks of K
                       back-to-back launches (HIP events on the launch
                       stream), interleaved with blocks of K layer calls; its
                       algorithmic bytes per launch
                       against MI355X's 8 TB/s, the HBM traffic per launch from
                       the committed rocprofv3 counter summary (or null), and
                       the measured read ceiling of the same bytes;
  configs              every BASELINE configuration (1, 2, 3 at 1 and 4 query
                       tokens, 4, 5): layer call (eager mean and the median of
                       graph-replayed calls, >= 200 launches; the median of
                       the interleaved blocks), attention and combine kernels
                       alone (median of the interleaved blocks), GB/s or TFLOP/s against the roofline, and
                       the CPU baseline. Inputs smaller than 1 GiB are rotated
                       over copies so that at least 1 GiB passes between two
                       reads of the same bytes (cold MALL);
  read_ceiling         bench_hip/ceilings.hip: config 2's exact cache bytes read
                       with the attention kernel's load pattern and discarded;
  mfma_ceiling         bench_hip/ceilings.hip: dense bf16 MFMA rate at 8 waves
                       per CU;
  cpu_baseline         the repository's CPU oracle (fp64 restatement of the
                       reference's CPU path) on a bounded sample of the
                       headline workload, on the host cores (threads used and
                       the host's CPU count stated).

Usage: python bench.py [--steps K] [--warmup W] [--config 1..5] [--query-tokens 1|4]
                       [--no-cpu] [--only-headline]
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO / "pth-flash-attn_amd" / "python"))
sys.path.insert(1, str(REPO))

PEAK_HBM_GBS = 8000.0
PEAK_BF16_TFLOPS = 2500.0
METRIC = "µs/layer-call + achieved HBM GB/s (% peak), int8 paged decode D=128"


# Untimed warm-up lasts at least this long (seconds of GPU work), W steps at least.
WARMUP_MIN_S = 0.3
GRAPH_REPLAYS = 10  # x 20 layer calls per replay: the median covers 200 launches
KERNEL_BLOCKS = 5  # interleaved blocks of K launches for the per-kernel medians

def workload(config: int, query_tokens: int = 1):
    """(name, q_lens, seq_lens, Hq, Hkv, window, is_prefill) of a BASELINE config.
    query_tokens: config 3's query tokens, 1 (plain decode) or 4 (MTP verify,
    causal within the 4 drafted positions)."""
    import numpy as np

    if config == 1:
        return "cfg1-decode-1seq-4q1kv-L1024", [1], [1024], 4, 1, 0, False
    if config == 2:
        lens = [int(x) for x in np.random.default_rng(2024).integers(1024, 32768 + 1, 64)]
        return "cfg2-decode-64seq-32q8kv-L1k-32k", [1] * 64, lens, 32, 8, 0, False
    if config == 3:
        if query_tokens == 4:
            return "cfg3-verify4-1seq-L131072", [4], [131072], 32, 8, 0, False
        if query_tokens != 1:
            raise SystemExit("config 3 runs at 1 or 4 query tokens")
        return "cfg3-decode-1seq-L131072", [1], [131072], 32, 8, 0, False
    if config == 4:
        lens = [int(x) for x in np.random.default_rng(4044).integers(8192, 65536 + 1, 8)]
        return "cfg4-window2048-verify16-8seq", [16] * 8, lens, 32, 8, 2048, False
    if config == 5:
        rng = np.random.default_rng(5055)
        offs = [int(x) for x in rng.integers(0, 30 * 1024 + 1, 4)]
        dec = [int(x) for x in np.random.default_rng(5056).integers(2048, 65536 + 1, 60)]
        return ("cfg5-mixed-4x2048prefill-60decode", [2048] * 4 + [1] * 60,
                [o + 2048 for o in offs] + dec, 32, 8, 0, True)
    raise SystemExit(f"unknown config {config}")


def visible_keys(q_lens, seq_lens, window, causal=True):
    """Per request: number of distinct keys any of its queries sees, and the
    sum over its queries of visible keys (for flops). Query i of a request
    with q queries and L keys sits at p = L - q + i and sees [lo, hi]:
    lo = p - W + 1 (W > 0) or 0; hi = p (causal), p + W - 1 (non-causal with
    a window) or L - 1, clipped to [0, L - 1]."""
    union, pairs = [], 0
    for q, L in zip(q_lens, seq_lens):
        first_lo, last_hi = L, -1
        for i in range(q):
            p = L - q + i
            lo = max(0, p - window + 1) if window > 0 else 0
            hi = p if causal else (min(L - 1, p + window - 1) if window > 0 else L - 1)
            first_lo, last_hi = min(first_lo, lo), max(last_hi, hi)
            pairs += hi - lo + 1
        union.append(max(0, last_hi - first_lo + 1))
    return union, pairs


def algorithmic(q_lens, seq_lens, Hq, Hkv, window, block_size=16, D=128, causal=True):
    """Bytes and flops one layer-call must move / do (reference crediting:
    Hkv (2D + 8) per visible key of each request, plus q, out and metadata;
    4 D Hq per visible query-key pair)."""
    union, pairs = visible_keys(q_lens, seq_lens, window, causal)
    T = sum(q_lens)
    kv = sum(union) * Hkv * (2 * D + 8)
    q_out = 2 * T * Hq * D * 2
    meta = sum(math.ceil(L / block_size) for L in seq_lens) * 4 + 4 * len(seq_lens) + 4 * (len(seq_lens) + 1)
    return kv + q_out + meta, kv + q_out // 2 + meta, 4 * D * Hq * pairs


def cpu_baseline(cache, q, qsl, q_lens, seq_lens, Hq, Hkv, window, threads,
                 budget_s: float = 4.0) -> dict:
    """Time the CPU oracle on a bounded sample of the workload (about
    budget_s of CPU work): whole requests from the first on, or for a batch
    whose first request is a long prefill chunk, its first query tokens.
    The rate is in the workload's unit: GB/s of credited bytes, or TFLOP/s
    of credited flops for a batch with prefill chunks."""
    import torch

    import oracle
    from pth_flash_attn import capi

    host = cache.to("cpu")
    qh, qslh = q.cpu(), qsl.cpu()
    out = torch.empty(qh.shape, dtype=torch.float32)
    args = capi.attn_args(q=qh, out=out, k_cache=host.k_cache, v_cache=host.v_cache,
                          k_scale=host.k_scale, v_scale=host.v_scale,
                          block_table=host.block_table, seq_lens=host.seq_lens,
                          query_start_loc=qslh, bq=1, num_splits=1,
                          softmax_scale=1.0 / math.sqrt(128), window=window)
    prefill = max(q_lens) > 64
    total_bytes, _, total_flops = algorithmic(q_lens, seq_lens, Hq, Hkv, window)
    if prefill:
        # Query tokens [0, n) of the first request (a prefill chunk).
        n, elapsed = 16, 0.0
        while True:
            n = min(n, q_lens[0])
            t0 = time.perf_counter()
            oracle.attention(args, threads=threads, rows=(0, n))
            elapsed = time.perf_counter() - t0
            if elapsed > budget_s or n == q_lens[0]:
                break
            n = max(n * 2, int(n * 2.0 * budget_s / max(elapsed, 1e-3)))
        L, ql = seq_lens[0], q_lens[0]
        pairs = sum(min(L - ql + i, L - 1) + 1 for i in range(n))  # causal, no window
        flops = 4 * 128 * Hq * pairs
        return {"value": round(flops / elapsed / 1e12, 4), "unit": "TFLOP/s", "cores": threads,
                "host_cpus": os.cpu_count(), "kind": "port",
                "sample": f"query tokens [0, {n}) of the first 2048-token prefill chunk, "
                          f"{elapsed:.2f} s, fp64 oracle/oracle.c",
                "us_per_layer_call_extrapolated": round(elapsed * 1e6 * total_flops / flops, 1)}
    starts = [0]
    for ql in q_lens:
        starts.append(starts[-1] + ql)
    n, elapsed, done = 1, 0.0, 0
    while True:
        n_req = min(n, len(q_lens))
        t0 = time.perf_counter()
        oracle.attention(args, threads=threads, rows=(0, starts[n_req]))
        elapsed = time.perf_counter() - t0
        done = n_req
        if elapsed > budget_s or n_req == len(q_lens):
            break
        n = max(n * 2, int(n * 2.0 * budget_s / max(elapsed, 1e-3)))
    byts, _, _ = algorithmic(q_lens[:done], seq_lens[:done], Hq, Hkv, window)
    return {"value": round(byts / elapsed / 1e9, 3), "unit": "GB/s", "cores": threads,
            "host_cpus": os.cpu_count(), "kind": "port",
            "sample": f"first {done} of {len(q_lens)} requests ({sum(q_lens[:done])} query tokens), "
                      f"{elapsed:.2f} s, fp64 oracle/oracle.c",
            "us_per_layer_call_extrapolated": round(elapsed * 1e6 * total_bytes / byts, 1)}


def profile_traffic(kernel_prefix: str, workload_name: str):
    """HBM bytes per launch of the attention kernel from committed rocprofv3
    counter summaries (profiles/*traffic*.json), or None."""
    f = REPO / "profiles" / f"traffic_{workload_name}.json"
    if not f.is_file():
        return None
    try:
        d = json.loads(f.read_text())
        return d.get(kernel_prefix)
    except (OSError, ValueError):
        return None


def bench_lib():
    """bench_hip/libpth_bench.so (the measured ceilings), loaded with ctypes."""
    import ctypes

    path = REPO / "bench_hip" / "libpth_bench.so"
    if not path.is_file():
        raise SystemExit(f"{path} is not built (python bench_hip/build.py)")
    lib = ctypes.CDLL(str(path))
    f32, i32, i64, vp = ctypes.c_float, ctypes.c_int32, ctypes.c_int64, ctypes.c_void_p
    lib.pth_bench_read_groups.restype = f32
    lib.pth_bench_read_groups.argtypes = [vp, i64, i32, i32, vp, i32, i32, vp, i32, vp]
    lib.pth_bench_mfma.restype = f32
    lib.pth_bench_mfma.argtypes = [i32, i32, vp, i32, vp]
    return lib


def read_ceiling(cache, seq_lens, cus: int, reps: int = 10) -> dict:
    """The headline's exact cache bytes (every cached token's slot row of 8
    cells), read with the attention kernel's load pattern and discarded."""
    import torch

    groups = []
    bt = cache.block_table.cpu()
    for r, L in enumerate(seq_lens):
        for blk in range((L + 15) // 16):
            groups.append((int(bt[r, blk]), min(16, L - 16 * blk)))
    g = torch.tensor(groups, dtype=torch.int32, device="cuda:0")
    sink = torch.zeros(1, dtype=torch.int32, device="cuda:0")
    row = cache.Hkv * (2 * cache.D + 8)
    stream = torch.cuda.current_stream()
    ms = bench_lib().pth_bench_read_groups(cache.k_cache.data_ptr(), cache.k_cache.stride(0), 0, row,
                                           g.data_ptr(), len(groups), cus, sink.data_ptr(), reps,
                                           stream.cuda_stream)
    if ms <= 0:
        raise RuntimeError(f"read ceiling failed ({ms})")
    byts = sum(n for _, n in groups) * row
    gbs = byts / (ms * 1e-3) / 1e9
    return {"value": round(gbs, 1), "unit": "GB/s", "frac_of_peak": round(gbs / PEAK_HBM_GBS, 4),
            "bytes": byts, "us": round(ms * 1e3, 2),
            "what": "bench_hip/ceilings.hip read_groups: config 2's cache bytes, whole slot rows "
                    "in 16-byte non-temporal register loads, two 16-key groups in flight per work-group, "
                    f"one work-group per CU, mean of {reps} launches"}


def mfma_ceiling(cus: int, iters: int = 20000, reps: int = 5) -> dict:
    """Dense bf16 MFMA rate (v_mfma_f32_16x16x32_bf16) at 8 waves per CU."""
    import torch

    sink = torch.zeros(1, device="cuda:0")
    ms = bench_lib().pth_bench_mfma(cus, iters, sink.data_ptr(), reps,
                                    torch.cuda.current_stream().cuda_stream)
    if ms <= 0:
        raise RuntimeError(f"mfma ceiling failed ({ms})")
    flops = cus * 8 * iters * 8 * 16 * 16 * 32 * 2
    tf = flops / (ms * 1e-3) / 1e12
    return {"value": round(tf, 1), "unit": "TFLOP/s", "frac_of_peak": round(tf / PEAK_BF16_TFLOPS, 4),
            "what": "bench_hip/ceilings.hip mfma_loop: v_mfma_f32_16x16x32_bf16, 8 waves per CU, "
                    "8 independent accumulators per wave"}


# The reference's published kernel rows closest to this path (its
# docs/benchmarks.md:157-166, 190, 194; RTX 3080 20 GB at 220 W), each as
# (q_lens, seq_lens, Hq, Hkv, D, block_size, window, causal, published us).
# They are latency or small-bandwidth shapes on other hardware: context for a
# user switching over, not the BASELINE metric.
REFERENCE_ROWS = {
    "drafter-16q4kv": ([8], [2056], 16, 4, 128, 864, 2048, False, 16.74),
    "drafter-32q8kv": ([8], [2056], 32, 8, 128, 864, 2048, False, 24.16),
    "drafter-16q4kv-L131080": ([8], [131080], 16, 4, 128, 864, 2048, False, 16.74),
    "d256-decode-12q2kv-L128k": ([1], [131072], 12, 2, 256, 16, 0, True, 209.8),
    "d256-verify4-12q2kv-L128k": ([4], [131072], 12, 2, 256, 16, 0, True, 247.2),
}


def reference_row(name: str, steps: int, warmup: int) -> dict:
    """One of the reference's published rows through the op, steady state
    (HIP events over `steps` layer calls after `warmup`)."""
    import torch

    from pth_flash_attn import ops, planner
    from pth_flash_attn.cache import build_cache, make_queries

    q_lens, seq_lens, Hq, Hkv, D, BS, window, causal, published = REFERENCE_ROWS[name]
    dev = "cuda:0"
    cache = build_cache(seq_lens, Hkv=Hkv, D=D, block_size=BS, seed=11, device=dev)
    q, qsl = make_queries(q_lens, Hq=Hq, D=D, seed=12, device=dev)
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    q_max = max(q_lens)
    ws_ts = planner.workspace_token_splits(max_num_seqs=len(q_lens), q_dec_max=q_max, Hkv=Hkv,
                                           D=D, num_sms=cus)
    plan = planner.plan_launch(num_tokens=len(q), num_reqs=len(q_lens), max_query_len=q_max,
                               G=Hq // Hkv, Hkv=Hkv, D=D, num_sms=cus, is_prefill=False,
                               ws_token_splits=max(ws_ts, len(q)), window=window)
    S = plan.num_splits
    out = torch.empty_like(q)
    ws_o = torch.empty(plan.ws_o_shape if S > 1 else (0,), device=dev)
    ws_lse = torch.empty(plan.ws_lse_shape if S > 1 else (0,), device=dev)

    def step():
        ops.pth_flash_attn_fwd(out, q, cache.k_cache, cache.v_cache, cache.k_scale,
                               cache.v_scale, cache.block_table, cache.seq_lens, qsl, q_max,
                               plan.wm, S, 1.0 / math.sqrt(D), ws_o, ws_lse, window, causal)

    for _ in range(max(warmup, 200)):
        step()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        step()
    e1.record()
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) / steps * 1e3
    # The same layer calls replayed from a captured graph (the reference times
    # graph-replayed launches): no host launch work between the calls.
    per_graph = 20
    graph = torch.cuda.CUDAGraph()
    cap = torch.cuda.Stream()
    cap.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(cap):
        step()
        cap.synchronize()
        with torch.cuda.graph(graph, stream=cap):
            for _ in range(per_graph):
                step()
    torch.cuda.current_stream().wait_stream(cap)
    for _ in range(5):
        graph.replay()
    torch.cuda.synchronize()
    reps = max(steps // per_graph, 10)
    e0.record()
    for _ in range(reps):
        graph.replay()
    e1.record()
    torch.cuda.synchronize()
    us_graph = e0.elapsed_time(e1) / (reps * per_graph) * 1e3
    byts, _, _ = algorithmic(q_lens, seq_lens, Hq, Hkv, window, block_size=BS, D=D,
                             causal=causal)
    return {"metric": "us/layer-call, reference published row (warm)", "row": name,
            "value": round(us, 2), "unit": "us", "higher_is_better": False, "steps": steps,
            "us_graph_replay": round(us_graph, 2),
            "reference_published_us": published, "reference_hardware": "RTX 3080 20 GB, 220 W",
            "ratio_reference_over_ours": round(published / us, 2),
            "ratio_reference_over_ours_graph": round(published / us_graph, 2),
            "gbs": round(byts / us / 1e3, 1),
            "config": {"q_lens": q_lens, "seq_lens": seq_lens, "Hq": Hq, "Hkv": Hkv, "D": D,
                       "block_size": BS, "window": window, "causal": causal,
                       "plan": {"wm": plan.wm, "num_splits": S}}}


ROTATE_BYTES = 1 << 30  # inputs smaller than this are rotated over copies


def _input_copies(cache, q, qsl, n: int) -> list:
    """n more sets of the same inputs, carved from one allocation per tensor
    (one copy kernel each, however many sets)."""
    import dataclasses

    from pth_flash_attn.cache import carve_views

    if n <= 0:
        return []
    store = cache.storage.unsqueeze(0).repeat(n, 1)
    bts = cache.block_table.unsqueeze(0).repeat(n, 1, 1)
    sls = cache.seq_lens.unsqueeze(0).repeat(n, 1)
    qs = q.unsqueeze(0).repeat(n, 1, 1, 1)
    qsls = qsl.unsqueeze(0).repeat(n, 1)
    sets = []
    for i in range(n):
        k, v, ks, vs = carve_views(store[i], num_blocks=cache.num_blocks,
                                   block_size=cache.block_size, Hkv=cache.Hkv, D=cache.D,
                                   layout=cache.layout, pad_page_bytes=cache.pad_page_bytes,
                                   offset_bytes=cache.offset_bytes)
        c = dataclasses.replace(cache, storage=store[i], k_cache=k, v_cache=v, k_scale=ks,
                                v_scale=vs, block_table=bts[i], seq_lens=sls[i])
        sets.append((c, qs[i], qsls[i]))
    return sets


def _events_ms(stream, n, fn) -> float:
    """Mean ms of n calls of fn() on `stream` (HIP events, synchronised)."""
    import torch

    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record(stream)
    for i in range(n):
        fn(i)
    e1.record(stream)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / n


def measure_config(config: int, query_tokens: int, steps: int, warmup: int, cpu_threads: int,
                   cus: int, graph: bool = True, keep_inputs: bool = False) -> dict:
    """One BASELINE configuration through the op: see the module docstring."""
    import statistics

    import torch

    from pth_flash_attn import capi, ops, planner
    from pth_flash_attn.cache import build_cache, make_queries

    dev = "cuda:0"
    name, q_lens, seq_lens, Hq, Hkv, window, is_prefill = workload(config, query_tokens)
    G, D, BS = Hq // Hkv, 128, 16
    cache = build_cache(seq_lens, Hkv=Hkv, D=D, block_size=BS, seed=config, device=dev)
    q, qsl = make_queries(q_lens, Hq=Hq, D=D, seed=config + 100, device=dev)
    T, R, q_max = len(q), len(q_lens), max(q_lens)
    ws_ts = planner.workspace_token_splits(max_num_seqs=R, q_dec_max=q_max if not is_prefill else 1,
                                           Hkv=Hkv, D=D, num_sms=cus)
    plan = planner.plan_launch(num_tokens=T, num_reqs=R, max_query_len=q_max, G=G, Hkv=Hkv, D=D,
                               num_sms=cus, is_prefill=is_prefill, ws_token_splits=max(ws_ts, T),
                               window=window)
    S = plan.num_splits
    out = torch.empty_like(q)
    ws_o = torch.empty(plan.ws_o_shape if S > 1 else (0,), device=dev)
    ws_lse = torch.empty(plan.ws_lse_shape if S > 1 else (0,), device=dev)
    scale = 1.0 / math.sqrt(D)
    in_bytes = cache.storage.numel() + q.numel() * q.element_size()
    copies = 1 if in_bytes >= ROTATE_BYTES else -(-ROTATE_BYTES // in_bytes) + 1
    sets = [(cache, q, qsl)] + _input_copies(cache, q, qsl, copies - 1)

    def step(i):
        c, qq, ql = sets[i % copies]
        ops.pth_flash_attn_fwd(out, qq, c.k_cache, c.v_cache, c.k_scale, c.v_scale,
                               c.block_table, c.seq_lens, ql, q_max, plan.wm, S, scale,
                               ws_o, ws_lse, window, True)

    stream = torch.cuda.current_stream()
    # Untimed warm-up: W steps, continued until they add up to WARMUP_MIN_S of
    # GPU work (the clocks and the TLBs settle; about 4 % slower on config 2
    # after 4 ms).
    warm_t0 = time.perf_counter()
    warm = 0
    while warm < warmup or time.perf_counter() - warm_t0 < WARMUP_MIN_S:
        step(warm)
        warm += 1
        if warm % 10 == 0:
            torch.cuda.synchronize()
    # Exactly `steps` layer calls, synchronised on both sides.
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ms = _events_ms(stream, steps, step)
    wall = time.perf_counter() - t0

    # The two kernels of the layer call alone, through the C ABI exactly as the
    # op launches them, on the same stream: KERNEL_BLOCKS blocks of K
    # back-to-back launches of each, interleaved with blocks of K op layer
    # calls, and the median block of each. The GPU sometimes runs a whole
    # block of launches in a slower state (the same kernel 10-20 % slower for
    # tens of launches, seen in rocprofv3 traces of identical launches), so
    # a single block of one kind against a single block of another compares
    # states, not kernels; interleaved medians compare the kernels.
    lib = capi.AttnLib()
    bq = 16 * plan.wm // G
    if 1 <= q_max < bq and planner.wm_for_rows(q_max * G) == plan.wm:
        bq = q_max
    arg_sets = [capi.attn_args(q=qq, out=out, k_cache=c.k_cache, v_cache=c.v_cache,
                               k_scale=c.k_scale, v_scale=c.v_scale, block_table=c.block_table,
                               seq_lens=c.seq_lens, query_start_loc=ql, bq=bq, num_splits=S,
                               softmax_scale=scale, ws_o=ws_o, ws_lse=ws_lse, window=window)
                for c, qq, ql in sets]
    sp = stream.cuda_stream
    blocks = {"layer": [], "attention": [], "combine": []}
    for _ in range(KERNEL_BLOCKS):
        blocks["layer"].append(_events_ms(stream, steps, step))
        blocks["attention"].append(_events_ms(
            stream, steps, lambda i: lib.check(lib.attention_kernel(arg_sets[i % copies], sp))))
        if S > 1:
            blocks["combine"].append(_events_ms(
                stream, steps, lambda i: lib.check(lib.combine_kernel(arg_sets[i % copies], sp))))
    attn_ms = statistics.median(blocks["attention"])
    comb_ms = statistics.median(blocks["combine"]) if S > 1 else None
    layer_blocks_ms = statistics.median(blocks["layer"])

    # The same layer calls replayed from a captured graph (the reference times
    # graph-replayed launches): the median over GRAPH_REPLAYS replays of 20 calls each
    # (at least 200 launches).
    graph_us = None
    if graph:
        per_graph = 20
        g = torch.cuda.CUDAGraph()
        cap = torch.cuda.Stream()
        cap.wait_stream(stream)
        with torch.cuda.stream(cap):
            step(0)
            cap.synchronize()
            with torch.cuda.graph(g, stream=cap):
                for i in range(per_graph):
                    step(i)
        stream.wait_stream(cap)
        for _ in range(3):
            g.replay()
        torch.cuda.synchronize()
        reps = []
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        for _ in range(GRAPH_REPLAYS):
            e0.record(stream)
            g.replay()
            e1.record(stream)
            e1.synchronize()
            reps.append(e0.elapsed_time(e1) / per_graph)
        graph_us = statistics.median(reps) * 1e3
        del g

    byts, attn_bytes, flops = algorithmic(q_lens, seq_lens, Hq, Hkv, window)
    res = {
        "workload": name, "config": config, "query_tokens_per_request": q_max if config == 3 else None,
        "num_seqs": R, "query_tokens": T, "context_tokens": sum(seq_lens), "window": window,
        "plan": {"wm": plan.wm, "num_splits": S},
        "us_per_layer_call": round(ms * 1e3, 2),
        "us_per_layer_call_graph_median": None if graph_us is None else round(graph_us, 2),
        "us_per_layer_call_block_median": round(layer_blocks_ms * 1e3, 2),
        "kernels_us": {"attention": round(attn_ms * 1e3, 2),
                       "combine": None if comb_ms is None else round(comb_ms * 1e3, 2)},
        "algorithmic_bytes": byts, "flops": flops,
        "gbs": round(byts / (ms * 1e-3) / 1e9, 1),
        "cold": {"input_copies": copies, "input_bytes": in_bytes,
                 "note": ("inputs rotated over copies: >= 1 GiB between reuses" if copies > 1
                          else "inputs exceed 1 GiB: read once per call")},
        "steps": steps, "warmup_steps_run": warm, "wall_s": round(wall, 3),
    }
    if S == 1:
        res["kernels_note"] = ("one launch per layer call (num_splits 1): kernels_us.attention and "
                               "the layer call time the same kernel (interleaved-block medians against "
                               "one timed loop); their difference is run-to-run noise")
    if is_prefill:
        tf = flops / (attn_ms * 1e-3) / 1e12
        res["roofline"] = {"bound": "mfma", "achieved": round(tf, 1), "peak": PEAK_BF16_TFLOPS,
                           "unit": "TFLOP/s", "frac": round(tf / PEAK_BF16_TFLOPS, 4)}
        res["tflops"] = round(flops / (ms * 1e-3) / 1e12, 1)
    else:
        gbs = attn_bytes / (attn_ms * 1e-3) / 1e9
        res["roofline"] = {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS,
                           "unit": "GB/s", "frac": round(gbs / PEAK_HBM_GBS, 4),
                           "algorithmic_bytes": attn_bytes,
                           "traffic": profile_traffic("attn_fwd_d128", name)}
    res["pct_of_peak_hbm"] = round(100.0 * res["gbs"] / PEAK_HBM_GBS, 2)
    if graph_us is not None:
        # The whole layer call (attention + combine) at its graph-replayed median.
        if is_prefill:
            res["roofline"]["frac_layer_call_graph_median"] = round(
                flops / (graph_us * 1e-6) / 1e12 / PEAK_BF16_TFLOPS, 4)
        else:
            res["roofline"]["frac_layer_call_graph_median"] = round(
                byts / (graph_us * 1e-6) / 1e9 / PEAK_HBM_GBS, 4)
    if cpu_threads > 0:
        res["cpu_baseline"] = cpu_baseline(cache, q, qsl, q_lens, seq_lens, Hq, Hkv, window,
                                           cpu_threads)
    if keep_inputs:
        res["_inputs"] = (cache, seq_lens)
    del sets, arg_sets, out, ws_o, ws_lse
    return res


# The five BASELINE configurations, config 3 at both query counts.
ALL_CONFIGS = ((1, 1), (2, 1), (3, 1), (3, 4), (4, 1), (5, 1))


def xcd_spread(steps: int, warmup: int, cus: int, config: int = 2, query_tokens: int = 1) -> dict:
    """Start and finishing times of the page-row attention kernel by XCD on a
    configuration it runs (2 or 3): the kernel as bench_hip/build.py builds it
    with PA_WAVE_CLOCK (each wave records its XCD and its start and end time,
    s_memrealtime at 100 MHz), launched through the C ABI after three
    back-to-back layer calls (attention, then combine); per launch, every time relative to
    the launch's first wave start; reported as medians over `steps`
    launches. Records left by waves of earlier launches (slots beyond this
    grid) are those that started more than 30 µs before the last start."""
    import ctypes
    import statistics

    import numpy as np
    import torch

    from pth_flash_attn import capi, planner
    from pth_flash_attn.cache import build_cache, make_queries

    lib = capi.AttnLib(REPO / "bench_hip" / "libpth_attn_clock.so")
    read = lib.lib.pth_attn_debug_wave_clock
    read.restype = ctypes.c_int32
    read.argtypes = [ctypes.c_void_p, ctypes.c_int64]
    name, q_lens, seq_lens, Hq, Hkv, window, is_prefill = workload(config, query_tokens)
    G, D = Hq // Hkv, 128
    cache = build_cache(seq_lens, Hkv=Hkv, D=D, block_size=16, seed=config, device="cuda:0")
    q, qsl = make_queries(q_lens, Hq=Hq, D=D, seed=config + 100, device="cuda:0")
    T, R, q_max = len(q), len(q_lens), max(q_lens)
    ws_ts = planner.workspace_token_splits(max_num_seqs=R, q_dec_max=q_max, Hkv=Hkv, D=D, num_sms=cus)
    plan = planner.plan_launch(num_tokens=T, num_reqs=R, max_query_len=q_max, G=G, Hkv=Hkv, D=D,
                               num_sms=cus, is_prefill=is_prefill, ws_token_splits=max(ws_ts, T),
                               window=window)
    S = plan.num_splits
    # The op's row-tile height (csrc/torch_op.cpp tile_tokens).
    cap = 16 * plan.wm // G
    bq = q_max if 1 <= q_max < cap and planner.wm_for_rows(q_max * G) == plan.wm else cap
    out = torch.empty_like(q)
    ws_o = torch.empty(plan.ws_o_shape, device="cuda:0")
    ws_lse = torch.empty(plan.ws_lse_shape, device="cuda:0")
    args = capi.attn_args(q=q, out=out, k_cache=cache.k_cache, v_cache=cache.v_cache,
                          k_scale=cache.k_scale, v_scale=cache.v_scale,
                          block_table=cache.block_table, seq_lens=cache.seq_lens,
                          query_start_loc=qsl, bq=bq, num_splits=S,
                          softmax_scale=1.0 / math.sqrt(D), ws_o=ws_o, ws_lse=ws_lse,
                          window=window)
    sp = torch.cuda.current_stream().cuda_stream
    waves = 8192
    buf = np.zeros(waves * 3, dtype=np.uint64)
    for _ in range(max(warmup, 10)):
        lib.check(lib.attention_kernel(args, sp))
    torch.cuda.synchronize()
    per_xcd_mean, per_xcd_p10, per_xcd_p90, per_xcd_start, last = {}, {}, {}, {}, []
    overall = {k: [] for k in ("start_p50", "start_p90", "start_max", "end_p10", "end_p50", "end_p90")}
    counted = []
    for _ in range(steps):
        # Three layer calls back to back before the recorded launch: its
        # work-groups then start as the previous call's combine drains, as
        # in the timed loops (after an idle gap, the XCDs' first work-groups
        # start up to 4 us apart; back to back, within 0.4 us).
        for _r in range(3):
            lib.check(lib.attention_kernel(args, sp))
            if S > 1:
                lib.check(lib.combine_kernel(args, sp))
        lib.check(lib.attention_kernel(args, sp))
        torch.cuda.synchronize()
        if read(buf.ctypes.data, waves) != 0:
            raise RuntimeError("pth_attn_debug_wave_clock failed")
        x = buf.reshape(waves, 3).astype(np.int64)
        x = x[x[:, 1] >= x[:, 1].max() - 3000]
        xcd, t0 = x[:, 0], x[:, 1].min()
        start = (x[:, 1] - t0) / 100.0  # µs
        end = (x[:, 2] - t0) / 100.0
        counted.append(len(x))
        last.append(float(end.max()))
        overall["start_p50"].append(float(np.percentile(start, 50)))
        overall["start_p90"].append(float(np.percentile(start, 90)))
        overall["start_max"].append(float(start.max()))
        for q_, k_ in ((10, "end_p10"), (50, "end_p50"), (90, "end_p90")):
            overall[k_].append(float(np.percentile(end, q_)))
        for k in np.unique(xcd):
            e = end[xcd == k]
            per_xcd_mean.setdefault(int(k), []).append(float(e.mean()))
            per_xcd_start.setdefault(int(k), []).append(float(np.median(start[xcd == k])))
            per_xcd_p10.setdefault(int(k), []).append(float(np.percentile(e, 10)))
            per_xcd_p90.setdefault(int(k), []).append(float(np.percentile(e, 90)))
    med = statistics.median
    return {
        "workload": name, "kernel": "attn_fwd_pagerows", "launches": steps,
        "waves": int(med(counted)), "num_splits": S,
        "last_wave_end_us": round(med(last), 1),
        "all_waves_us": {k: round(med(v), 1) for k, v in overall.items()},
        "by_xcd": {k: {"start_p50_us": round(med(per_xcd_start[k]), 2),
                       "mean_end_us": round(med(v), 1),
                       "p10_end_us": round(med(per_xcd_p10[k]), 1),
                       "p90_end_us": round(med(per_xcd_p90[k]), 1)}
                   for k, v in sorted(per_xcd_mean.items())},
    }


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--config", type=int, default=2,
                    help="the headline configuration (default 2, BASELINE's metric)")
    ap.add_argument("--query-tokens", type=int, default=1,
                    help="config 3 only: 1 (decode) or 4 (MTP verify)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baselines")
    ap.add_argument("--only-headline", action="store_true",
                    help="measure the headline configuration only (no configs array, no ceilings)")
    ap.add_argument("--cpu-threads", type=int, default=0)
    ap.add_argument("--reference-row", choices=sorted(REFERENCE_ROWS),
                    help="time one of the reference's published rows instead of a config")
    ap.add_argument("--xcd-spread", action="store_true",
                    help="only report the page-row kernel's start and finishing times by XCD "
                         "on --config (2 or 3) "
                         "(needs bench_hip/libpth_attn_clock.so, built by bench_hip/build.py)")
    ap.add_argument("--copy-probe-mib", type=int, default=0,
                    help="only run a plain device copy of this many MiB, --steps times "
                         "(the reference point that scales rocprofv3 FETCH_SIZE/WRITE_SIZE)")
    a = ap.parse_args()
    if a.gpus != 1:
        print("bench.py measures one GPU: this path runs on one device (the op has no "
              "multi-GPU form; a multi-GPU deployment shards the KV heads or the requests "
              "and runs one launch per GPU on its shard). "
              "Run with --gpus 1.", file=sys.stderr)
        return 2

    import torch

    if a.copy_probe_mib:
        src = torch.empty(a.copy_probe_mib << 20, dtype=torch.uint8, device="cuda:0")
        dst = torch.empty_like(src)
        for _ in range(a.steps):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_probe_bytes": src.numel(), "launches": a.steps}))
        return 0

    from pth_flash_attn import ops

    if not ops.is_available():
        raise SystemExit("pth_flash_attn op library is not built (python pth-flash-attn_amd/build.py)")
    torch.cuda.set_device(0)
    if a.reference_row:
        print(json.dumps(reference_row(a.reference_row, a.steps * 4, a.warmup)))
        return 0
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    if a.xcd_spread:
        print(json.dumps(xcd_spread(a.steps, a.warmup, cus, a.config, a.query_tokens)))
        return 0
    threads = 0 if a.no_cpu else (a.cpu_threads or min(16, os.cpu_count() or 1))
    t_start = time.perf_counter()
    head = measure_config(a.config, a.query_tokens, a.steps, a.warmup, threads, cus,
                          keep_inputs=True)
    cache, seq_lens = head.pop("_inputs")
    result = {
        "metric": METRIC,
        "value": head["gbs"],
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "warmup_steps_run": head["warmup_steps_run"],
        "ms_per_step": round(head["us_per_layer_call"] / 1e3, 5),
        "us_per_layer_call": head["us_per_layer_call"],
        "us_per_layer_call_graph_median": head["us_per_layer_call_graph_median"],
        "pct_of_peak_hbm": head["pct_of_peak_hbm"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8 KV / bf16 q,out / fp32 accumulate",
        "data": "synthetic (seeded N(0,1) K/V quantised by the vLLM int8 writer rule, bf16 q)",
        "config": {"workload": head["workload"], "num_seqs": head["num_seqs"],
                   "query_tokens": head["query_tokens"], "Hq": 32 if a.config != 1 else 4,
                   "Hkv": 8 if a.config != 1 else 1, "D": 128, "block_size": 16,
                   "context_tokens": head["context_tokens"], "window": head["window"],
                   "plan": head["plan"], "parallelism": "single GPU"},
        "kernels_us": head["kernels_us"],
        "roofline": head["roofline"],
    }
    if "cpu_baseline" in head:
        result["cpu_baseline"] = head["cpu_baseline"]
    if not a.only_headline:
        if result["roofline"]["bound"] == "hbm":
            rc = read_ceiling(cache, seq_lens, cus)
            result["read_ceiling"] = rc
            result["roofline"]["frac_of_read_ceiling"] = round(
                result["roofline"]["achieved"] / rc["value"], 4)
        del cache
        torch.cuda.empty_cache()
        mc = mfma_ceiling(cus)
        result["mfma_ceiling"] = mc
        configs = []
        for cfg, qt in ALL_CONFIGS:
            if (cfg, qt) == (a.config, a.query_tokens):
                entry = head
            else:
                steps = a.steps if cfg != 5 else max(5, a.steps // 5)
                entry = measure_config(cfg, qt, steps, a.warmup, threads, cus)
                torch.cuda.empty_cache()
            if entry["roofline"]["bound"] == "mfma":
                entry["roofline"]["frac_of_mfma_ceiling"] = round(
                    entry["roofline"]["achieved"] / mc["value"], 4)
            configs.append(entry)
        result["configs"] = configs
    result["wall_s"] = round(time.perf_counter() - t_start, 1)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
