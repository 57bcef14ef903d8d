#!/usr/bin/env python3
"""Benchmark of the hot path: int8 paged decode attention, D = 128, on one MI355X.

Default workload ("config 2"): 64 decode sequences, 1 query
token each, 32 q / 8 KV heads, D = 128, context lengths uniform in [1k, 32k]
(seeded), vLLM block size 16 with a shuffled block table over one shared pool,
int8 K/V with inline fp32 per-token-head scales, bf16 queries ~ N(0, 1).
A step is one layer-call: the torch op pth_flash_attn_fwd (attention kernel +
split combine) with the planner's plan, inputs resident in HBM.

Printed (one JSON line on stdout): value = achieved HBM GB/s of the whole
layer-call (algorithmic bytes / time), ms_per_step (x1000 = us per
layer-call), and
  roofline     - the attention kernel alone: algorithmic bytes of one launch /
                 its average duration (HIP events on the launch stream), against
                 MI355X's 8 TB/s, with HBM traffic per launch from rocprofv3
                 counters when a profile summary is present (else null);
  cpu_baseline - the repository's CPU oracle (fp64 restatement of the
                 reference's CPU path) on a bounded sample of the same workload.

Warm-up: W untimed steps, continued until they add up to at least 0.3 s of
GPU work (the step count run is printed as warmup_steps_run).

Usage: python bench.py [--steps K] [--warmup W] [--config 1..5] [--query-tokens 1|4] [--no-cpu]
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


def cpu_baseline(cache, q, qsl, q_lens, seq_lens, Hq, Hkv, window, threads):
    """Time the CPU oracle on a bounded sample (about 10 s) of the workload."""
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
        if elapsed > 4.0 or n_req == len(q_lens):
            break
        n = max(n * 2, int(n * 8.0 / max(elapsed, 1e-3)))
    byts, _, flops = algorithmic(q_lens[:done], seq_lens[:done], Hq, Hkv, window)
    return {"value": round(byts / elapsed / 1e9, 3), "unit": "GB/s", "cores": threads,
            "kind": "port",
            "sample": f"first {done} of {len(q_lens)} requests ({sum(q_lens[:done])} query tokens), "
                      f"{elapsed:.2f} s, fp64 oracle/oracle.c",
            "us_per_layer_call_extrapolated": round(
                elapsed * 1e6 * algorithmic(q_lens, seq_lens, Hq, Hkv, window)[0] / byts, 1)}


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


def copy_ceiling(mib: int = 1024, reps: int = 10) -> dict:
    """Achievable streaming HBM throughput on this device, for context next to
    the nominal peak: a plain device copy of ``mib`` MiB (read + write bytes
    over its time, HIP events). Measured: ~6.1-6.2 TB/s also for pure reads
    of the paged cache, by any access pattern."""
    import torch
    src = torch.empty(mib << 20, dtype=torch.uint8, device="cuda:0")
    dst = torch.empty_like(src)
    dst.copy_(src)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        dst.copy_(src)
    e1.record()
    torch.cuda.synchronize()
    sec = e0.elapsed_time(e1) / reps * 1e-3
    gbs = 2 * src.numel() / sec / 1e9
    del src, dst
    return {"value": round(gbs, 1), "unit": "GB/s",
            "what": f"device copy of {mib} MiB, read + write bytes / time",
            "frac_of_peak": round(gbs / PEAK_HBM_GBS, 4)}


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


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--config", type=int, default=2)
    ap.add_argument("--query-tokens", type=int, default=1,
                    help="config 3 only: 1 (decode) or 4 (MTP verify)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--cpu-threads", type=int, default=0)
    ap.add_argument("--reference-row", choices=sorted(REFERENCE_ROWS),
                    help="time one of the reference's published rows instead of a config")
    ap.add_argument("--copy-probe-mib", type=int, default=0,
                    help="only run a plain device copy of this many MiB, --steps times "
                         "(the reference point that scales rocprofv3 FETCH_SIZE/WRITE_SIZE)")
    a = ap.parse_args()
    if a.gpus != 1:
        print("bench.py measures one GPU: this path runs on one device (the op has no "
              "multi-GPU form; sharding is by KV head or request, see DESIGN.md). "
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

    from pth_flash_attn import capi, ops, planner
    from pth_flash_attn.cache import build_cache, make_queries

    if a.reference_row:
        if not ops.is_available():
            raise SystemExit("pth_flash_attn op library is not built")
        torch.cuda.set_device(0)
        print(json.dumps(reference_row(a.reference_row, a.steps * 4, a.warmup)))
        return 0
    if not ops.is_available():
        raise SystemExit("pth_flash_attn op library is not built (python pth-flash-attn_amd/build.py)")
    dev = "cuda:0"
    torch.cuda.set_device(0)
    name, q_lens, seq_lens, Hq, Hkv, window, is_prefill = workload(a.config, a.query_tokens)
    G, D, BS = Hq // Hkv, 128, 16
    cache = build_cache(seq_lens, Hkv=Hkv, D=D, block_size=BS, seed=a.config, device=dev)
    q, qsl = make_queries(q_lens, Hq=Hq, D=D, seed=a.config + 100, device=dev)
    T, R, q_max = len(q), len(q_lens), max(q_lens)
    cus = torch.cuda.get_device_properties(0).multi_processor_count
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

    def step():
        ops.pth_flash_attn_fwd(out, q, cache.k_cache, cache.v_cache, cache.k_scale, cache.v_scale,
                               cache.block_table, cache.seq_lens, qsl, q_max, plan.wm, S, scale,
                               ws_o, ws_lse, window, True)

    stream = torch.cuda.current_stream()
    # Untimed warm-up: the W steps asked for, continued until they add up to
    # WARMUP_MIN_S of GPU work, so that the first timed steps do not run while
    # the clocks and the TLBs settle (about 4 % slower on config 2 after 4 ms).
    warm_t0 = time.perf_counter()
    warm_steps = 0
    while warm_steps < a.warmup or time.perf_counter() - warm_t0 < WARMUP_MIN_S:
        step()
        warm_steps += 1
        if warm_steps % 10 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(a.steps):
        step()
    e1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms = e0.elapsed_time(e1) / a.steps

    # The attention kernel alone (the dominant kernel), launched through the C
    # ABI exactly as the op launches it, on the same stream.
    lib = capi.AttnLib()
    bq = 16 * plan.wm // G
    if 1 <= q_max < bq and planner.wm_for_rows(q_max * G) == plan.wm:
        bq = q_max
    args = capi.attn_args(q=q, out=out, k_cache=cache.k_cache, v_cache=cache.v_cache,
                          k_scale=cache.k_scale, v_scale=cache.v_scale,
                          block_table=cache.block_table, seq_lens=cache.seq_lens,
                          query_start_loc=qsl, bq=bq, num_splits=S, softmax_scale=scale,
                          ws_o=ws_o, ws_lse=ws_lse, window=window)
    sp = stream.cuda_stream
    e0.record(stream)
    for _ in range(a.steps):
        lib.check(lib.attention_kernel(args, sp))
    e1.record(stream)
    torch.cuda.synchronize()
    attn_ms = e0.elapsed_time(e1) / a.steps
    # The split combine as the op launches it (it reads only the splits each
    # request used): the layer-call minus the attention kernel.
    comb_ms = max(ms - attn_ms, 0.0) if S > 1 else None

    byts, attn_bytes, flops = algorithmic(q_lens, seq_lens, Hq, Hkv, window)
    gbs = byts / (ms * 1e-3) / 1e9
    attn_gbs = attn_bytes / (attn_ms * 1e-3) / 1e9
    traffic = profile_traffic("attn_fwd_d128", name)
    result = {
        "metric": METRIC,
        "value": round(gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "warmup_steps_run": warm_steps,
        "ms_per_step": round(ms, 5),
        "us_per_layer_call": round(ms * 1e3, 2),
        "pct_of_peak_hbm": round(100.0 * gbs / PEAK_HBM_GBS, 2),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8 KV / bf16 q,out / fp32 accumulate",
        "data": "synthetic (seeded N(0,1) K/V quantised by the vLLM int8 writer rule, bf16 q)",
        "config": {"workload": name, "num_seqs": R, "query_tokens": T, "Hq": Hq, "Hkv": Hkv,
                   "D": D, "block_size": BS, "context_tokens": sum(seq_lens), "window": window,
                   "plan": {"wm": plan.wm, "num_splits": S}, "parallelism": "single GPU"},
        "kernels_us": {"attention": round(attn_ms * 1e3, 2),
                       "combine_and_launch_gaps": None if comb_ms is None else round(comb_ms * 1e3, 2)},
        "roofline": {"bound": "hbm", "achieved": round(attn_gbs, 1), "peak": PEAK_HBM_GBS,
                     "unit": "GB/s", "frac": round(attn_gbs / PEAK_HBM_GBS, 4),
                     "traffic": traffic, "algorithmic_bytes": attn_bytes},
        "wall_s": round(wall, 3),
    }
    result["roofline"]["copy_ceiling"] = copy_ceiling()
    if a.config == 5:
        result["mfma"] = {"flops": flops, "tflops_achieved": round(flops / (ms * 1e-3) / 1e12, 1),
                          "peak_tflops": PEAK_BF16_TFLOPS}
    if not a.no_cpu:
        threads = a.cpu_threads or min(16, os.cpu_count() or 1)
        result["cpu_baseline"] = cpu_baseline(cache, q, qsl, q_lens, seq_lens, Hq, Hkv, window, threads)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
