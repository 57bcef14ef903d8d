"""bench.py on the CPU: the workloads are BASELINE.json's configurations, the
work it credits (bytes and flops) matches a brute-force count, and the
multi-GPU form is refused.

The crediting follows the reference's (bench/kernel_bench.py:313-324): bytes
= Hkv (2D + 8) per distinct key a request's queries see, plus q, out and the
metadata; flops = 4 D Hq per visible query-key pair.
"""

from __future__ import annotations

import math
import subprocess
import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(REPO))
import bench  # noqa: E402


def test_workloads_are_the_baseline_configs():
    name, q, L, Hq, Hkv, W, pf = bench.workload(1)
    assert (q, L, Hq, Hkv, W) == ([1], [1024], 4, 1, 0)
    name, q, L, Hq, Hkv, W, pf = bench.workload(2)
    assert q == [1] * 64 and (Hq, Hkv, W) == (32, 8, 0) and not pf
    assert len(L) == 64 and all(1024 <= x <= 32768 for x in L)
    name, q, L, Hq, Hkv, W, pf = bench.workload(3)
    assert (q, L, Hq, Hkv) == ([1], [131072], 32, 8)
    name, q, L, Hq, Hkv, W, pf = bench.workload(3, 4)
    assert (q, L, Hq, Hkv) == ([4], [131072], 32, 8) and "verify4" in name
    name, q, L, Hq, Hkv, W, pf = bench.workload(4)
    assert q == [16] * 8 and W == 2048 and all(8192 <= x <= 65536 for x in L)
    name, q, L, Hq, Hkv, W, pf = bench.workload(5)
    assert q == [2048] * 4 + [1] * 60 and pf
    assert all(2048 <= x <= 30 * 1024 + 2048 for x in L[:4])
    assert all(2048 <= x <= 65536 for x in L[4:])


def _brute(q_lens, seq_lens, Hq, Hkv, window, D=128, block_size=16, causal=True):
    """Count visible keys one query at a time (bottom-right causal, or the
    non-causal window [p - W + 1, p + W - 1] / every key)."""
    keys_seen, pairs = 0, 0
    for q, L in zip(q_lens, seq_lens):
        seen = set()
        for i in range(q):
            p = L - q + i
            vis = [k for k in range(L)
                   if (window == 0 or k > p - window)
                   and (k <= p if causal else (window == 0 or k < p + window))]
            pairs += len(vis)
            seen.update(vis)
        keys_seen += len(seen)
    T = sum(q_lens)
    kv = keys_seen * Hkv * (2 * D + 8)
    meta = (sum(math.ceil(L / block_size) for L in seq_lens) * 4 + 4 * len(seq_lens)
            + 4 * (len(seq_lens) + 1))
    total = kv + 2 * T * Hq * D * 2 + meta
    attn = kv + T * Hq * D * 2 + meta
    return total, attn, 4 * D * Hq * pairs


@pytest.mark.parametrize("q_lens,seq_lens,window", [
    ([1], [1024], 0),
    ([1, 1, 1], [17, 4096, 33], 0),
    ([4], [300], 0),
    ([16, 16], [3000, 40], 64),
    ([200, 3], [900, 5], 100),
])
def test_algorithmic_work_matches_a_brute_force_count(q_lens, seq_lens, window):
    got = bench.algorithmic(q_lens, seq_lens, 32, 8, window)
    assert got == _brute(q_lens, seq_lens, 32, 8, window)


@pytest.mark.parametrize("q_lens,seq_lens,window,D", [
    ([8], [2056], 2048, 128),   # the reference's drafter rows: non-causal, window 2048
    ([8], [300], 64, 128),
    ([3, 5], [40, 700], 0, 256),
])
def test_algorithmic_work_non_causal_and_d256(q_lens, seq_lens, window, D):
    got = bench.algorithmic(q_lens, seq_lens, 16, 4, window, D=D, causal=False)
    assert got == _brute(q_lens, seq_lens, 16, 4, window, D=D, causal=False)


def test_reference_rows_are_the_published_shapes():
    row = bench.REFERENCE_ROWS["d256-decode-12q2kv-L128k"]
    assert row[:6] == ([1], [131072], 12, 2, 256, 16) and row[-1] == 209.8
    row = bench.REFERENCE_ROWS["drafter-32q8kv"]
    assert row[:8] == ([8], [2056], 32, 8, 128, 864, 2048, False) and row[-1] == 24.16


def test_config2_bytes_closed_form():
    """Decode (q = 1): every key of every request, once per KV head."""
    _, q, L, Hq, Hkv, W, _ = bench.workload(2)
    total, attn, flops = bench.algorithmic(q, L, Hq, Hkv, W)
    kv = sum(L) * Hkv * 264
    assert attn - kv == 64 * Hq * 128 * 2 + sum(math.ceil(x / 16) for x in L) * 4 + 4 * 64 + 4 * 65
    assert flops == 4 * 128 * Hq * sum(L)


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, str(REPO / "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode != 0 and "--gpus 1" in r.stderr
