"""Planner tests (CPU only).

The formulas are the reference's (python/pth_flash_attn/planner.py:24-73);
only CTAS_PER_SM differs on MI355X. With the reference's own sm_86 constants
patched in, the plans must equal the reference's published known answers:
docs/api.md:170-197 (68 SMs, Hkv=2, G=6, D=256), the production decode table
tests/cpu/test_planner.py:227-260 and the drafter plans
tests/cpu/test_planner.py:813-858. Those numbers are the pin; the MI355X plans
that the GPU tests use are checked beside them.
"""

from __future__ import annotations

import ast
import dataclasses
import itertools
import math
import random
from pathlib import Path

import pytest

from pth_flash_attn import planner
from pth_flash_attn.planner import (
    LaunchPlan,
    max_tokens_per_tile,
    plan_launch,
    s_alone,
    split_tile_range,
    workspace_bytes,
    workspace_shapes,
    workspace_token_splits,
)

# The reference's sm_86 kernel-trait constants (reference planner.py:91).
SM86_CTAS_PER_SM = {64: 3, 128: 2, 256: 1}
PROD = {"G": 6, "Hkv": 2, "D": 256, "num_sms": 68}


@pytest.fixture
def sm86(monkeypatch):
    monkeypatch.setattr(planner, "CTAS_PER_SM", dict(SM86_CTAS_PER_SM))


def _ws(q_dec_max: int, max_num_seqs: int = 2, **geom: int) -> int:
    g = {**PROD, **geom}
    return workspace_token_splits(max_num_seqs=max_num_seqs, q_dec_max=q_dec_max,
                                  Hkv=g["Hkv"], D=g["D"], num_sms=g["num_sms"])


def _decode(q: int, reqs: int, ws: int, **geom) -> LaunchPlan:
    g = {**PROD, **geom}
    return plan_launch(num_tokens=q * reqs, num_reqs=reqs, max_query_len=q,
                       is_prefill=False, ws_token_splits=ws, **g)


def test_api_example_plans(sm86):
    """docs/api.md:170-197 printed values."""
    w_ts = _ws(4)
    assert s_alone(Hkv=2, D=256, num_sms=68) == 34
    assert w_ts == 272
    assert workspace_shapes(ws_token_splits=w_ts, Hq=12, D=256) == ((272, 12, 256), (272, 12))
    assert workspace_bytes(ws_token_splits=w_ts, Hq=12, D=256) / 2**20 == 3.199951171875
    p = plan_launch(num_tokens=4, num_reqs=1, max_query_len=4, is_prefill=False,
                    ws_token_splits=w_ts, **PROD)
    assert p == LaunchPlan(wm=2, bq=5, q_tiles_upper=1, num_splits=34, num_tokens=4,
                           G=6, Hkv=2, D=256, is_prefill=False)
    assert p.grid == (1, 2, 34)
    assert p.ws_o_shape == (34, 4, 12, 256) and p.ws_lse_shape == (34, 4, 12)
    p = plan_launch(num_tokens=2048, num_reqs=1, max_query_len=2048, is_prefill=True,
                    ws_token_splits=w_ts, **PROD)
    assert (p.wm, p.bq, p.num_splits, p.ws_o_shape) == (4, 10, 1, (0, 2048, 12, 256))


@pytest.mark.parametrize(("q", "ws_q", "wm", "bq", "rows", "splits"), [
    (1, 4, 1, 2, 12, 34),
    (4, 4, 2, 5, 30, 34),
    (10, 4, 4, 10, 60, 13),
    (10, 16, 4, 10, 60, 34),
    (16, 16, 4, 10, 60, 17),
    (16, 4, 4, 10, 60, 8),
])
def test_production_decode_plans(sm86, q, ws_q, wm, bq, rows, splits):
    """reference tests/cpu/test_planner.py:227-260."""
    p = _decode(q, 2, _ws(ws_q))
    assert (p.wm, p.bq, p.rows_per_cta, p.num_splits) == (wm, bq, rows, splits)
    assert p.grid == (p.num_tokens // bq + 2, 2, splits)


@pytest.mark.parametrize(("Hkv", "num_sms", "splits"), [
    (4, 68, 34), (4, 70, 34), (4, 82, 34), (8, 68, 17), (8, 70, 18), (8, 82, 21)])
def test_drafter_plans(sm86, Hkv, num_sms, splits):
    """reference tests/cpu/test_planner.py:813-858 (D=128, G=4, window 2048, q=8)."""
    geom = {"G": 4, "Hkv": Hkv, "D": 128, "num_sms": num_sms}
    ws = workspace_token_splits(max_num_seqs=2, q_dec_max=8, Hkv=Hkv, D=128, num_sms=num_sms)
    for reqs in (1, 2):
        desc = {"num_tokens": 8 * reqs, "num_reqs": reqs, "max_query_len": 8,
                "is_prefill": False, "ws_token_splits": ws, **geom}
        p = plan_launch(**desc, window=2048)
        assert (p.wm, p.bq, p.rows_per_cta) == (2, 8, 32)
        assert p.num_splits == splits
        assert p == dataclasses.replace(plan_launch(**desc), num_splits=splits)
        assert plan_launch(**desc, window=64).num_splits == 3


def test_rt_keeps_rows_within_one_tile():
    """bq * G <= 64 and rt = ceil(q / floor(64 / G)) for every decode shape
    (reference tests/cpu/test_planner.py:263-295); q = 21, G = 6 is the case
    where the naive ceil(q G / 64) rule overflows a tile."""
    p = _decode(21, 1, 0)
    assert (p.wm, p.bq, p.rows_per_cta) == (4, 10, 60)
    for g in range(1, 65):
        for q in range(1, 200):
            p = plan_launch(num_tokens=q, num_reqs=1, max_query_len=q, G=g, Hkv=1, D=128,
                            num_sms=256, is_prefill=False, ws_token_splits=0)
            assert p.rows_per_cta <= 16 * p.wm <= 64
            assert math.ceil(q / p.bq) == math.ceil(q / max_tokens_per_tile(g)), (g, q)
            if 64 % g == 0:
                assert math.ceil(q / p.bq) == math.ceil(q * g / 64)


def test_mi355x_plans_of_the_benchmark_configs():
    """The plans the MI355X benchmark configs run with (256 CUs, 8 waves/CU):
    C_target = 2048 units, so one decode request alone gets 2048 / Hkv splits."""
    assert planner.c_target(D=128, num_sms=256) == 2048
    geom = {"G": 4, "Hkv": 8, "D": 128, "num_sms": 256}
    # config 2: 64 decodes, workspace sized for them.
    ws = workspace_token_splits(max_num_seqs=64, q_dec_max=1, Hkv=8, D=128, num_sms=256)
    assert ws == 64 * 256
    p = plan_launch(num_tokens=64, num_reqs=64, max_query_len=1, is_prefill=False,
                    ws_token_splits=ws, **geom)
    assert (p.wm, p.bq, p.num_splits, p.q_tiles_upper) == (1, 4, 256, 80)
    # config 3: one request, q = 4 -> one 16-row tile.
    p = plan_launch(num_tokens=4, num_reqs=1, max_query_len=4, is_prefill=False,
                    ws_token_splits=ws, **geom)
    assert (p.wm, p.bq, p.num_splits) == (1, 4, 256)
    # config 4: window 2048, q = 16 causal -> 64 rows, cap ceil(2062 / 64) + 1 = 34.
    p = plan_launch(num_tokens=128, num_reqs=8, max_query_len=16, is_prefill=False,
                    ws_token_splits=ws, window=2048, **geom)
    assert (p.wm, p.bq, p.num_splits) == (4, 16, 34)


def test_window_cap_formula():
    for w in (1, 2, 63, 64, 65, 2048, 4095):
        for q in (1, 2, 8, 16):
            p = plan_launch(num_tokens=q, num_reqs=1, max_query_len=q, G=4, Hkv=1, D=128,
                            num_sms=256, is_prefill=False, ws_token_splits=10**9, window=w)
            assert p.num_splits == min(2048, math.ceil((w + q - 2) / 64) + 1)


def test_workspace_clamp():
    """S * T never exceeds the reserved token-splits."""
    rng = random.Random(3)
    for _ in range(500):
        q = rng.randint(1, 16)
        reqs = rng.randint(1, 8)
        ws = rng.randint(0, 4096)
        p = plan_launch(num_tokens=q * reqs, num_reqs=reqs, max_query_len=q, G=4, Hkv=8,
                        D=128, num_sms=256, is_prefill=False, ws_token_splits=ws)
        assert p.num_splits == 1 or p.num_splits * p.num_tokens <= ws


def test_plans_independent_of_lengths():
    """No parameter can carry a sequence length (graph replay safety)."""
    good = {"num_tokens": 8, "num_reqs": 2, "max_query_len": 4, "is_prefill": False}
    with pytest.raises(TypeError):
        plan_launch(**good, **PROD, ws_token_splits=272, seq_lens=[100, 200])
    with pytest.raises(TypeError):
        plan_launch(8, 2, 4, 6, 2, 256, 68, False, 272)


@pytest.mark.parametrize("bad", [
    {"num_tokens": 0}, {"num_tokens": True}, {"G": 65}, {"D": 96}, {"max_query_len": 9},
    {"is_prefill": 1}, {"window": -1}])
def test_invalid_descriptors_raise(bad):
    desc = {"num_tokens": 8, "num_reqs": 2, "max_query_len": 4, "G": 4, "Hkv": 8, "D": 128,
            "num_sms": 256, "is_prefill": False, "ws_token_splits": 0}
    desc.update(bad)
    with pytest.raises((TypeError, ValueError)):
        plan_launch(**desc)


def test_split_tile_ranges_partition_and_balance():
    """reference tests/cpu/test_planner.py:860-879."""
    for S in range(1, 70):
        for T in range(0, 300, 7):
            r = [split_tile_range(split=s, num_splits=S, num_tiles=T) for s in range(S)]
            assert r[0][0] == 0 and r[-1][1] == T
            assert all(a[1] == b[0] for a, b in itertools.pairwise(r))
            sizes = [e - b for b, e in r]
            assert min(sizes) >= 0 and max(sizes) - min(sizes) <= 1
            assert sizes.count(0) == max(0, S - T)


def test_planner_is_host_only():
    """The planner imports only the standard library and never names a device."""
    path = Path(planner.__file__)
    tree = ast.parse(path.read_text())
    mods = {a.name.split(".")[0] for n in ast.walk(tree) if isinstance(n, ast.Import) for a in n.names}
    mods |= {n.module.split(".")[0] for n in ast.walk(tree)
             if isinstance(n, ast.ImportFrom) and n.module}
    assert mods <= {"__future__", "dataclasses"}, mods
    assert "cuda" not in {n.attr for n in ast.walk(tree) if isinstance(n, ast.Attribute)}
