"""Pins the CPU oracle (CPU only).

Each oracle function is checked against something independent of its own
formula:

* writer ``oracle_quantize_rows``: the reference's known-answer vector
  (reference tests/cpu/test_reference.py:41-56), the scale floor and the
  full-scale extremes (test_reference.py:58-85), and bit equality with the
  torch writer mirror the cache builder uses;
* attention ``oracle_attention``: a plain numpy per-row loop on dense
  dequantised K/V (tiny cases), closed forms (one visible key: out = v and
  lse = the score; equal keys: out = mean of V; lse = logsumexp of the
  scaled scores), and the reference's own compiled CPU path
  ``oracle/_ref/libpth_ref_host.so`` (skipped when it is not built);
* combine ``oracle_combine``: the split identity (attention over disjoint key
  sets merged by lse equals attention over their union), empty splits with
  NaN partials, natural-log misuse as a negative control, and the
  reference's compiled combine.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import oracle
from pth_flash_attn import capi
from pth_flash_attn.cache import SCALE_FLOOR, build_cache, make_queries
from pth_flash_attn.cache import quantize_rows as torch_quantize_rows

# The launch arguments carry softmax_scale as fp32.
SCALE = float(np.float32(1.0 / math.sqrt(128)))


# ----------------------------------------------------------------- writer
def test_writer_known_answer():
    x = np.array([[127.0, 2.5, -2.5, 0.5, -0.5, 3.5, -126.5]], dtype=np.float32)
    q, s = oracle.quantize_rows(x)
    assert s.tolist() == [1.0]
    assert q.tolist() == [[127, 3, -3, 1, -1, 4, -127]]
    tq, ts = torch_quantize_rows(torch.from_numpy(x))
    assert tq.tolist() == q.tolist() and ts.tolist() == [1.0]
    # Negative control: round-half-to-even differs on these ties.
    assert np.round(x / s[:, None]).astype(np.int8).tolist() != q.tolist()


def test_writer_scale_floor_and_extremes():
    rng = np.random.default_rng(0)
    zero = np.zeros((3, 128), np.float32)
    tiny = (rng.uniform(-1.2e-4, 1.2e-4, (5, 128))).astype(np.float32)
    for x in (zero, tiny):
        q, s = oracle.quantize_rows(x)
        assert np.all(s == np.float32(SCALE_FLOOR))
        assert np.all(np.abs(q.astype(np.int32)) <= 127)
    big = rng.standard_normal((64, 128)).astype(np.float32) * 1e3
    q, s = oracle.quantize_rows(big)
    assert q.min() >= -127 and q.max() <= 127
    # the row maximum lands on +-127 exactly
    assert np.all(np.abs(q).max(axis=1) == 127)
    # Negative control: without the floor, the zero rows would get scale 0.
    assert not np.all(zero.max(axis=1) / 127.0 == np.float32(SCALE_FLOOR))


def test_writer_mirrors_agree_bitwise():
    rng = np.random.default_rng(1)
    x = (rng.standard_normal((4096, 128)) * rng.uniform(1e-5, 50, (4096, 1))).astype(np.float32)
    q, s = oracle.quantize_rows(x)
    tq, ts = torch_quantize_rows(torch.from_numpy(x))
    assert np.array_equal(q, tq.numpy()) and np.array_equal(s, ts.numpy())


# -------------------------------------------------------------- attention
def dense_kv(cache, r: int) -> tuple[np.ndarray, np.ndarray]:
    """Dequantised fp64 K/V [L, Hkv, D] of request r, read through the block table."""
    L = int(cache.seq_lens[r])
    pos = torch.arange(L)
    blk = cache.block_table[r].long()[pos // cache.block_size]
    slot = pos % cache.block_size
    k = cache.k_cache[blk, slot].double() * cache.k_scale[blk, slot].double()[..., None]
    v = cache.v_cache[blk, slot].double() * cache.v_scale[blk, slot].double()[..., None]
    return k.numpy(), v.numpy()


def run_oracle(q, qsl, cache, window=0, causal=True, scale=None):
    D = q.shape[-1]
    scale = SCALE if scale is None else scale
    out = torch.empty(q.shape, dtype=torch.float32)
    a = capi.attn_args(q=q, out=out, k_cache=cache.k_cache, v_cache=cache.v_cache,
                       k_scale=cache.k_scale, v_scale=cache.v_scale,
                       block_table=cache.block_table, seq_lens=cache.seq_lens,
                       query_start_loc=qsl, bq=1, num_splits=1, softmax_scale=scale,
                       window=window, causal=causal)
    return oracle.attention(a)


SMALL = [
    # q_lens, seq_lens, Hq, Hkv, block, window, causal, layout
    ([1], [1], 4, 1, 16, 0, True, "NHD"),
    ([1, 3, 0, 2], [37, 5, 9, 64], 8, 2, 16, 0, True, "NHD"),
    ([4, 1], [100, 17], 8, 2, 16, 0, False, "HND"),
    ([5, 2], [130, 40], 4, 1, 32, 16, True, "NHD"),
    ([3, 6], [70, 6], 6, 3, 16, 7, False, "HND"),
    ([16], [200], 16, 4, 16, 64, True, "NHD"),
]


@pytest.mark.parametrize("case", SMALL, ids=[str(i) for i in range(len(SMALL))])
def test_oracle_matches_numpy_loop(case):
    q_lens, seq_lens, Hq, Hkv, bs, W, causal, layout = case
    D = 128
    cache = build_cache(seq_lens, Hkv=Hkv, D=D, block_size=bs, seed=7, layout=layout)
    q, qsl = make_queries(q_lens, Hq=Hq, D=D, seed=8)
    out, lse, valid = run_oracle(q, qsl, cache, W, causal)
    ks, vs = zip(*(dense_kv(cache, r) for r in range(len(seq_lens))))
    ref_o, ref_l = oracle.attention_numpy(q.float().numpy(), list(ks), list(vs),
                                         qsl.tolist(), seq_lens, SCALE,
                                         window=W, causal=causal)
    assert valid.sum() == sum(q_lens)
    np.testing.assert_allclose(out, ref_o, rtol=0, atol=1e-12)
    np.testing.assert_allclose(lse[valid], ref_l[valid], rtol=0, atol=1e-12)
    assert np.all(np.isneginf(lse[~valid]))


def test_oracle_closed_forms():
    D, Hq = 128, 4
    # One visible key (L = 1): out is that key's V row exactly, lse its score.
    cache = build_cache([1], Hkv=1, D=D, block_size=16, seed=3)
    q, qsl = make_queries([1], Hq=Hq, D=D, seed=4)
    out, lse, _ = run_oracle(q, qsl, cache)
    k, v = dense_kv(cache, 0)
    for h in range(Hq):
        np.testing.assert_array_equal(out[0, h], v[0, 0])
        s = float(k[0, 0] @ q[0, h].double().numpy()) * SCALE
        assert math.isclose(lse[0, h], s, rel_tol=1e-13, abs_tol=1e-13)
    # Every key equal: softmax is uniform, out = mean of V, lse = s + ln L.
    L = 50
    cache = build_cache([L], Hkv=1, D=D, block_size=16, seed=5)
    blk = cache.block_table[0].long()[torch.arange(L) // 16]
    slot = torch.arange(L) % 16
    cache.k_cache[blk, slot] = cache.k_cache[blk[0], slot[0]].clone()
    cache.k_scale[blk, slot] = cache.k_scale[blk[0], slot[0]].clone()
    out, lse, _ = run_oracle(q, qsl, cache)
    k, v = dense_kv(cache, 0)
    np.testing.assert_allclose(out[0], np.broadcast_to(v[:, 0].mean(0), (Hq, D)), atol=1e-13)
    s = k[0, 0] @ q[0].double().numpy().T * SCALE
    np.testing.assert_allclose(lse[0], s + math.log(L), atol=1e-12)
    # lse is the natural-log logsumexp of the scaled scores (not log2).
    cache = build_cache([300], Hkv=1, D=D, block_size=16, seed=6)
    out, lse, _ = run_oracle(q, qsl, cache)
    k, _ = dense_kv(cache, 0)
    sc = k[:, 0] @ q[0].double().numpy().T * SCALE
    want = np.log(np.exp(sc - sc.max(0)).sum(0)) + sc.max(0)
    np.testing.assert_allclose(lse[0], want, atol=1e-12)
    assert np.all(np.abs(lse[0] - want / math.log(2)) > 1e-3)  # negative control


def test_oracle_reads_only_visible_keys():
    """Changing a key outside every visible range leaves the result unchanged;
    changing a visible key changes it."""
    D = 128
    cache = build_cache([80], Hkv=1, D=D, block_size=16, seed=9)
    q, qsl = make_queries([2], Hq=2, D=D, seed=10)
    base, _, _ = run_oracle(q, qsl, cache, window=16)
    for pos, changes in ((10, False), (70, True)):
        c2 = build_cache([80], Hkv=1, D=D, block_size=16, seed=9)
        b = int(c2.block_table[0, pos // 16])
        c2.v_cache[b, pos % 16] = -c2.v_cache[b, pos % 16]
        got, _, _ = run_oracle(q, qsl, c2, window=16)
        assert (not np.array_equal(got, base)) == changes, pos


# ----------------------------------------------------------------- combine
def test_combine_split_identity():
    """Attention over keys split into S disjoint sets, merged by log2-LSE,
    equals attention over all keys; empty splits (-inf, NaN o) are ignored."""
    rng = np.random.default_rng(11)
    T, Hq, D, n = 3, 2, 16, 97
    s = rng.standard_normal((T, Hq, n)) * 4
    v = rng.standard_normal((n, D))
    w = np.exp(s - s.max(-1, keepdims=True))
    full = (w / w.sum(-1, keepdims=True)) @ v
    full_lse = np.log(w.sum(-1)) + s.max(-1)
    cuts = [0, 10, 10, 60, 97]  # split 1 is empty
    S = len(cuts) - 1
    ws_o = np.full((S, T, Hq, D), np.nan, np.float32)
    ws_l = np.full((S, T, Hq), -np.inf, np.float32)
    for i in range(S):
        a, b = cuts[i], cuts[i + 1]
        if a == b:
            continue
        ss = s[..., a:b]
        m = ss.max(-1, keepdims=True)
        e = np.exp(ss - m)
        ws_o[i] = (e / e.sum(-1, keepdims=True)) @ v[a:b]
        ws_l[i] = (np.log2(e.sum(-1)) + m[..., 0] / math.log(2))
    out, lse = oracle.combine(ws_o, ws_l)
    np.testing.assert_allclose(out, full, atol=1e-5)
    np.testing.assert_allclose(lse, full_lse, atol=1e-5)
    # Negative control: weighting by e^lse (natural log) instead of 2^lse is wrong.
    wrong = np.exp(ws_l - np.nanmax(ws_l, 0))
    wrong_out = np.nansum(np.where(np.isfinite(ws_l)[..., None], wrong[..., None] * np.nan_to_num(ws_o), 0), 0)
    wrong_out /= wrong.sum(0)[..., None]
    assert np.abs(wrong_out - full).max() > 1e-2
    # All splits empty: zero output, lse -inf.
    out, lse = oracle.combine(np.full((2, 1, 1, D), np.nan, np.float32),
                              np.full((2, 1, 1), -np.inf, np.float32))
    assert np.all(out == 0) and np.all(np.isneginf(lse))


# ---------------------------------------------- the reference's own CPU path
needs_ref = pytest.mark.skipif(not oracle.REF_LIB_PATH.is_file(),
                               reason="oracle/_ref not built (needs /root/reference)")

REF_CASES = [
    ([1], [1024], 4, 1, 0, True),       # config 1
    ([1, 4, 2], [300, 77, 16], 8, 2, 0, True),
    ([3, 1], [200, 90], 8, 2, 32, False),
    ([16, 5], [260, 64], 4, 1, 100, True),
]


@needs_ref
@pytest.mark.parametrize("case", REF_CASES, ids=[str(i) for i in range(len(REF_CASES))])
def test_oracle_matches_reference_cpu(case):
    q_lens, seq_lens, Hq, Hkv, W, causal = case
    D = 128
    cache = build_cache(seq_lens, Hkv=Hkv, D=D, block_size=16, seed=12)
    q, qsl = make_queries(q_lens, Hq=Hq, D=D, seed=13)
    out, lse, valid = run_oracle(q, qsl, cache, W, causal)
    ref_out = torch.zeros(q.shape, dtype=torch.float32)
    a = capi.attn_args(q=q, out=ref_out, k_cache=cache.k_cache, v_cache=cache.v_cache,
                       k_scale=cache.k_scale, v_scale=cache.v_scale,
                       block_table=cache.block_table, seq_lens=cache.seq_lens,
                       query_start_loc=qsl, bq=4, num_splits=1,
                       softmax_scale=1.0 * SCALE, window=W, causal=causal)
    oracle.reference_attention(a)
    # The reference path computes in fp32: agreement to fp32 accumulation error.
    np.testing.assert_allclose(ref_out.numpy()[valid], out[valid], atol=2e-6, rtol=0)


@needs_ref
def test_combine_matches_reference_cpu():
    """Split partials from the reference's CPU path merged by the reference's
    combine equal the oracle's unsplit attention and the oracle's combine."""
    D, Hq, S = 128, 4, 3
    q_lens, seq_lens = [2, 1], [400, 201]
    cache = build_cache(seq_lens, Hkv=1, D=D, block_size=16, seed=14)
    q, qsl = make_queries(q_lens, Hq=Hq, D=D, seed=15)
    T = q.shape[0]
    ws_o = torch.zeros(S, T, Hq, D)
    ws_l = torch.zeros(S, T, Hq)
    out = torch.zeros(T, Hq, D)
    a = capi.attn_args(q=q, out=out, k_cache=cache.k_cache, v_cache=cache.v_cache,
                       k_scale=cache.k_scale, v_scale=cache.v_scale,
                       block_table=cache.block_table, seq_lens=cache.seq_lens,
                       query_start_loc=qsl, bq=4, num_splits=S,
                       softmax_scale=1.0 * SCALE, ws_o=ws_o, ws_lse=ws_l)
    oracle.reference_attention(a)
    c = capi.combine_args(ws_o=ws_o, ws_lse=ws_l, out=out, query_start_loc=qsl,
                          num_reqs=len(q_lens), num_splits=S)
    oracle.reference_combine(c)
    want, want_lse, valid = run_oracle(q, qsl, cache)
    np.testing.assert_allclose(out.numpy()[valid], want[valid], atol=2e-6, rtol=0)
    mine, mine_lse = oracle.combine(ws_o.numpy(), ws_l.numpy())
    np.testing.assert_allclose(mine[valid], want[valid], atol=2e-6, rtol=0)
    np.testing.assert_allclose(mine_lse[valid], want_lse[valid], atol=2e-6, rtol=0)
