"""The vLLM backend's engine-independent core (``pth_flash_attn.slices``), the
packed-cache views and the plugin, on CPU tensors.

Mirrors the reference's builder and Impl tests (reference
tests/cpu/test_backend_builder.py, which need vLLM and skip without it) on the
core that holds that logic here: the decode threshold table, slicing of
decode / mixed / prefill-only / padded batches, the device-side rebase of the
prefill ``query_start_loc`` into one persistent buffer, plans equal to
``plan_launch`` of each slice's own descriptor and independent of the
sequence lengths, S * T within the reserved workspace for random batches,
every refusal with its reason, and at most two op calls per forward with the
exact tensors they get. The geometry is the reference tests' production one
(Hq 12, Hkv 2, D 256, 68 compute units, MTP k = 3) plus MI355X's 256 CUs.
"""

from __future__ import annotations

import importlib
import random
import subprocess
import sys

import pytest
import torch

from pth_flash_attn import planner, slices
from pth_flash_attn.cache import build_cache, carve_views, vllm_packed_views

HQ, HKV, D, CUS = 12, 2, 256, 68
G = HQ // HKV


def make_builder(*, heads=HQ, kv=HKV, head_size=D, window=0, k=3, max_num_seqs=2, cus=CUS):
    return slices.SliceBuilder(
        num_heads_q=heads, num_kv_heads=kv, head_size=head_size, window=window,
        max_num_seqs=max_num_seqs, q_verify=slices.verify_query_len(k), num_cus=cus,
        device="cpu",
    )


def make_step(q_lens, seq_lens=None, *, device_qsl=None, max_reqs=8):
    """Keyword arguments of ``SliceBuilder.build`` for a batch (CPU tensors)."""
    qsl = [0]
    for q in q_lens:
        qsl.append(qsl[-1] + q)
    seqs = seq_lens if seq_lens is not None else [q + 500 for q in q_lens]
    qsl_t = torch.tensor(qsl, dtype=torch.int32)
    seq_buf = torch.zeros(max_reqs, dtype=torch.int32)
    seq_buf[: len(seqs)] = torch.tensor(seqs, dtype=torch.int32)
    return dict(
        query_start_loc=torch.tensor(device_qsl, dtype=torch.int32) if device_qsl else qsl_t,
        query_start_loc_cpu=qsl_t, seq_lens=seq_buf[: len(q_lens)],
        block_table=torch.zeros(max_reqs, 8, dtype=torch.int32), num_reqs=len(q_lens),
        num_actual_tokens=qsl[-1], max_query_len=max(q_lens),
    )


def expected_plan(b, tokens, reqs, q_max, is_prefill):
    return planner.plan_launch(num_tokens=tokens, num_reqs=reqs, max_query_len=q_max, G=b.group,
                               Hkv=b.num_kv_heads, D=b.head_size, num_sms=b.num_cus,
                               is_prefill=is_prefill, ws_token_splits=b.ws_token_splits,
                               window=b.window)


# ------------------------------------------------------------------ constants


@pytest.mark.parametrize("heads, kv, k, want", [
    (12, 2, 3, 10),    # G = 6, MTP k = 3: floor(64/6) = 10
    (12, 2, None, 10),  # no speculation
    (12, 2, 15, 16),   # a verify of 16 outgrows the row tile
    (32, 8, 3, 16),    # G = 4
    (8, 1, 3, 8),      # G = 8
    (16, 1, 3, 4),     # G = 16: 64 // 16 = 4 = 1 + k
    (64, 1, 3, 4),     # G = 64: floor(64/64) = 1, raised by spec-as-decode
])
def test_decode_threshold(heads, kv, k, want):
    """reorder_batch_threshold = max(floor(64 / G), 1 + k)
    (reference tests/cpu/test_backend_builder.py:189-205)."""
    assert make_builder(heads=heads, kv=kv, k=k, head_size=128).reorder_batch_threshold == want


def test_verify_query_len():
    assert slices.verify_query_len(None) == 1
    assert slices.verify_query_len(0) == 1
    assert slices.verify_query_len(7) == 8
    with pytest.raises(ValueError):
        slices.verify_query_len(-1)


def test_reserved_workspace_is_the_planner_formula():
    b = make_builder()
    assert b.ws_token_splits == planner.workspace_token_splits(
        max_num_seqs=2, q_dec_max=4, Hkv=HKV, D=D, num_sms=CUS)
    # MI355X: one long request's split count is 2048 / Hkv.
    b = make_builder(heads=32, kv=8, head_size=128, k=0, max_num_seqs=64, cus=256)
    assert b.ws_token_splits == 64 * 1 * 256


# -------------------------------------------------------------------- slicing


def test_split_decodes_and_prefills_rules():
    qsl = torch.tensor([0, 4, 8, 9, 309, 329], dtype=torch.int32)
    f = slices.split_decodes_and_prefills
    assert f(qsl, num_reqs=5, num_tokens=329, max_query_len=300, threshold=10) == (3, 2, 9, 320)
    assert f(qsl, num_reqs=5, num_tokens=329, max_query_len=300, threshold=400) == (5, 0, 329, 0)
    first_long = torch.tensor([0, 300, 301], dtype=torch.int32)
    assert f(first_long, num_reqs=2, num_tokens=301, max_query_len=300, threshold=10) == (0, 2, 0, 301)
    # A decode after the first prefill stays in the prefill part.
    mixed = torch.tensor([0, 1, 301, 302], dtype=torch.int32)
    assert f(mixed, num_reqs=3, num_tokens=302, max_query_len=300, threshold=10) == (1, 2, 1, 301)


def test_all_decode_batch_is_one_decode_slice():
    """Two MTP verifies (q = 4): one decode launch, no prefill launch."""
    b = make_builder()
    kw = make_step([4, 4])
    st = b.build(**kw)
    assert st.prefill is None and st.decode is not None
    d = st.decode
    assert (d.token_start, d.token_end, d.max_query_len) == (0, 8, 4)
    assert d.plan == expected_plan(b, 8, 2, 4, False)
    assert d.plan.wm == 2 and d.plan.num_splits > 1
    # The step's persistent tensors are used as they are.
    assert d.query_start_loc is kw["query_start_loc"]
    assert d.seq_lens.data_ptr() == kw["seq_lens"].data_ptr()
    assert st.num_actual_tokens == 8 and st.causal is True


def test_mixed_batch_splits_into_decode_and_prefill():
    b = make_builder()
    st = b.build(**make_step([4, 4, 1, 300, 20]))
    d, p = st.decode, st.prefill
    assert (d.token_start, d.token_end, d.max_query_len) == (0, 9, 4)
    assert d.plan == expected_plan(b, 9, 3, 4, False)
    assert (p.token_start, p.token_end, p.max_query_len) == (9, 329, 300)
    assert p.plan == expected_plan(b, 320, 2, 300, True)
    assert p.plan.wm == 4 and p.plan.bq == 10
    assert p.seq_lens.shape == (2,) and p.block_table.shape[0] == 2
    assert p.query_start_loc.tolist() == [0, 300, 320]


def test_prefill_query_start_loc_is_rebased_on_the_device_value():
    """The device qsl is authoritative (adaptive verification trims drafts on it)."""
    b = make_builder()
    st = b.build(**make_step([2, 2, 300], device_qsl=[0, 3, 5, 305]))
    assert st.prefill.query_start_loc.tolist() == [0, 300]
    assert st.decode.query_start_loc.tolist() == [0, 3, 5]
    assert st.decode.max_query_len == 2  # the host bound


def test_prefill_rebase_buffer_is_persistent():
    b = make_builder()
    p1 = b.build(**make_step([1, 300])).prefill
    p2 = b.build(**make_step([1, 40, 40])).prefill
    assert p1.query_start_loc.data_ptr() == p2.query_start_loc.data_ptr()
    assert p2.query_start_loc.tolist() == [0, 40, 80]


def test_too_many_prefill_requests_fail_loudly():
    b = make_builder(max_num_seqs=2)
    with pytest.raises(RuntimeError, match="exceed max_num_seqs"):
        b.build(**make_step([1, 300, 300, 300]))


def test_prefill_only_batch():
    b = make_builder()
    st = b.build(**make_step([300]))
    assert st.decode is None and st.prefill.plan == expected_plan(b, 300, 1, 300, True)
    assert st.prefill.query_start_loc.tolist() == [0, 300]


def test_short_extend_counts_as_decode():
    """A chunk tail of 8 tokens (<= threshold 10) is decode-like."""
    st = make_builder().build(**make_step([8, 300]))
    assert st.decode.token_end == 8 and st.decode.max_query_len == 8
    assert st.decode.plan.wm == 4  # 8 tokens x 6 heads = 48 rows


def test_padded_graph_batch_is_all_decode():
    """Padding requests of a captured descriptor have q = 0 and stay in the slice."""
    b = make_builder()
    st = b.build(**make_step([4, 4, 0, 0], seq_lens=[10, 10, 0, 0]))
    assert st.prefill is None and st.decode.plan == expected_plan(b, 8, 4, 4, False)
    assert st.decode.seq_lens.shape == (4,)


def test_capture_build_sets_seq_lens_to_one():
    kw = make_step([4, 4], seq_lens=[9000, 9000])
    st = make_builder().build_for_graph_capture(**kw)
    assert st.decode.seq_lens.tolist() == [1, 1] and kw["seq_lens"].tolist() == [1, 1]


def test_plan_is_independent_of_sequence_length():
    b = make_builder()
    plans = {b.build(**make_step([4, 4], seq_lens=[s, s])).decode.plan
             for s in (8, 1000, 131072, 262144)}
    assert len(plans) == 1


@pytest.mark.parametrize("cus", [CUS, 256])
def test_splits_never_exceed_the_reserved_workspace(cus):
    """For random batches every slice has S * T <= W_ts (or S == 1)."""
    rng = random.Random(cus)
    for _ in range(300):
        k = rng.choice([None, 3, 7, 15])
        max_seqs = rng.choice([1, 2, 8, 64])
        b = make_builder(k=k, max_num_seqs=max_seqs, cus=cus)
        n_reqs = rng.randint(1, min(max_seqs, 9))
        n_dec = rng.randint(0, n_reqs)
        q = [rng.randint(1, b.reorder_batch_threshold) for _ in range(n_dec)]
        q += [rng.choice([11, 20, 64, 512, 8192]) for _ in range(n_reqs - n_dec)]
        st = b.build(**make_step(q, max_reqs=16))
        for part in (st.decode, st.prefill):
            if part is not None and part.plan.num_splits > 1:
                assert part.plan.num_splits * part.plan.num_tokens <= b.ws_token_splits


def test_window_caps_the_split_count():
    """A windowed group plans with its window (fewer splits than without)."""
    plain = make_builder(heads=32, kv=8, head_size=128, k=7, cus=256)
    win = make_builder(heads=32, kv=8, head_size=128, k=7, window=2048, cus=256)
    sp = plain.build(**make_step([8, 8])).decode.plan.num_splits
    sw = win.build(**make_step([8, 8])).decode.plan.num_splits
    assert sw < sp and sw == expected_plan(win, 16, 2, 8, False).num_splits


# ----------------------------------------------------------------- refusals


def test_per_request_causal_tensors_are_refused():
    for b in (make_builder(), make_builder(heads=16, kv=4, head_size=128, window=2048)):
        with pytest.raises(NotImplementedError, match="per-request causal"):
            b.build(**make_step([1]), causal=torch.tensor([True]))


@pytest.mark.parametrize("head_size", [64, 256])
def test_non_causal_and_window_off_d128_are_refused(head_size):
    b = make_builder(head_size=head_size)
    assert b.build(**make_step([1])).decode is not None
    with pytest.raises(NotImplementedError, match=f"non-causal attention at head size {head_size}"):
        b.build(**make_step([1]), causal=False)
    with pytest.raises(NotImplementedError, match=f"sliding window at head size {head_size}"):
        make_builder(head_size=head_size, window=2048)


def test_non_causal_windowed_d128_builds():
    b = make_builder(heads=16, kv=4, head_size=128, window=2048, k=7)
    st = b.build(**make_step([8, 8]), causal=False)
    assert st.causal is False and st.decode.plan.num_splits >= 1


def test_cascade_rswa_and_multimodal_prefixes_are_refused():
    b = make_builder()
    with pytest.raises(NotImplementedError, match="cascade"):
        b.build(**make_step([1]), common_prefix_len=16)
    with pytest.raises(NotImplementedError, match="R-SWA"):
        b.build(**make_step([1]), rswa_prefix_lens=torch.zeros(1, dtype=torch.int32))
    with pytest.raises(NotImplementedError, match="multimodal prefix"):
        b.build(**make_step([1, 1]), mm_req_doc_ranges={0: [(2, 6)], 1: []})
    assert b.build(**make_step([1, 1]), mm_req_doc_ranges={0: [], 1: []}).decode


def test_unsupported_geometry_is_refused():
    with pytest.raises(NotImplementedError, match="head size"):
        make_builder(head_size=80)
    with pytest.raises(ValueError, match="exceeds"):
        make_builder(heads=130, kv=1, head_size=128)
    with pytest.raises(ValueError, match="multiple"):
        make_builder(heads=12, kv=5, head_size=128)


@pytest.mark.parametrize("kwargs, what", [
    ({"alibi": True}, "ALiBi"),
    ({"sliding_window": 4096}, "sliding window at head size 256"),
    ({"sliding_window": 2048, "head_size": 64}, "sliding window at head size 64"),
    ({"sliding_window": 0}, "sliding window 0"),
    ({"logits_soft_cap": 30.0}, "soft cap"),
    ({"sinks": True}, "sinks"),
    ({"chunk_lookback": 8}, "chunk lookback"),
    ({"is_decoder": False}, "attention type"),
    ({"kv_cache_dtype": "auto"}, "kv_cache_dtype"),
    ({"kv_cache_dtype": "fp8"}, "kv_cache_dtype"),
    ({"head_size": 80}, "head size"),
])
def test_impl_refusals(kwargs, what):
    """reference tests/cpu/test_backend_builder.py:441-460."""
    args = {"head_size": D, **kwargs}
    reasons = slices.impl_refusals(**args)
    assert len(reasons) == 1 and what in reasons[0]


def test_production_and_drafter_layers_are_served():
    assert slices.impl_refusals(head_size=256) == []
    assert slices.impl_refusals(head_size=128, sliding_window=2048) == []


# ---------------------------------------------------------------- forward


class Recorder:
    """Stands in for the op: records each call's arguments."""

    def __init__(self):
        self.calls = []

    def __call__(self, *args):
        self.calls.append(args)


def _forward(step, b, *, T, reserved=None):
    query = torch.zeros(T, HQ, D, dtype=torch.bfloat16)
    output = torch.zeros_like(query)
    caches = tuple(torch.zeros(1) for _ in range(4))
    none = torch.empty(0)
    asked = []

    def workspace(o_shape, lse_shape):
        asked.append((o_shape, lse_shape))
        return torch.empty(o_shape), torch.empty(lse_shape)

    rec = Recorder()
    out = slices.run_slices(step, query=query, output=output, caches=caches, scale=0.0625,
                            window=0, workspace=workspace, no_workspace=none,
                            reserved_token_splits=b.ws_token_splits if reserved is None else reserved,
                            op=rec)
    return out, output, query, caches, none, asked, rec.calls


def test_at_most_two_op_calls_and_their_arguments():
    b = make_builder()
    step = b.build(**make_step([4, 4, 1, 300, 20]))
    out, output, query, caches, none, asked, calls = _forward(step, b, T=329)
    assert out is output and len(calls) == 2
    for call, part in zip(calls, (step.decode, step.prefill)):
        o, q, k, v, ks, vs, bt, sl, qsl, max_q, wm, S, scale, ws_o, ws_lse, window, causal = call
        assert o.data_ptr() == output[part.token_start:].data_ptr()
        assert o.shape[0] == q.shape[0] == part.token_end - part.token_start
        assert (k, v, ks, vs) == caches
        assert bt is part.block_table and sl is part.seq_lens and qsl is part.query_start_loc
        assert (max_q, wm, S) == (part.max_query_len, part.plan.wm, part.plan.num_splits)
        assert scale == 0.0625 and window == 0 and causal is True
        if S > 1:
            assert ws_o.shape == part.plan.ws_o_shape and ws_lse.shape == part.plan.ws_lse_shape
        else:
            assert ws_o is none and ws_lse is none
    assert len(asked) == sum(p.plan.num_splits > 1 for p in (step.decode, step.prefill))


def test_decode_only_forward_is_one_call_without_slicing():
    b = make_builder()
    step = b.build(**make_step([4, 4]))
    _, output, query, _, _, _, calls = _forward(step, b, T=8)
    assert len(calls) == 1
    assert calls[0][0] is output and calls[0][1] is query


def test_launch_beyond_the_reservation_fails_loudly():
    b = make_builder()
    step = b.build(**make_step([4, 4]))
    need = step.decode.plan.num_splits * step.decode.plan.num_tokens
    with pytest.raises(RuntimeError, match="token-splits"):
        _forward(step, b, T=8, reserved=need - 1)


# ------------------------------------------------------------- cache views


@pytest.mark.parametrize("pad, D_", [(0, 128), (64, 128), (0, 64), (0, 256)])
def test_vllm_packed_views_equal_the_hnd_cell_views(pad, D_):
    """vLLM's packed layer cache [blocks, heads, slots, 2 (D + 4)] is the HND
    cell layout: the views carved from it are the op's views, element for
    element and stride for stride."""
    Hkv, BS = 2, 16
    cache = build_cache([37, 5], Hkv=Hkv, D=D_, block_size=BS, seed=3, layout="HND",
                        pad_page_bytes=pad)
    C = 2 * (D_ + 4)
    packed = torch.as_strided(cache.storage, (cache.num_blocks, Hkv, BS, C),
                              (cache.page_bytes, BS * C, C, 1))
    got = vllm_packed_views(packed)
    want = (cache.k_cache, cache.v_cache, cache.k_scale, cache.v_scale)
    for g, w in zip(got, want):
        assert g.shape == w.shape and g.stride() == w.stride() and g.dtype == w.dtype
        assert torch.equal(g, w)
    ref = carve_views(cache.storage, num_blocks=cache.num_blocks, block_size=BS, Hkv=Hkv, D=D_,
                      layout="HND", pad_page_bytes=pad)
    assert all(torch.equal(a, b) for a, b in zip(got, ref))


def test_vllm_packed_views_accept_uint8_storage():
    packed = torch.randint(0, 256, (3, 2, 16, 264), dtype=torch.uint8)
    got = vllm_packed_views(packed)
    want = vllm_packed_views(packed.view(torch.int8))

    def bits(t):  # random bytes may form NaN scales: compare bit patterns
        return t.view(torch.int32) if t.dtype == torch.float32 else t

    assert all(a.dtype == b.dtype and torch.equal(bits(a), bits(b)) for a, b in zip(got, want))


def test_vllm_packed_views_refuse_bad_layouts():
    with pytest.raises(ValueError):
        vllm_packed_views(torch.zeros(2, 2, 16, 264, dtype=torch.float16))
    with pytest.raises(ValueError):
        vllm_packed_views(torch.zeros(2, 2, 16, 263, dtype=torch.int8))
    with pytest.raises(ValueError):
        vllm_packed_views(torch.zeros(2, 2, 16, 264, dtype=torch.int8).transpose(2, 3))


# ------------------------------------------------------------------ plugin


def _vllm_installed() -> bool:
    return importlib.util.find_spec("vllm") is not None


def test_importing_the_plugin_imports_neither_vllm_nor_the_backend():
    code = ("import sys, pth_flash_attn.plugin as p; "
            "assert p.BACKEND_CLASS_PATH == 'pth_flash_attn.vllm_backend.PthFlashAttnBackend'; "
            "assert 'vllm' not in sys.modules and 'pth_flash_attn.vllm_backend' not in sys.modules")
    import os

    import pth_flash_attn

    env = dict(os.environ)
    pkg_parent = os.path.dirname(os.path.dirname(pth_flash_attn.__file__))
    env["PYTHONPATH"] = pkg_parent + os.pathsep + env.get("PYTHONPATH", "")
    subprocess.run([sys.executable, "-c", code], check=True, env=env)


@pytest.mark.skipif(_vllm_installed(), reason="vLLM is installed")
def test_without_vllm_register_and_the_backend_raise_import_error():
    from pth_flash_attn import plugin

    with pytest.raises(ImportError):
        plugin.register()
    with pytest.raises(ImportError):
        importlib.import_module("pth_flash_attn.vllm_backend")


def test_carve_views_of_a_slice_of_a_larger_buffer():
    """Views carved from a storage that is itself a slice (bench.py rotates
    input copies carved from one allocation) address that slice's bytes."""
    c = build_cache([100, 37], Hkv=2, D=128, block_size=16, seed=1)
    big = c.storage.unsqueeze(0).repeat(3, 1)
    big[0].fill_(7)
    for i in (1, 2):
        got = carve_views(big[i], num_blocks=c.num_blocks, block_size=16, Hkv=2, D=128)
        for g, w in zip(got, (c.k_cache, c.v_cache, c.k_scale, c.v_scale)):
            assert torch.equal(g, w)
