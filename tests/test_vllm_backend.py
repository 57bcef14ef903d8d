"""The vLLM adapter (``pth_flash_attn.vllm_backend``, ``plugin``) executed on the
CPU against stand-ins for the vLLM names it imports (``tests/vllm_stub.py``;
vLLM is not installed here), with the op replaced by a recorder, as the
reference drives its own backend (``tests/cpu/test_backend_builder.py``).

What is protected, in the reference's terms (MI355X constants: 256 CUs):
* graph-level constants: ``UNIFORM_BATCH`` (2), reorder threshold
  ``max(floor(64 / G), 1 + k)`` with spec-as-decode, draft-metadata update;
* every launch slice is ``plan_launch`` of its own descriptor, and the prefill
  ``query_start_loc`` is rebased on the device value (reference
  vllm_backend.py:287-446);
* the Impl reserves ``W_ts`` token-splits of workspace at construction, and
  with the workspace locked a forward of every planned size allocates nothing;
  a launch beyond the reservation fails loudly (reference :645-678, 751-796);
* at most two op calls per forward, with the exact tensors (reference
  :704-796);
* refusals with their reasons (reference :185-211, 251-255, 589-632);
* the plugin registers the class path under ``CUSTOM`` and leaves another
  plugin's registration alone (reference plugin.py:28-45).
"""

from __future__ import annotations

import logging
import math
from types import SimpleNamespace

import pytest
import torch

import vllm_stub
from pth_flash_attn import ops, planner

HQ, HKV, D, CUS, K_SPEC = 32, 8, 128, 256, 3
G = HQ // HKV
KV_DTYPE = "int8_per_token_head"


@pytest.fixture(scope="module")
def vb():
    with vllm_stub.installed():
        import pth_flash_attn.vllm_backend as mod

        yield mod


@pytest.fixture(autouse=True)
def fixed_cu_count(vb, monkeypatch):
    """The CU count is a planner input; no GPU is asked for it."""
    monkeypatch.setattr(vb, "_num_cus", lambda device=None: CUS)
    vllm_stub.reset_workspace_manager()
    yield
    vllm_stub.reset_workspace_manager()


def make_config(*, k=K_SPEC, max_num_seqs=8, heads=HQ, rswa=None, dbo=False):
    spec = None if k is None else SimpleNamespace(num_speculative_tokens=k)
    return SimpleNamespace(
        model_config=SimpleNamespace(rswa_window=rswa, get_num_attention_heads=lambda pc: heads),
        parallel_config=SimpleNamespace(use_ubatching=dbo, num_ubatches=2 if dbo else 1),
        scheduler_config=SimpleNamespace(max_num_seqs=max_num_seqs),
        speculative_config=spec,
        compilation_config=SimpleNamespace(static_forward_context={}),
    )


def make_builder(vb, *, num_kv_heads=HKV, head_size=D, sliding_window=None, **cfg):
    spec = vllm_stub.AttentionSpec(num_kv_heads=num_kv_heads, head_size=head_size,
                                   sliding_window=sliding_window)
    return vb.PthFlashAttnMetadataBuilder(spec, ["layers.0.attn"], make_config(**cfg),
                                          torch.device("cpu"))


def make_cam(q_lens, seq_lens, block_size=16):
    qsl = torch.tensor([0] + list(torch.tensor(q_lens).cumsum(0).tolist()), dtype=torch.int32)
    nblk = max(math.ceil(L / block_size) for L in seq_lens)
    bt = torch.arange(len(q_lens) * nblk, dtype=torch.int32).reshape(len(q_lens), nblk)
    T = int(qsl[-1])
    return vllm_stub.CommonAttentionMetadata(
        query_start_loc=qsl.clone(), query_start_loc_cpu=qsl.clone(),
        seq_lens=torch.tensor(seq_lens, dtype=torch.int32), num_reqs=len(q_lens),
        num_actual_tokens=T, max_query_len=max(q_lens), max_seq_len=max(seq_lens),
        block_table_tensor=bt, slot_mapping=torch.arange(T, dtype=torch.int64), causal=True)


def plan_of(builder, *, tokens, reqs, q_max, prefill):
    return planner.plan_launch(num_tokens=tokens, num_reqs=reqs, max_query_len=q_max, G=G,
                               Hkv=HKV, D=D, num_sms=CUS, is_prefill=prefill,
                               ws_token_splits=builder.ws_token_splits, window=0)


# ------------------------------------------------------------------ builder
def test_builder_graph_constants(vb):
    b = make_builder(vb)
    assert b._cudagraph_support is vllm_stub.AttentionCGSupport.UNIFORM_BATCH
    assert b._cudagraph_support.value == 2
    assert b.supports_draft_decode_metadata_update
    assert b.reorder_batch_threshold == max(64 // G, 1 + K_SPEC) == 16
    assert vb.PthFlashAttnMetadataBuilder.get_varlen_cudagraph_max_query_len(
        make_config(), vllm_stub.AttentionSpec(num_kv_heads=HKV, head_size=D)) == 16
    assert b.ws_token_splits == planner.workspace_token_splits(
        max_num_seqs=8, q_dec_max=1 + K_SPEC, Hkv=HKV, D=D, num_sms=CUS)
    # The reference's production shape (G = 6, MTP k = 3): threshold 10.
    b6 = make_builder(vb, num_kv_heads=2, head_size=256, heads=12)
    assert b6.reorder_batch_threshold == max(64 // 6, 4) == 10
    # No speculation: floor(64 / G).
    assert make_builder(vb, k=None).reorder_batch_threshold == 16


@pytest.mark.parametrize(("kw", "msg"), [
    (dict(dbo=True), "dual-batch overlap"),
    (dict(rswa=128), "R-SWA"),
    (dict(head_size=96), "head size 96"),
    (dict(head_size=256, num_kv_heads=2, heads=12, sliding_window=1024), "sliding window"),
])
def test_builder_refusals(vb, kw, msg):
    with pytest.raises(NotImplementedError, match=msg):
        make_builder(vb, **kw)


def test_build_mixed_batch_plans_each_slice(vb):
    b = make_builder(vb)
    q_lens, seq_lens = [1, 1, 4, 1, 300, 50], [4000, 900, 2000, 17, 800, 3050]
    cam = make_cam(q_lens, seq_lens)
    step = b.build(0, cam)
    assert step.decode.plan == plan_of(b, tokens=7, reqs=4, q_max=4, prefill=False)
    assert step.prefill.plan == plan_of(b, tokens=350, reqs=2, q_max=300, prefill=True)
    assert (step.decode.token_start, step.decode.token_end) == (0, 7)
    assert (step.prefill.token_start, step.prefill.token_end) == (7, 357)
    assert step.decode.query_start_loc.tolist() == [0, 1, 2, 6, 7]
    assert step.prefill.query_start_loc.tolist() == [0, 300, 350]  # rebased on the device copy
    assert step.prefill.query_start_loc.data_ptr() == b.core.prefill_qsl.data_ptr()
    assert step.decode.seq_lens.tolist() == seq_lens[:4]
    assert step.prefill.seq_lens.tolist() == seq_lens[4:]
    assert torch.equal(step.prefill.block_table, cam.block_table_tensor[4:])
    # The names vLLM's runners and speculators read.
    assert step.query_start_loc is cam.query_start_loc and step.seq_lens is cam.seq_lens
    assert step.block_table is cam.block_table_tensor and step.slot_mapping is cam.slot_mapping
    assert step.max_seq_len == 4000 and step.use_cascade is False and step.common_prefix_len == 0


def test_build_rebases_on_the_device_value(vb):
    """Under adaptive verification the host copy of query_start_loc can
    differ from the device copy: the prefill slice subtracts the device value."""
    b = make_builder(vb)
    cam = make_cam([2, 40, 10], [100, 200, 300])
    cam.query_start_loc = cam.query_start_loc + 0  # a separate device copy
    cam.query_start_loc[1:] -= 1  # the first request verified one token fewer
    step = b.build(0, cam)
    assert step.prefill.query_start_loc.tolist() == [0, 40, 50]


def test_build_decode_only_and_refusals(vb):
    b = make_builder(vb)
    step = b.build(0, make_cam([1] * 5, [100, 200, 300, 400, 500]))
    assert step.prefill is None and step.decode.plan == plan_of(b, tokens=5, reqs=5, q_max=1,
                                                                prefill=False)
    with pytest.raises(NotImplementedError, match="cascade"):
        b.build(16, make_cam([1], [100]))
    cam = make_cam([1, 1], [100, 100])
    cam.causal = torch.tensor([True, False])
    with pytest.raises(NotImplementedError, match="per-request causal"):
        b.build(0, cam)


def test_build_for_cudagraph_capture(vb):
    b = make_builder(vb)
    cam = make_cam([4] * 3, [500, 600, 700])
    step = b.build_for_cudagraph_capture(cam)
    assert step.seq_lens.tolist() == [1, 1, 1]
    assert step.decode.plan == plan_of(b, tokens=12, reqs=3, q_max=4, prefill=False)
    b.update_draft_decode_metadata(step)  # nothing to update


# ------------------------------------------------------------------ backend
def test_backend_queries(vb):
    B = vb.PthFlashAttnBackend
    assert B.get_name() == "CUSTOM"
    assert B.get_impl_cls() is vb.PthFlashAttnImpl
    assert B.get_builder_cls() is vb.PthFlashAttnMetadataBuilder
    assert B.get_supported_kernel_block_sizes() == [vllm_stub.MultipleOf(16)]
    assert all(B.supports_block_size(s) for s in (None, 16, 32, 528))
    assert not B.supports_block_size(8)
    assert all(B.supports_head_size(d) for d in (64, 128, 256)) and not B.supports_head_size(96)
    assert B.supports_attn_type(vllm_stub.AttentionType.DECODER)
    assert not B.supports_attn_type(vllm_stub.AttentionType.ENCODER)
    assert B.supports_non_causal() and B.supports_sliding_window()
    assert not (B.supports_rswa() or B.supports_sink() or B.supports_mm_prefix()
                or B.supports_alibi_sqrt() or B.supports_batch_invariance())
    assert B.supported_kv_cache_dtypes == [KV_DTYPE]
    cap = vllm_stub.DeviceCapability
    assert B.supports_compute_capability(cap(9, 5)) == ops.is_available()
    assert not B.supports_compute_capability(cap(9, 4))


def test_validate_configuration_reasons(vb):
    B = vb.PthFlashAttnBackend
    cap = vllm_stub.DeviceCapability(9, 5)
    base = dict(dtype=torch.bfloat16, kv_cache_dtype=KV_DTYPE, block_size=16, use_mla=False,
                has_sink=False, use_sparse=False, device_capability=cap)
    w256 = B.validate_configuration(head_size=256, has_sliding_window=True, **base)
    assert any("sliding window at head size 256" in r for r in w256)
    nc64 = B.validate_configuration(head_size=64, use_non_causal=True, **base)
    assert any("non-causal attention at head size 64" in r for r in nc64)
    ok = B.validate_configuration(head_size=128, has_sliding_window=True, use_non_causal=True,
                                  **base)
    assert not any("head size" in r for r in ok)
    bad = B.validate_configuration(head_size=128, **{**base, "kv_cache_dtype": "auto"})
    assert "kv_cache_dtype not supported" in bad


# --------------------------------------------------------------------- Impl
def make_impl(vb, **kw):
    args = dict(num_heads=HQ, head_size=D, scale=D ** -0.5, num_kv_heads=HKV, alibi_slopes=None,
                sliding_window=None, kv_cache_dtype=KV_DTYPE)
    args.update(kw)
    return vb.PthFlashAttnImpl(**args)


@pytest.mark.parametrize(("kw", "msg"), [
    (dict(alibi_slopes=[0.5]), "ALiBi"),
    (dict(logits_soft_cap=30.0), "logits soft cap"),
    (dict(sinks=torch.zeros(HQ)), "attention sinks"),
    (dict(chunk_lookback=8), "chunk lookback"),
    (dict(attn_type=vllm_stub.AttentionType.ENCODER), "other than decoder"),
    (dict(kv_cache_dtype="auto"), "kv_cache_dtype auto"),
    (dict(head_size=256, sliding_window=512), "sliding window at head size 256"),
])
def test_impl_refusals(vb, kw, msg):
    with pytest.raises(NotImplementedError, match=msg):
        make_impl(vb, **kw)
    with pytest.raises(ValueError, match="multiple"):
        make_impl(vb, num_heads=30)


def test_impl_reserves_the_workspace_at_load(vb):
    impl = make_impl(vb)  # no workspace manager yet: nothing reserved
    assert impl._ws_token_splits == 0
    mgr = vllm_stub.init_workspace_manager("cpu")
    cfg = make_config()
    with vllm_stub.current_config(cfg):
        impl = make_impl(vb)
    w_ts = vb.reserved_token_splits(cfg, num_kv_heads=HKV, head_size=D, num_sms=CUS)
    assert impl._ws_token_splits == w_ts > 0
    o_shape, lse_shape = planner.workspace_shapes(ws_token_splits=w_ts, Hq=HQ, D=D)
    assert mgr.buffer.numel() >= 4 * (math.prod(o_shape) + math.prod(lse_shape))
    assert impl._no_workspace is not None and impl._no_workspace.numel() == 0


class Recorder:
    def __init__(self):
        self.calls = []

    def __call__(self, *args):
        self.calls.append(args)


def packed_cache(num_blocks=64, block_size=16):
    return torch.zeros(num_blocks, HKV, block_size, 2 * (D + 4), dtype=torch.int8)


def test_forward_makes_two_op_calls_and_allocates_nothing(vb, monkeypatch):
    mgr = vllm_stub.init_workspace_manager("cpu")
    cfg = make_config()
    with vllm_stub.current_config(cfg):
        impl = make_impl(vb)
    mgr.lock()
    grows = mgr.grows
    rec = Recorder()
    monkeypatch.setattr(ops, "pth_flash_attn_fwd", rec)
    b = make_builder(vb)
    q_lens, seq_lens = [1, 1, 4, 1, 300, 50], [4000, 900, 2000, 17, 800, 3050]
    step = b.build(0, make_cam(q_lens, seq_lens))
    T = sum(q_lens)
    query = torch.randn(T, HQ, D).to(torch.bfloat16)
    output = torch.empty_like(query)
    kv = packed_cache()
    out = impl.forward(None, query, None, None, kv, step, output)
    assert out is output
    assert len(rec.calls) == 2 and mgr.grows == grows
    views = vb.vllm_packed_views(kv)
    for call, part, (t0, t1) in zip(rec.calls, (step.decode, step.prefill), ((0, 7), (7, T))):
        (o, q, k, v, ks, vs, bt, sl, qsl, mql, wm, S, scale, ws_o, ws_lse, window, causal) = call
        assert o.data_ptr() == output[t0:t1].data_ptr() and o.shape[0] == t1 - t0
        assert q.data_ptr() == query[t0:t1].data_ptr()
        for got, want in zip((k, v, ks, vs), views):
            assert got.data_ptr() == want.data_ptr() and got.stride() == want.stride()
        assert bt is part.block_table and sl is part.seq_lens and qsl is part.query_start_loc
        assert (mql, wm, S) == (part.max_query_len, part.plan.wm, part.plan.num_splits)
        assert scale == pytest.approx(D ** -0.5) and window == 0 and causal is True
        if S > 1:
            assert tuple(ws_o.shape) == part.plan.ws_o_shape
            assert tuple(ws_lse.shape) == part.plan.ws_lse_shape
            assert ws_o.dtype == ws_lse.dtype == torch.float32
        else:
            assert ws_o.numel() == 0 and ws_lse.numel() == 0
    assert rec.calls[0][11] > 1  # the decode part runs split (workspace views used)
    # The cache views are carved once per cache tensor.
    impl.forward(None, query, None, None, kv, step, output)
    assert rec.calls[2][2].data_ptr() == rec.calls[0][2].data_ptr()
    # A decode-only step: one call.
    rec.calls.clear()
    step1 = b.build(0, make_cam([1] * 5, [100, 200, 300, 400, 500]))
    impl.forward(None, query[:5], None, None, kv, step1, output[:5])
    assert len(rec.calls) == 1 and mgr.grows == grows


def test_forward_profile_run_and_refusals(vb, monkeypatch):
    rec = Recorder()
    monkeypatch.setattr(ops, "pth_flash_attn_fwd", rec)
    impl = make_impl(vb)
    output = torch.ones(3, HQ, D)
    assert impl.forward(None, output, None, None, packed_cache(), None, output) is output
    assert torch.count_nonzero(output) == 0 and not rec.calls
    with pytest.raises(NotImplementedError, match="output quantisation"):
        impl.forward(None, output, None, None, packed_cache(), None, output,
                     output_scale=torch.ones(1))


def test_forward_beyond_the_reservation_fails_loudly(vb, monkeypatch):
    vllm_stub.init_workspace_manager("cpu")
    with vllm_stub.current_config(make_config(max_num_seqs=1, k=None)):
        impl = make_impl(vb)
    monkeypatch.setattr(ops, "pth_flash_attn_fwd", Recorder())
    b = make_builder(vb, max_num_seqs=64)
    step = b.build(0, make_cam([1] * 64, [32768] * 64))
    assert step.decode.plan.num_splits * 64 > impl._ws_token_splits
    q = torch.zeros(64, HQ, D, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="were reserved"):
        impl.forward(None, q, None, None, packed_cache(), step, torch.empty_like(q))


# ------------------------------------------------------------------- plugin
def test_plugin_registers_custom(vb, caplog):
    from pth_flash_attn import plugin

    reg = vllm_stub.AttentionBackendEnum
    plugin.register()
    assert reg.CUSTOM.get_path() == plugin.BACKEND_CLASS_PATH
    plugin.register()  # idempotent
    assert reg.CUSTOM.get_path() == plugin.BACKEND_CLASS_PATH
    vllm_stub.register_backend(reg.CUSTOM, "other.Backend")
    with caplog.at_level(logging.WARNING):
        plugin.register()
    assert reg.CUSTOM.get_path() == "other.Backend"
    assert "already registered" in caplog.text
