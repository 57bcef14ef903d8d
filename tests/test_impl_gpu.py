"""``PthFlashAttnImpl.forward`` on the GPU, builder to kernel, through the vLLM
adapter itself (``pth_flash_attn.vllm_backend``) under the stand-ins for the
vLLM names it imports (``tests/vllm_stub.py``; vLLM is not installed).

Mirrors the reference's tests/gpu/test_backend_impl.py:1-25, 129-230:

* a mixed batch (two MTP verifies of 4 tokens, a decode, a 300-token chunk
  with a prefix and a 20-token chunk): the builder splits it into its
  decode-like and prefill slices, the Impl runs the real op on each, and the
  output is checked against the fp64 oracle;
* the build and the forward run under ``torch.cuda.set_sync_debug_mode("error")``,
  so any host synchronisation raises;
* after the first call a forward allocates nothing (``memory_allocated`` and
  the workspace buffer unchanged);
* the Impl captured in a CUDA graph for a uniform verify batch replays equal,
  bit for bit, to the eager call after ``seq_lens`` changed on the device.

Geometries: this build's tuned one (32q/8kv, D = 128, page 16) and the
reference's production one (12q/2kv, D = 256, page 816).
"""

from __future__ import annotations

import math
from types import SimpleNamespace

import pytest
import torch

import vllm_stub
from cases import Batch, Case, assert_parity, compare, oracle_of
from pth_flash_attn.cache import build_cache, make_queries

pytestmark = pytest.mark.gpu

DEV = "cuda"
KV_DTYPE = "int8_per_token_head"
MAX_SEQS = 6
GEOMETRIES = [(32, 8, 128, 16), (12, 2, 256, 816)]
GEO_IDS = ["32q8kv-d128-p16", "12q2kv-d256-p816"]
MIXED_Q = [4, 4, 1, 300, 20]
MIXED_L = [3000, 5000, 100, 2000, 400]


@pytest.fixture(scope="module")
def vb():
    if not torch.cuda.is_available():
        pytest.fail("no GPU visible")
    with vllm_stub.installed():
        import pth_flash_attn.vllm_backend as mod

        yield mod


@pytest.fixture
def workspace(vb):
    mgr = vllm_stub.init_workspace_manager(DEV)
    yield mgr
    vllm_stub.reset_workspace_manager()


def make_config(Hq: int, k: int = 3) -> SimpleNamespace:
    return SimpleNamespace(
        model_config=SimpleNamespace(rswa_window=None, get_num_attention_heads=lambda pc: Hq),
        parallel_config=SimpleNamespace(use_ubatching=False, num_ubatches=1),
        scheduler_config=SimpleNamespace(max_num_seqs=MAX_SEQS),
        speculative_config=SimpleNamespace(num_speculative_tokens=k),
        compilation_config=SimpleNamespace(static_forward_context={}),
    )


def packed(cache, Hkv: int, D: int, BS: int) -> torch.Tensor:
    """vLLM's packed layer cache [blocks, kv_heads, block_size, 2 (D + 4)]
    over the HND storage the cache was built in."""
    C = 2 * (D + 4)
    return torch.as_strided(cache.storage, (cache.num_blocks, Hkv, BS, C),
                            (cache.page_bytes, BS * C, C, 1), cache.storage.storage_offset())


def device_cam(q_lens, seq_lens, cache):
    qsl = torch.tensor([0, *torch.tensor(q_lens).cumsum(0).tolist()], dtype=torch.int32)
    T = int(qsl[-1])
    return vllm_stub.CommonAttentionMetadata(
        query_start_loc=qsl.to(DEV), query_start_loc_cpu=qsl,
        seq_lens=cache.seq_lens, num_reqs=len(q_lens), num_actual_tokens=T,
        max_query_len=max(q_lens), max_seq_len=max(seq_lens),
        block_table_tensor=cache.block_table,
        slot_mapping=torch.zeros(T, dtype=torch.int64, device=DEV))


def setup(vb, geo, q_lens, seq_lens, seed):
    Hq, Hkv, D, BS = geo
    cfg = make_config(Hq)
    with vllm_stub.current_config(cfg):
        impl = vb.PthFlashAttnImpl(num_heads=Hq, head_size=D, scale=D ** -0.5,
                                   num_kv_heads=Hkv, alibi_slopes=None, sliding_window=None,
                                   kv_cache_dtype=KV_DTYPE)
    assert impl._ws_token_splits > 0, "the Impl reserved no workspace"
    spec = vllm_stub.AttentionSpec(num_kv_heads=Hkv, head_size=D)
    builder = vb.PthFlashAttnMetadataBuilder(spec, ["layers.3.attn"], cfg, torch.device(DEV))
    cache = build_cache(seq_lens, Hkv=Hkv, D=D, block_size=BS, seed=seed, device=DEV,
                        layout="HND")
    q, qsl = make_queries(q_lens, Hq=Hq, D=D, seed=seed + 1, device=DEV)
    return impl, builder, cache, q, qsl, packed(cache, Hkv, D, BS)


def check_oracle(name, geo, q_lens, seq_lens, cache, q, qsl, out):
    Hq, Hkv, D, BS = geo
    case = Case(name, q_lens=list(q_lens), seq_lens=list(seq_lens), Hq=Hq, Hkv=Hkv, D=D,
                block_size=BS, layout="HND")
    ref_out, ref_lse, valid = oracle_of(Batch(case, cache, q, qsl))
    res = compare(out, None, ref_out, ref_lse, valid)
    print(f"  {name} oracle: {res}", flush=True)
    assert_parity(res, name=name, strict=False)


@pytest.mark.parametrize("geo", GEOMETRIES, ids=GEO_IDS)
def test_mixed_batch_matches_the_oracle(vb, workspace, geo):
    print(f"impl mixed {geo}", flush=True)
    impl, builder, cache, q, qsl, kv = setup(vb, geo, MIXED_Q, MIXED_L, seed=3)
    step = builder.build(0, device_cam(MIXED_Q, MIXED_L, cache))
    assert step.decode is not None and step.prefill is not None
    assert step.decode.plan.num_splits > 1  # the decode slice uses the workspace
    out = torch.full_like(q, float("nan"))
    assert impl.forward(None, q, None, None, kv, step, out) is out
    torch.cuda.synchronize()
    assert not torch.isnan(out.float()).any(), "a row was not written"
    check_oracle(f"impl-mixed-{geo[2]}", geo, MIXED_Q, MIXED_L, cache, q, qsl, out)


@pytest.mark.parametrize("geo", GEOMETRIES, ids=GEO_IDS)
def test_build_and_forward_make_no_host_sync_and_allocate_nothing(vb, workspace, geo):
    print(f"impl no-sync {geo}", flush=True)
    impl, builder, cache, q, qsl, kv = setup(vb, geo, MIXED_Q, MIXED_L, seed=5)
    cam = device_cam(MIXED_Q, MIXED_L, cache)
    out = torch.empty_like(q)
    impl.forward(None, q, None, None, kv, builder.build(0, cam), out)  # warm
    torch.cuda.synchronize()
    workspace.lock()
    buf = workspace.buffer
    ptr, size = buf.data_ptr(), buf.numel()
    before = torch.cuda.memory_allocated()
    torch.cuda.set_sync_debug_mode("error")
    try:
        step = builder.build(0, cam)
        for _ in range(3):
            impl.forward(None, q, None, None, kv, step, out)
    finally:
        torch.cuda.set_sync_debug_mode("default")
    torch.cuda.synchronize()
    assert torch.cuda.memory_allocated() == before
    assert (workspace.buffer.data_ptr(), workspace.buffer.numel()) == (ptr, size)
    check_oracle(f"impl-nosync-{geo[2]}", geo, MIXED_Q, MIXED_L, cache, q, qsl, out)


@pytest.mark.parametrize("geo", GEOMETRIES, ids=GEO_IDS)
def test_uniform_verify_graph_replay_equals_eager(vb, workspace, geo):
    """Capture the Impl for two MTP verifies; replay after seq_lens changed
    on the device, each replay against an eager call (eager work and a
    synchronisation between replays)."""
    print(f"impl graph {geo}", flush=True)
    q_lens, seq_lens = [4, 4], [30000, 20000]
    impl, builder, cache, q, qsl, kv = setup(vb, geo, q_lens, seq_lens, seed=7)
    workspace.lock()
    cam = device_cam(q_lens, seq_lens, cache)
    step = builder.build(0, cam)
    assert step.prefill is None and step.decode.plan.num_splits > 1
    out_graph = torch.zeros_like(q)
    out_eager = torch.zeros_like(q)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        impl.forward(None, q, None, None, kv, step, out_graph)  # warm-up
    stream.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        impl.forward(None, q, None, None, kv, step, out_graph)
    base = cam.seq_lens.clone()
    for i, new in enumerate((base, base // 3, base - 100, base)):
        cam.seq_lens.copy_(new)
        out_graph.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        impl.forward(None, q, None, None, kv, step, out_eager)
        torch.cuda.synchronize()
        assert not torch.isnan(out_graph.float()).any()
        assert torch.equal(out_graph.view(torch.int16), out_eager.view(torch.int16)), f"replay {i}"
    # The last replay ran on the original lengths: check it against the oracle.
    check_oracle(f"impl-graph-{geo[2]}", geo, q_lens, seq_lens, cache, q, qsl, out_graph)
    del graph
    torch.cuda.synchronize()
    assert math.isfinite(float(out_graph.float().abs().max()))
