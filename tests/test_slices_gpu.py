"""The vLLM backend's forward on the GPU: a step's decode and prefill slices
(``slices.SliceBuilder`` + ``slices.run_slices``) reading vLLM's packed layer
cache through ``cache.vllm_packed_views``, against the fp64 oracle.

Mirrors the reference's backend Impl tests (reference
tests/gpu/test_backend_impl.py:129-147 mixed batch against the fp64
reference; tests/gpu/test_backend_impl_window.py the drafter's windowed
non-causal layer), without vLLM: the builder gets the step's device tensors
directly and the workspace is one reserved buffer handed out as views, as
vLLM's workspace manager does.
"""

from __future__ import annotations

import math

import pytest
import torch

from cases import Batch, Case, assert_parity, compare, oracle_of
from pth_flash_attn import planner, slices
from pth_flash_attn.cache import build_cache, make_queries, vllm_packed_views

pytestmark = pytest.mark.gpu

DEV = "cuda"
CUS = 256

# (name, Hq, Hkv, D, k (speculative tokens), window, causal, q_lens, seq_lens)
STEPS = [
    ("mixed-d128", 32, 8, 128, 3, 0, True, [1, 4, 4, 1, 300, 77], [2000, 517, 4096, 33, 700, 900]),
    ("mixed-d256-g6", 12, 2, 256, 3, 0, True, [4, 4, 1, 180], [5000, 3000, 64, 400]),
    ("mixed-d64", 16, 4, 64, 0, 0, True, [1, 1, 1, 120], [3000, 65, 1, 500]),
    ("drafter-window", 16, 4, 128, 7, 2048, False, [8, 8, 8], [9000, 2100, 8]),
    ("decode-only-long", 32, 8, 128, 0, 0, True, [1, 1], [40000, 17]),
]


# Bits of a quiet NaN that no kernel writes: every float of the reserved
# buffer starts with it, and those outside the views the launches were given
# (the reservation's unused tail and a guard after each region) must keep it.
CANARY = 0x7FBADBAD
GUARD = 4096  # floats after each region


def _workspace(builder: slices.SliceBuilder, Hq: int, D: int):
    """The reservation the builder sized (o partials, guard, LSE partials,
    guard), handed out as views from the start of each region, as vLLM's
    workspace manager does; returns (provide, asked, check)."""
    o_shape, lse_shape = planner.workspace_shapes(ws_token_splits=builder.ws_token_splits, Hq=Hq, D=D)
    n_o, n_l = math.prod(o_shape), math.prod(lse_shape)
    l0 = n_o + GUARD
    buf = torch.full((l0 + n_l + GUARD,), CANARY, dtype=torch.int32, device=DEV).view(torch.float32)
    asked = []

    def provide(o, lse):
        asked.append((o, lse))
        no, nl = math.prod(o), math.prod(lse)
        assert no <= n_o and nl <= n_l, "launch beyond the reservation"
        return buf[:no].view(o), buf[l0:l0 + nl].view(lse)

    def check():
        """Floats outside every view handed out still hold the canary."""
        used_o = max((math.prod(o) for o, _ in asked), default=0)
        used_l = max((math.prod(lse) for _, lse in asked), default=0)
        bits = buf.view(torch.int32)
        for lo, hi in ((used_o, l0), (l0 + used_l, bits.numel())):
            bad = int((bits[lo:hi] != CANARY).sum())
            assert bad == 0, f"{bad} floats written outside the workspace views in [{lo}, {hi})"
        return used_o, used_l

    return provide, asked, check


@pytest.mark.parametrize("name,Hq,Hkv,D,k,window,causal,q_lens,seq_lens", STEPS,
                         ids=[s[0] for s in STEPS])
def test_step_slices_match_the_oracle(name, Hq, Hkv, D, k, window, causal, q_lens, seq_lens):
    if not torch.cuda.is_available():
        pytest.fail("no GPU visible")
    print(f"step {name}: q {q_lens} L {seq_lens}", flush=True)
    BS = 16
    cache = build_cache(seq_lens, Hkv=Hkv, D=D, block_size=BS, seed=11, device=DEV, layout="HND")
    C = 2 * (D + 4)
    packed = torch.as_strided(cache.storage, (cache.num_blocks, Hkv, BS, C),
                              (cache.page_bytes, BS * C, C, 1))
    views = vllm_packed_views(packed)
    q, qsl = make_queries(q_lens, Hq=Hq, D=D, seed=12, device=DEV)
    out = torch.full_like(q, float("nan"))

    builder = slices.SliceBuilder(
        num_heads_q=Hq, num_kv_heads=Hkv, head_size=D, window=window,
        max_num_seqs=len(q_lens), q_verify=slices.verify_query_len(k), num_cus=CUS, device=DEV)
    step = builder.build(
        query_start_loc=qsl, query_start_loc_cpu=qsl.cpu(), seq_lens=cache.seq_lens,
        block_table=cache.block_table, num_reqs=len(q_lens), num_actual_tokens=q.shape[0],
        max_query_len=max(q_lens), causal=causal)
    provide, asked, check = _workspace(builder, Hq, D)
    none = torch.empty(0, dtype=torch.float32, device=DEV)
    slices.run_slices(step, query=q, output=out, caches=views, scale=1.0 / math.sqrt(D),
                      window=window, workspace=provide, no_workspace=none,
                      reserved_token_splits=builder.ws_token_splits)
    torch.cuda.synchronize()
    parts = [p for p in (step.decode, step.prefill) if p is not None]
    print(f"  slices: {[(p.token_start, p.token_end, p.plan.num_splits) for p in parts]}", flush=True)
    assert len(parts) >= 1 and not torch.isnan(out.float()).any()
    used = check()
    print(f"  workspace: {used} floats of ({builder.ws_token_splits} token-splits) used, "
          f"canaries intact", flush=True)

    case = Case(name, q_lens=list(q_lens), seq_lens=list(seq_lens), Hq=Hq, Hkv=Hkv, D=D,
                window=window, causal=causal, layout="HND")
    ref_out, ref_lse, valid = oracle_of(Batch(case, cache, q, qsl))
    res = compare(out, None, ref_out, ref_lse, valid)
    print(f"  oracle: {res}", flush=True)
    assert_parity(res, name=name, strict=False)
