"""HIP-graph replay, torch.library.opcheck and torch.compile of the op on the GPU.

vLLM captures one graph per padded batch shape and replays it while the
sequence lengths grow on the device (reference tests/gpu/test_graph_replay.py,
test_attn_graph.py). The launch must therefore read ``seq_lens`` and
``query_start_loc`` from device memory on every replay and bake no length
into its grid or arguments. Each case here captures the op once, then
replays it after rewriting ``seq_lens`` / ``query_start_loc`` in place
(lengths across page and chunk edges, a shrink, an empty request). After
every replay the valid rows must equal an eager launch on the same device
contents byte for byte (the kernels are deterministic), with eager work and
synchronisations between replays. Selected steps are also checked against
the fp64 oracle. The negative control: the lengths do change the output.

The op launches no memset, so the graph holds kernels only.
"""

from __future__ import annotations

import math

import pytest
import torch

from cases import Batch, Case, assert_parity, compare, oracle_of
from pth_flash_attn import ops, planner
from pth_flash_attn.cache import build_cache, make_queries

pytestmark = pytest.mark.gpu

DEV = "cuda"
CUS = 256

# (name, capacity q_lens, capacity seq_lens, steps of (q_lens, seq_lens),
#  num_splits (None: the planner's), prefill plan, window, causal)
GRAPH_CASES = [
    ("decode-split", (1, 1), (4096, 817),
     [((1, 1), (815, 1)), ((1, 1), (816, 64)), ((1, 1), (817, 65)), ((1, 1), (4096, 817)),
      ((1, 1), (65, 16)), ((1, 0), (1000, 0))], None, False, 0, True),
    ("decode-s1", (1, 1), (4096, 817),
     [((1, 1), (815, 1)), ((1, 1), (4096, 817)), ((1, 1), (65, 16)), ((1, 0), (1000, 0))],
     1, False, 0, True),
    ("verify-window", (16, 16), (5000, 3000),
     [((16, 16), (5000, 3000)), ((16, 16), (2100, 16)), ((16, 3), (4000, 2049))],
     None, False, 2048, True),
    ("prefill-rows", (300, 40), (2000, 1000),
     [((300, 40), (2000, 1000)), ((64, 40), (64, 41)), ((1, 33), (700, 999)),
      ((300, 0), (301, 0))], 1, True, 0, True),
]


def _run_op(out, q, cache, seq_lens, qsl, max_q, wm, S, ws_o, ws_lse, window, causal):
    ops.pth_flash_attn_fwd(out, q, cache.k_cache, cache.v_cache, cache.k_scale, cache.v_scale,
                           cache.block_table, seq_lens, qsl, max_q, wm, S,
                           1.0 / math.sqrt(128), ws_o, ws_lse, window, causal)


@pytest.mark.parametrize("name,cap_q,cap_l,steps,S_force,prefill,window,causal", GRAPH_CASES,
                         ids=[c[0] for c in GRAPH_CASES])
def test_graph_replay_equals_eager_with_changing_lengths(name, cap_q, cap_l, steps, S_force,
                                                         prefill, window, causal):
    if not torch.cuda.is_available():
        pytest.fail("no GPU visible")
    print(f"graph case {name}: capacity q {cap_q} L {cap_l} window {window}", flush=True)
    Hq, Hkv, D = 32, 8, 128
    pad_rows = 2
    cache = build_cache(list(cap_l), Hkv=Hkv, D=D, block_size=16, seed=77, device=DEV)
    q, qsl = make_queries(list(cap_q), Hq=Hq, D=D, seed=78, device=DEV)
    q = torch.cat([q, torch.zeros(pad_rows, Hq, D, dtype=q.dtype, device=DEV)])
    T, R, max_q = q.shape[0], len(cap_q), max(cap_q)
    w_ts = planner.workspace_token_splits(max_num_seqs=R, q_dec_max=1 if prefill else max_q,
                                          Hkv=Hkv, D=D, num_sms=CUS)
    # Planned for the real tokens (the planner refuses padding rows), launched
    # over all T rows.
    plan = planner.plan_launch(num_tokens=min(T, R * max_q), num_reqs=R, max_query_len=max_q,
                               G=Hq // Hkv, Hkv=Hkv, D=D, num_sms=CUS, is_prefill=prefill,
                               ws_token_splits=max(w_ts, T), window=window)
    S = plan.num_splits if S_force is None else S_force
    ws_o = torch.empty((S, T, Hq, D) if S > 1 else (0,), device=DEV)
    ws_lse = torch.empty((S, T, Hq) if S > 1 else (0,), device=DEV)
    ws_oe = torch.empty_like(ws_o)
    ws_le = torch.empty_like(ws_lse)
    seq_lens = cache.seq_lens  # rewritten in place below
    out_g = torch.zeros_like(q)

    args = (q, cache, seq_lens, qsl, max_q, plan.wm, S)
    # Warm up on a side stream, as torch's graph capture requires.
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        _run_op(out_g, *args, ws_o, ws_lse, window, causal)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        _run_op(out_g, *args, ws_o, ws_lse, window, causal)
    torch.cuda.synchronize()

    previous = None
    for i, (q_lens, lens) in enumerate(steps):
        starts = [0]
        for n in q_lens:
            starts.append(starts[-1] + n)
        seq_lens.copy_(torch.tensor(lens, dtype=torch.int32))
        qsl.copy_(torch.tensor(starts, dtype=torch.int32))
        # Eager work of the program's own between replays.
        junk = torch.randn(512, 512, device=DEV)
        (junk @ junk).sum().item()
        g.replay()
        torch.cuda.synchronize()
        out_e = torch.full_like(q, float("nan"))
        _run_op(out_e, *args, ws_oe, ws_le, window, causal)
        torch.cuda.synchronize()
        n_valid = starts[-1]
        print(f"  step {i}: q_lens {q_lens} seq_lens {lens}", flush=True)
        assert torch.equal(out_g[:n_valid].view(torch.int16), out_e[:n_valid].view(torch.int16)), \
            f"{name} step {i}: replay differs from eager"
        if i in (0, len(steps) - 1):
            case = Case(f"{name}-{i}", q_lens=list(q_lens), seq_lens=list(lens), Hq=Hq, Hkv=Hkv,
                        window=window, causal=causal)
            ref_out, ref_lse, valid = oracle_of(Batch(case, cache, q[:n_valid], qsl))
            res = compare(out_g[:n_valid], None, ref_out, ref_lse, valid)
            print(f"    oracle: {res}", flush=True)
            assert_parity(res, name=f"{name} step {i}", strict=False)
        if previous is not None and previous[0] == n_valid and n_valid > 0:
            # Negative control: different lengths give a different output.
            assert not torch.equal(out_g[:n_valid], previous[1]), f"{name} step {i}: lengths ignored"
        previous = (n_valid, out_g[:n_valid].clone())


def _small_call(device: str):
    Hq, Hkv, D = 8, 2, 128
    cache = build_cache([300, 77], Hkv=Hkv, D=D, block_size=16, seed=5, device=device)
    q, qsl = make_queries([4, 1], Hq=Hq, D=D, seed=6, device=device)
    T = q.shape[0]
    S = 3
    return (torch.zeros_like(q), q, cache.k_cache, cache.v_cache, cache.k_scale, cache.v_scale,
            cache.block_table, cache.seq_lens, qsl, 4, 1, S, 1.0 / math.sqrt(D),
            torch.empty(S, T, Hq, D, device=device), torch.empty(S, T, Hq, device=device), 0,
            True)


def test_opcheck():
    """torch.library.opcheck: schema, fake tensor, autograd registration and
    AOT dispatch checks of the registered op on GPU tensors."""
    if not torch.cuda.is_available():
        pytest.fail("no GPU visible")
    args = _small_call(DEV)
    torch.library.opcheck(torch.ops.pth_flash_attn.pth_flash_attn_fwd.default, args)


def test_torch_compile_fullgraph_equals_eager():
    """The op traced by dynamo (its fake kernel gives the meta behaviour) and
    run through AOT autograd equals the eager call bitwise."""
    if not torch.cuda.is_available():
        pytest.fail("no GPU visible")
    args = _small_call(DEV)
    out_c = args[0]
    out_e = torch.zeros_like(out_c)

    def f(out, *rest):
        torch.ops.pth_flash_attn.pth_flash_attn_fwd(out, *rest)
        return out

    compiled = torch.compile(f, backend="aot_eager", fullgraph=True)
    compiled(*args)
    f(out_e, *args[1:])
    torch.cuda.synchronize()
    assert torch.equal(out_c.view(torch.int16), out_e.view(torch.int16))
