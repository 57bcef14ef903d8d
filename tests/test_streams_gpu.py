"""Concurrent launches of the op on several HIP streams.

The library keeps no device state between launches outside the caller's
tensors: the split partition, the split-count markers and the partials live
in each launch's own workspace, and the kernels read the lengths from the
launch's own ``seq_lens`` / ``query_start_loc``. So launches of different
batches, each with its own workspace and output, may run at the same time
on different streams (vLLM's separate prefill and decode streams, two
models in one process) and must give exactly what each gives alone. The
cases cover the page-row kernel with splits and the combine, the
register-load kernel for a window, and the row-block kernel (one split);
each is run alone first (and checked against the fp64 oracle), then all of them are enqueued on three streams at
once, several times and in changing order, and every output must equal its
serial one byte for byte.
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
Hq, Hkv, D = 32, 8, 128

# (name, q_lens, seq_lens, prefill plan, window, num_splits (None: the
# planner's; 1: a single-split launch, which runs the row-block kernel))
STREAM_CASES = [
    ("decode-split", [1] * 12, [977, 4096, 15000, 33, 2049, 8191, 600, 12000, 7, 3000, 5000, 64],
     False, 0, None),
    ("verify-window", [16, 16, 16], [5000, 3000, 2100], False, 2048, None),
    ("prefill-rows", [300, 40, 1, 1], [2000, 1000, 4000, 700], True, 0, 1),
]


class _Launch:
    def __init__(self, name, q_lens, seq_lens, prefill, window, S_force, seed):
        self.name = name
        self.case = Case(name, q_lens=list(q_lens), seq_lens=list(seq_lens), Hq=Hq, Hkv=Hkv,
                         window=window)
        self.cache = build_cache(seq_lens, Hkv=Hkv, D=D, block_size=16, seed=seed, device=DEV)
        self.q, self.qsl = make_queries(q_lens, Hq=Hq, D=D, seed=seed + 1, device=DEV)
        T, R, max_q = self.q.shape[0], len(q_lens), max(q_lens)
        w_ts = planner.workspace_token_splits(max_num_seqs=R, q_dec_max=1 if prefill else max_q,
                                              Hkv=Hkv, D=D, num_sms=CUS)
        plan = planner.plan_launch(num_tokens=T, num_reqs=R, max_query_len=max_q, G=Hq // Hkv,
                                   Hkv=Hkv, D=D, num_sms=CUS, is_prefill=prefill,
                                   ws_token_splits=max(w_ts, T), window=window)
        self.max_q, self.wm, self.window = max_q, plan.wm, window
        self.S = plan.num_splits if S_force is None else S_force
        self.ws_o = torch.empty((self.S, T, Hq, D) if self.S > 1 else (0,), device=DEV)
        self.ws_lse = torch.empty((self.S, T, Hq) if self.S > 1 else (0,), device=DEV)
        self.out = torch.empty_like(self.q)

    def run(self):
        c = self.cache
        ops.pth_flash_attn_fwd(self.out, self.q, c.k_cache, c.v_cache, c.k_scale, c.v_scale,
                               c.block_table, c.seq_lens, self.qsl, self.max_q, self.wm, self.S,
                               1.0 / math.sqrt(D), self.ws_o, self.ws_lse, self.window, True)


def test_concurrent_streams_equal_serial():
    if not torch.cuda.is_available():
        pytest.fail("no GPU visible")
    launches = [_Launch(*c, seed=300 + 10 * i) for i, c in enumerate(STREAM_CASES)]
    assert [x.S > 1 for x in launches] == [True, True, False], [x.S for x in launches]
    serial = []
    for x in launches:
        print(f"serial {x.name}: S {x.S} wm {x.wm}", flush=True)
        x.out.fill_(float("nan"))
        x.run()
        torch.cuda.synchronize()
        ref_out, ref_lse, valid = oracle_of(Batch(x.case, x.cache, x.q, x.qsl))
        res = compare(x.out, None, ref_out, ref_lse, valid)
        print(f"  oracle: {res}", flush=True)
        assert_parity(res, name=f"streams {x.name}", strict=False)
        serial.append(x.out.clone())

    streams = [torch.cuda.Stream() for _ in launches]
    main = torch.cuda.current_stream()
    for rep in range(4):
        order = list(range(len(launches)))
        order = order[rep % len(order):] + order[:rep % len(order)]
        print(f"concurrent round {rep}: order {[launches[i].name for i in order]}", flush=True)
        for x in launches:
            x.out.fill_(float("nan"))
            x.ws_o.fill_(float("nan"))
            x.ws_lse.fill_(float("nan"))
        for s in streams:
            s.wait_stream(main)
        # Each stream gets its launch twice in a row, so launches on
        # different streams overlap for longer than one kernel.
        for _ in range(2):
            for i in order:
                with torch.cuda.stream(streams[i]):
                    launches[i].run()
        for s in streams:
            main.wait_stream(s)
        torch.cuda.synchronize()
        for x, ref in zip(launches, serial):
            assert torch.equal(x.out.view(torch.int16), ref.view(torch.int16)), \
                f"round {rep}: {x.name} differs from its serial launch"
