"""Determinism under repetition: the same launch many times gives one result.

The kernels hand data between waves through LDS (the page-row and staged
kernels' shared chunk buffers, the row-block kernel's shared conversion and
key-part merge, the combine's cross-wave merge) and between work-groups
through the workspace (split partials and the split-count marker that the
combine reads). A missing barrier or wait shows up as an output that depends
on timing. Each case below is launched LAUNCHES times through the C ABI into
the same buffers; every third launch has a large copy running beside it on
another stream, so the work-groups' timing shifts between launches. Every
output and LSE must equal the first launch's bit for bit (the reference's
determinism stress, tests/gpu/attn_stress.py, runs the same check).
"""

from __future__ import annotations

import pytest
import torch

from cases import Case, launch_args, materialize, tile_tokens, uniform_lengths

pytestmark = pytest.mark.gpu

DEV = "cuda"
LAUNCHES = 120

# (case, forced num_splits or None for the planner's): one per kernel family.
STRESS = [
    (Case("pagerows-decode", q_lens=[1] * 64, seq_lens=uniform_lengths(64, 100, 6000, 90),
          seed=90), None),
    (Case("pagerows-verify4", q_lens=[4] * 8, seq_lens=uniform_lengths(8, 100, 9000, 91),
          seed=91), None),
    (Case("staged-1kv", q_lens=[1], seq_lens=[3000], Hq=4, Hkv=1, seed=92), None),
    (Case("regload-window", q_lens=[16] * 8, seq_lens=uniform_lengths(8, 600, 9000, 93),
          window=512, seed=93), None),
    (Case("rows-wide-and-parts", q_lens=[300, 1, 1, 40], seq_lens=[2000, 5000, 900, 700],
          is_prefill=True, seed=94), 1),
    (Case("paged256-decode", q_lens=[1, 1, 4], seq_lens=[8000, 300, 4000], Hq=12, Hkv=2, D=256,
          seed=95), None),
    (Case("generic-d64", q_lens=[1, 2, 1], seq_lens=[3000, 700, 64], Hq=16, Hkv=4, D=64,
          seed=96), None),
    (Case("combine-many-splits", q_lens=[1], seq_lens=[40000], Hq=8, Hkv=2, seed=97), 300),
]


@pytest.mark.parametrize("case,S_force", STRESS, ids=[c.name for c, _ in STRESS])
def test_repeated_launches_are_bitwise_identical(case, S_force):
    if not torch.cuda.is_available():
        pytest.fail("no GPU visible")
    from pth_flash_attn import capi

    plan = case.plan()
    S = plan.num_splits if S_force is None else S_force
    print(f"stress {case.name}: S={S} wm={plan.wm} launches={LAUNCHES}", flush=True)
    b = materialize(case, DEV)
    T = case.T
    out = torch.empty(b.q.shape, dtype=b.q.dtype, device=DEV)
    lse = torch.empty((T, case.Hq), device=DEV)
    ws_o = torch.empty((S, T, case.Hq, case.D), device=DEV) if S > 1 else None
    ws_lse = torch.empty((S, T, case.Hq), device=DEV) if S > 1 else None
    bq = tile_tokens(plan.wm, case.G, max(case.q_lens))
    args = launch_args(b, out, num_splits=S, bq=bq, ws_o=ws_o, ws_lse=ws_lse)
    lib = capi.AttnLib()
    main = torch.cuda.current_stream()
    side = torch.cuda.Stream()
    big_a = torch.empty(64 << 20, dtype=torch.float32, device=DEV).uniform_()
    big_b = torch.empty_like(big_a)

    first_out = first_lse = None
    differ = 0
    for i in range(LAUNCHES):
        out.fill_(float("nan"))
        lse.fill_(float("nan"))
        if i % 3 == 2:
            side.wait_stream(main)
            with torch.cuda.stream(side):
                big_b.copy_(big_a)  # 512 MB of traffic beside the launch
        lib.check(lib.attention_lse(args, lse, main.cuda_stream))
        if i % 3 == 2:
            main.wait_stream(side)
        if first_out is None:
            torch.cuda.synchronize()
            assert not torch.isnan(out.float()).any(), "first launch left rows unwritten"
            first_out, first_lse = out.clone(), lse.clone()
            continue
        same = torch.equal(out.view(torch.int16), first_out.view(torch.int16)) and \
            torch.equal(lse.view(torch.int32), first_lse.view(torch.int32))
        differ += 0 if same else 1
    torch.cuda.synchronize()
    print(f"  {differ} of {LAUNCHES - 1} repeated launches differ from the first", flush=True)
    assert differ == 0
