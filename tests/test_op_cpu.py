"""The torch op's interface on the CPU: schema, fake kernel and the C++
metadata checks (no GPU).

The op is a drop-in for the reference's ``pth_flash_attn_fwd``: the schema
string is the reference's (csrc/pth_attn/torch_bindings.cpp:22-26,
python/pth_flash_attn/ops.py:51-55) and each invalid argument fails with the
reference's message (reference tests/cpu/test_ops_fake.py:166-338 lists the
cases; the messages are part of the interface). The fake kernel (used under
torch.compile) and the C++ checks (run by the CPU registration, which then
refuses to compute) must agree case by case.
"""

from __future__ import annotations

from typing import Any, Callable

import pytest
import torch
from torch._subclasses.fake_tensor import FakeTensorMode

from pth_flash_attn import ops
from pth_flash_attn.planner import plan_launch, workspace_token_splits

REFERENCE_SCHEMA = (
    "pth_flash_attn_fwd(Tensor! out, Tensor q, Tensor k_cache, Tensor v_cache, "
    "Tensor k_scale, Tensor v_scale, Tensor block_table, Tensor seq_lens, "
    "Tensor query_start_loc, int max_query_len, int wm, int num_splits, "
    "float softmax_scale, Tensor! ws_o, Tensor! ws_lse, int window=0, "
    "bool causal=True) -> ()"
)
CPU_REFUSAL = "computes on CUDA tensors only"
NEEDS_D128 = "sliding-window and non-causal attention need head size D = 128"
needs_op = pytest.mark.skipif(not ops.is_available(), reason="_C.so not built")

ARG_NAMES = [a.name for a in torch._C.parse_schema(ops.OP_SCHEMA).arguments]
NUM_SMS = 68  # keeps the split count (and the workspace) small on the CPU


def make_args(*, reqs=2, q_len=4, G=6, Hkv=2, D=256, num_blocks=4, block_size=16,
              num_splits=None, window=0, causal=True) -> dict[str, Any]:
    """Valid CPU arguments: strided views into one packed int8 cell buffer
    [K D | ks f32 | V D | vs f32] per (block, slot, head), as vLLM lays it out."""
    cell = torch.zeros(num_blocks, block_size, Hkv, 2 * D + 8, dtype=torch.int8)
    T = reqs * q_len
    ws = workspace_token_splits(max_num_seqs=reqs, q_dec_max=q_len, Hkv=Hkv, D=D,
                                num_sms=NUM_SMS)
    plan = plan_launch(num_tokens=T, num_reqs=reqs, max_query_len=q_len, G=G, Hkv=Hkv, D=D,
                       num_sms=NUM_SMS, is_prefill=False, ws_token_splits=ws, window=window)
    S = plan.num_splits if num_splits is None else num_splits
    ws_t = S if S > 1 else 0
    args = {
        "out": torch.zeros(T, G * Hkv, D, dtype=torch.bfloat16),
        "q": torch.zeros(T, G * Hkv, D, dtype=torch.bfloat16),
        "k_cache": cell[..., :D],
        "v_cache": cell[..., D + 4:2 * D + 4],
        "k_scale": cell[..., D:D + 4].view(torch.float32)[..., 0],
        "v_scale": cell[..., 2 * D + 4:].view(torch.float32)[..., 0],
        "block_table": torch.zeros(reqs, num_blocks, dtype=torch.int32),
        "seq_lens": torch.full((reqs,), q_len, dtype=torch.int32),
        "query_start_loc": torch.arange(0, T + 1, q_len, dtype=torch.int32),
        "max_query_len": q_len,
        "wm": plan.wm,
        "num_splits": S,
        "softmax_scale": D ** -0.5,
        "ws_o": torch.empty(ws_t, T, G * Hkv, D, dtype=torch.float32),
        "ws_lse": torch.empty(ws_t, T, G * Hkv, dtype=torch.float32),
        "window": window,
        "causal": causal,
    }
    assert list(args) == ARG_NAMES
    return args


S_DEFAULT = make_args()["num_splits"]


def _with(**over) -> Callable[[], dict[str, Any]]:
    return lambda: {**make_args(), **over}


def _q_out(shape, dtype=torch.bfloat16) -> dict:
    return {"q": torch.zeros(shape, dtype=dtype), "out": torch.zeros(shape, dtype=dtype)}


DRAFTER = {"D": 128, "G": 4, "q_len": 8, "window": 2048, "causal": False}

CASES: list[tuple[str, Callable[[], dict], str | None]] = [
    ("valid_split", make_args, None),
    ("valid_s1_empty_ws", lambda: make_args(num_splits=1), None),
    ("q_rank", _with(q=torch.zeros(8, 3072, dtype=torch.bfloat16)), "q must be 3-D, got 2-D"),
    ("q_dtype", _with(**_q_out((8, 12, 256), torch.float32)),
     "q must be bfloat16 or float16, got float32"),
    ("head_size", _with(**_q_out((8, 12, 96))),
     "head size D = q.size(2) must be 64, 128 or 256, got 96"),
    ("q_inner_stride", _with(q=torch.zeros(8, 12, 512, dtype=torch.bfloat16)[..., ::2]),
     "q must have stride 1 in its last dimension, got 2"),
    ("out_dtype", _with(out=torch.zeros(8, 12, 256, dtype=torch.float16)),
     "out (same dtype as q) must be bfloat16, got float16"),
    ("out_tokens", _with(out=torch.zeros(7, 12, 256, dtype=torch.bfloat16)),
     "out.size(0) must equal T = 8, got 7"),
    ("k_cache_dtype", _with(k_cache=torch.zeros(4, 16, 2, 256, dtype=torch.uint8)),
     "k_cache must be int8, got an unsupported dtype"),
    ("k_cache_head_size", _with(k_cache=torch.zeros(4, 16, 2, 128, dtype=torch.int8)),
     "k_cache.size(3) must equal D = 256, got 128"),
    ("v_cache_blocks", _with(v_cache=torch.zeros(3, 16, 2, 256, dtype=torch.int8)),
     "v_cache.size(0) must equal NB = 4, got 3"),
    ("k_scale_dtype", _with(k_scale=torch.zeros(4, 16, 2, dtype=torch.float16)),
     "k_scale must be float32, got float16"),
    ("v_scale_block_size", _with(v_scale=torch.zeros(4, 8, 2)),
     "v_scale.size(1) must equal BS = 16, got 8"),
    ("hq_not_multiple", _with(**_q_out((8, 13, 256))),
     "Hq = 13 must be a positive multiple of Hkv = 2"),
    ("wm_value", _with(wm=3), "wm must be 1, 2 or 4, got 3"),
    ("group_over_64", _with(**_q_out((8, 130, 256)), wm=4,
                            ws_o=torch.empty(S_DEFAULT, 8, 130, 256),
                            ws_lse=torch.empty(S_DEFAULT, 8, 130)),
     "G = Hq/Hkv = 65 exceeds the supported maximum 64"),
    ("group_over_16wm", _with(**_q_out((8, 48, 256)), wm=1),
     "G = Hq/Hkv = 24 must be <= 16*wm = 16"),
    ("block_table_dtype", _with(block_table=torch.zeros(2, 4, dtype=torch.int64)),
     "block_table must be int32, got int64"),
    ("seq_lens_rank", _with(seq_lens=torch.zeros(2, 1, dtype=torch.int32)),
     "seq_lens must be 1-D, got 2-D"),
    ("qsl_length", _with(query_start_loc=torch.zeros(4, dtype=torch.int32)),
     "query_start_loc.size(0) must equal num_reqs + 1 = 3, got 4"),
    ("block_table_rows", _with(block_table=torch.zeros(1, 4, dtype=torch.int32)),
     "block_table has 1 rows, fewer than num_reqs = 2"),
    ("max_query_len", _with(max_query_len=9), "max_query_len must be in [0, T = 8], got 9"),
    ("num_splits_zero", _with(num_splits=0), "num_splits must be >= 1, got 0"),
    ("scale_nan", _with(softmax_scale=float("nan")),
     "softmax_scale must be finite and > 0, got nan"),
    ("scale_negative", _with(softmax_scale=-1.0), "softmax_scale must be finite and > 0, got -1"),
    ("scale_zero", _with(softmax_scale=0.0), "softmax_scale must be finite and > 0, got 0"),
    ("ws_o_too_few_splits", _with(ws_o=torch.empty(S_DEFAULT - 1, 8, 12, 256)),
     f"ws_o must have size(0) >= num_splits = {S_DEFAULT} and size(1) >= T = 8, "
     f"got [{S_DEFAULT - 1}, 8, ...]"),
    ("ws_o_dtype", _with(ws_o=torch.empty(S_DEFAULT, 8, 12, 256, dtype=torch.bfloat16)),
     "ws_o must be float32, got bfloat16"),
    ("ws_lse_heads", _with(ws_lse=torch.empty(S_DEFAULT, 8, 6)),
     "ws_lse.size(2) must equal Hq = 12, got 6"),
    ("window_negative", _with(window=-1), "window must be >= 0, got -1"),
    ("window_at_d256", _with(window=2048), f"{NEEDS_D128}, got 256"),
    ("non_causal_at_d256", _with(causal=False), f"{NEEDS_D128}, got 256"),
    ("window_at_d64", lambda: make_args(D=64, G=4, Hkv=2, window=64), f"{NEEDS_D128}, got 64"),
    ("non_causal_at_d64", lambda: make_args(D=64, G=4, Hkv=2, causal=False),
     f"{NEEDS_D128}, got 64"),
    ("valid_drafter_tp2", lambda: make_args(**DRAFTER, Hkv=4), None),
    ("valid_drafter_tp1", lambda: make_args(**DRAFTER, Hkv=8), None),
    ("valid_causal_window_d128", lambda: make_args(D=128, G=4, Hkv=2, window=64), None),
    ("valid_non_causal_d128", lambda: make_args(D=128, G=4, Hkv=2, causal=False), None),
    ("valid_causal_d64", lambda: make_args(D=64, G=4, Hkv=2), None),
]


def _fake_error(args: dict) -> str | None:
    with FakeTensorMode() as mode:
        fa = [mode.from_tensor(v) if isinstance(v, torch.Tensor) else v for v in args.values()]
        try:
            res = ops.pth_flash_attn_fwd_fake(*fa)
        except RuntimeError as e:
            return str(e)
    assert res is None
    return None


def test_schema_is_the_reference_schema():
    canon = lambda s: str(torch._C.parse_schema("pth_flash_attn::" + s))  # noqa: E731
    assert canon(ops.OP_SCHEMA) == canon(REFERENCE_SCHEMA)


@needs_op
def test_loaded_op_has_the_schema():
    op = torch.ops.pth_flash_attn.pth_flash_attn_fwd.default
    assert str(op._schema) == str(torch._C.parse_schema("pth_flash_attn::" + REFERENCE_SCHEMA))


@pytest.mark.parametrize(("case", "build", "expected"), CASES, ids=[c[0] for c in CASES])
def test_fake_checks(case, build, expected):
    err = _fake_error(build())
    if expected is None:
        assert err is None, err
    else:
        assert err is not None and expected in err, (case, err)


@needs_op
@pytest.mark.parametrize(("case", "build", "expected"), CASES, ids=[c[0] for c in CASES])
def test_cpp_checks_match_fake(case, build, expected):
    """The C++ op on CPU tensors: the same message as the fake for invalid
    arguments, the CPU refusal for valid ones."""
    args = build()
    with pytest.raises(RuntimeError) as ei:
        torch.ops.pth_flash_attn.pth_flash_attn_fwd(*args.values())
    msg = str(ei.value)
    if expected is None:
        assert CPU_REFUSAL in msg, msg
    else:
        assert expected in msg, (case, msg)
        fake = _fake_error(args)
        assert fake is not None and fake.split("\n")[0] in msg


@needs_op
def test_legacy_15_argument_call_is_causal_without_window():
    """The reference's original schema had no window/causal; the defaults keep
    such calls valid."""
    args = make_args(D=128, G=4, Hkv=2)
    legacy = list(args.values())[:15]
    with pytest.raises(RuntimeError, match=CPU_REFUSAL):
        torch.ops.pth_flash_attn.pth_flash_attn_fwd(*legacy)


def test_wrapper_fails_loudly_without_gpu():
    """The Python wrapper has no CPU compute path: CPU tensors raise."""
    args = make_args(D=128, G=4, Hkv=2)
    with pytest.raises(RuntimeError):
        ops.pth_flash_attn_fwd(**args)
