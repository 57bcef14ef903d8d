"""Golden vectors written by the reference's own compiled CPU path
(tests/golden/make_golden.py; inputs and the reference's fp32 outputs).

* CPU: the oracle reproduces every vector (the reference computes in fp32,
  so to fp32 accumulation error).
* GPU: the HIP path reproduces every vector through the C ABI, with the
  planner's split count and unsplit, to the parity tolerance on bf16 output
  (beyond bf16 storage rounding) and to 1e-4 on fp32 output (2e-3 for the
  row-block kernel's launches, whose P is fp16).
"""

from __future__ import annotations

import math
from pathlib import Path

import numpy as np
import pytest
import torch

import oracle
from cases import MAX_ABS, MEAN_ABS, half_ulp
from pth_flash_attn import capi, planner
from pth_flash_attn.cache import carve_views

GOLDEN = Path(__file__).resolve().parent / "golden"
NAMES = sorted(p.stem for p in GOLDEN.glob("*.npz"))


def load(name: str, device: str = "cpu") -> dict:
    z = np.load(GOLDEN / f"{name}.npz")  # allow_pickle stays False
    nb, bs, hkv, D, pad, hnd = (int(x) for x in z["geometry"])
    storage = torch.from_numpy(z["storage"].copy()).to(device)
    k, v, ks, vs = carve_views(storage, num_blocks=nb, block_size=bs, Hkv=hkv, D=D,
                               layout="HND" if hnd else "NHD", pad_page_bytes=pad)
    q = torch.from_numpy(z["q_bf16_bits"].copy()).view(torch.bfloat16).to(device)
    return {
        "storage": storage, "k_cache": k, "v_cache": v, "k_scale": ks, "v_scale": vs,
        "block_table": torch.from_numpy(z["block_table"].copy()).to(device),
        "seq_lens": torch.from_numpy(z["seq_lens"].copy()).to(device),
        "qsl": torch.from_numpy(z["query_start_loc"].copy()).to(device),
        "q": q, "window": int(z["window"]), "causal": bool(int(z["causal"])),
        "scale": float(z["softmax_scale"]), "out": z["out"], "Hkv": hkv, "D": D,
    }


def args_of(g: dict, out: torch.Tensor, *, bq: int, S: int, ws_o=None, ws_lse=None):
    return capi.attn_args(q=g["q"], out=out, k_cache=g["k_cache"], v_cache=g["v_cache"],
                          k_scale=g["k_scale"], v_scale=g["v_scale"],
                          block_table=g["block_table"], seq_lens=g["seq_lens"],
                          query_start_loc=g["qsl"], bq=bq, num_splits=S,
                          softmax_scale=g["scale"], ws_o=ws_o, ws_lse=ws_lse,
                          window=g["window"], causal=g["causal"])


def valid_rows(g: dict) -> np.ndarray:
    qsl = g["qsl"].cpu().numpy()
    v = np.zeros(g["q"].shape[0], bool)
    v[qsl[0]:qsl[-1]] = True
    return v


def test_golden_present():
    assert "config1" in NAMES and len(NAMES) >= 5


@pytest.mark.parametrize("name", NAMES)
def test_oracle_reproduces_golden(name):
    g = load(name)
    out = torch.empty(g["q"].shape, dtype=torch.float32)
    ref, _, valid = oracle.attention(args_of(g, out, bq=1, S=1))
    assert np.array_equal(valid, valid_rows(g))
    np.testing.assert_allclose(ref[valid], g["out"][valid], atol=2e-6, rtol=0)


@pytest.mark.gpu
@pytest.mark.parametrize("name", NAMES)
@pytest.mark.parametrize("split", ["planned", "one"])
def test_hip_reproduces_golden(name, split):
    if not torch.cuda.is_available():
        pytest.fail("no GPU visible: the gpu tests need a gfx950 device")
    print(f"golden {name} split={split}", flush=True)
    g = load(name, "cuda")
    T, Hq, D = g["q"].shape
    G = Hq // g["Hkv"]
    qsl = g["qsl"].cpu().tolist()
    q_lens = [b - a for a, b in zip(qsl, qsl[1:])]
    q_max = max(max(q_lens), 1)
    plan = planner.plan_launch(num_tokens=min(T, len(q_lens) * q_max), num_reqs=len(q_lens),
                               max_query_len=q_max, G=G, Hkv=g["Hkv"], D=D, num_sms=256,
                               is_prefill=False, ws_token_splits=1 << 20, window=g["window"])
    S = plan.num_splits if split == "planned" else 1
    valid = valid_rows(g)
    ref = g["out"][valid].astype(np.float64)
    lib = capi.AttnLib()
    stream = torch.cuda.current_stream().cuda_stream
    for dtype in (torch.bfloat16, torch.float32):
        out = torch.full((T, Hq, D), float("nan"), dtype=dtype, device="cuda")
        lse = torch.empty((T, Hq), device="cuda")
        ws_o = torch.empty((S, T, Hq, D), device="cuda") if S > 1 else None
        ws_l = torch.empty((S, T, Hq), device="cuda") if S > 1 else None
        a = args_of(g, out, bq=plan.bq, S=S, ws_o=ws_o, ws_lse=ws_l)
        lib.check(lib.attention_lse(a, lse, stream))
        torch.cuda.synchronize()
        o = out.float().cpu().numpy()[valid].astype(np.float64)
        err = np.abs(o - ref)
        if dtype == torch.float32:
            # Row-block launches keep P in fp16 (the reference's precision
            # class): BASELINE's 2e-3 on the arithmetic alone; 1e-4 otherwise.
            rows_kernel = (D == 128 and S == 1 and g["k_cache"].shape[1] % 16 == 0
                           and plan.bq * G >= 64)
            gate = 2e-3 if rows_kernel else 1e-4
            assert err.max() <= gate, f"{name}: fp32 max abs {err.max():.3g}"
        else:
            ex = np.maximum(err - half_ulp(ref, dtype), 0)
            assert ex.max() <= MAX_ABS and ex.mean() <= MEAN_ABS, (name, ex.max(), ex.mean())
