"""Shared test cases: seeded paged-cache batches, their launch arguments, and
the comparison against the CPU oracle at the parity tolerance.

Parity tolerance (from the path's specification): on bf16 outputs, max abs
error <= 2e-3 and mean abs error <= 2e-4 against the fp64 oracle; natural-log
LSE within 1e-3.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np
import torch

import oracle
from pth_flash_attn import capi, planner
from pth_flash_attn.cache import PagedCache, build_cache, make_queries

MAX_ABS = 2e-3
MEAN_ABS = 2e-4
LSE_ABS = 1e-3
MI355X_CUS = 256


@dataclass
class Case:
    """One batch: query lengths and KV lengths per request plus geometry."""

    name: str
    q_lens: list[int]
    seq_lens: list[int]
    Hq: int = 32
    Hkv: int = 8
    D: int = 128
    block_size: int = 16
    window: int = 0
    causal: bool = True
    layout: str = "NHD"
    q_dtype: torch.dtype = torch.bfloat16
    seed: int = 0
    pad_page_bytes: int = 0
    offset_bytes: int = 0
    pad_tokens: int = 0  # extra rows of q/out beyond qsl[R] (padded graph batch)
    is_prefill: bool | None = None
    num_splits: int | None = None  # override the planner
    extra: dict = field(default_factory=dict)

    @property
    def G(self) -> int:
        return self.Hq // self.Hkv

    @property
    def T(self) -> int:
        return sum(self.q_lens) + self.pad_tokens

    def plan(self, num_sms: int = MI355X_CUS) -> planner.LaunchPlan:
        q_max = max(self.q_lens)
        prefill = self.is_prefill
        if prefill is None:
            prefill = q_max > planner.max_tokens_per_tile(self.G)
        ws = planner.workspace_token_splits(
            max_num_seqs=len(self.q_lens), q_dec_max=max(q_max, 1), Hkv=self.Hkv,
            D=self.D, num_sms=num_sms)
        # A padded batch (pad_tokens) is planned for its real tokens; the
        # launch still covers all T rows.
        p = planner.plan_launch(
            num_tokens=min(self.T, len(self.q_lens) * q_max), num_reqs=len(self.q_lens), max_query_len=q_max, G=self.G,
            Hkv=self.Hkv, D=self.D, num_sms=num_sms, is_prefill=prefill,
            ws_token_splits=max(ws, self.T), window=self.window)
        if self.num_splits is not None:
            import dataclasses
            p = dataclasses.replace(p, num_splits=self.num_splits)
        return p


def tile_tokens(wm: int, G: int, max_query_len: int) -> int:
    """The op's row-tile height rule (torch_op.cpp tile_tokens)."""
    cap = 16 * wm // G
    if 1 <= max_query_len < cap and planner.wm_for_rows(max_query_len * G) == wm:
        return max_query_len
    return cap


@dataclass
class Batch:
    case: Case
    cache: PagedCache
    q: torch.Tensor
    qsl: torch.Tensor


def materialize(case: Case, device: str) -> Batch:
    cache = build_cache(case.seq_lens, Hkv=case.Hkv, D=case.D, block_size=case.block_size,
                        seed=case.seed, device=device, layout=case.layout,
                        pad_page_bytes=case.pad_page_bytes, offset_bytes=case.offset_bytes)
    q, qsl = make_queries(case.q_lens, Hq=case.Hq, D=case.D, seed=case.seed + 100,
                          dtype=case.q_dtype, device=device)
    if case.pad_tokens:
        pad = torch.full((case.pad_tokens, case.Hq, case.D), float("nan"), device=device)
        q = torch.cat([q, pad.to(q.dtype)])
    return Batch(case, cache, q, qsl)


def launch_args(b: Batch, out: torch.Tensor, *, num_splits: int, bq: int,
                ws_o: torch.Tensor | None = None, ws_lse: torch.Tensor | None = None
                ) -> capi.PthAttnArgs:
    c = b.cache
    return capi.attn_args(
        q=b.q, out=out, k_cache=c.k_cache, v_cache=c.v_cache, k_scale=c.k_scale,
        v_scale=c.v_scale, block_table=c.block_table, seq_lens=c.seq_lens,
        query_start_loc=b.qsl, bq=bq, num_splits=num_splits,
        softmax_scale=1.0 / math.sqrt(b.case.D), ws_o=ws_o, ws_lse=ws_lse,
        window=b.case.window, causal=b.case.causal)


def oracle_of(b: Batch, *, threads: int = 0) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """fp64 oracle (out, lse, valid) for a batch (copied to the host if needed)."""
    hb = b if b.q.device.type == "cpu" else Batch(b.case, b.cache.to("cpu"), b.q.cpu(), b.qsl.cpu())
    dummy = torch.empty(hb.q.shape, dtype=torch.float32)
    args = launch_args(hb, dummy, num_splits=1, bq=1)
    return oracle.attention(args, threads=threads)


def abs_v_batch(b: Batch) -> Batch:
    """A host copy of the batch whose V values are |V| (every int8 the writer
    produces lies in [-127, 127], so the absolute value is exact): the oracle
    on it gives sum_i p_i |v_id| / l per output element."""
    hc = b.cache.to("cpu")
    hc.v_cache.abs_()
    return Batch(b.case, hc, b.q.cpu(), b.qsl.cpu())


def half_ulp(ref: np.ndarray, dtype: torch.dtype) -> np.ndarray:
    """Half an ulp of ``ref`` in the output dtype: the rounding any exact kernel
    incurs when it stores ``ref`` (bf16: 8 significant bits, fp16: 11)."""
    bits = {torch.bfloat16: 8, torch.float16: 11, torch.float32: 24}[dtype]
    mag = np.maximum(np.abs(ref), 2.0 ** -126)
    return np.ldexp(1.0, (np.floor(np.log2(mag)) - bits).astype(np.int64))


def compare(out: torch.Tensor, lse: torch.Tensor | None, ref_out: np.ndarray,
            ref_lse: np.ndarray, valid: np.ndarray) -> dict:
    """Errors of a device result against the oracle on the valid rows.

    max_abs / mean_abs are the plain absolute errors; max_excess / mean_excess
    subtract the half-ulp rounding of the output dtype (what an exact kernel
    would also show), for cases whose outputs are large enough that storage
    rounding alone exceeds the absolute tolerance.
    """
    o = out.float().cpu().numpy()[valid].astype(np.float64)
    r = ref_out[valid]
    err = np.abs(o - r)
    hu = half_ulp(r, out.dtype)
    res = {"max_abs": float(err.max()) if err.size else 0.0,
           "mean_abs": float(err.mean()) if err.size else 0.0,
           "max_excess": float((err - hu).max()) if err.size else 0.0,
           "mean_excess": float(np.maximum(err - hu, 0).mean()) if err.size else 0.0,
           "finite": bool(np.isfinite(o).all())}
    if lse is not None:
        le = np.abs(lse.float().cpu().numpy()[valid] - ref_lse[valid])
        res["lse_max_abs"] = float(le.max()) if le.size else 0.0
    return res


# Every parity check of the session: (name, strict, result). The terminal
# summary (conftest.py) lists the relaxed-gate ones with their plain errors.
PARITY_LOG: list[tuple[str, bool, dict]] = []


def assert_parity(res: dict, *, name: str = "", strict: bool = True) -> None:
    """strict: the plain absolute gate (max 2e-3, mean 2e-4). Otherwise the
    gate applies to the error beyond the output dtype's own rounding; the
    plain errors are still recorded (PARITY_LOG) and reported."""
    PARITY_LOG.append((name, strict, dict(res)))
    assert res["finite"], f"{name}: non-finite output"
    mx, mn = (res["max_abs"], res["mean_abs"]) if strict else (res["max_excess"], res["mean_excess"])
    assert mx <= MAX_ABS, f"{name}: max abs {mx:.3g} > {MAX_ABS} ({res})"
    assert mn <= MEAN_ABS, f"{name}: mean abs {mn:.3g} > {MEAN_ABS} ({res})"
    if "lse_max_abs" in res:
        assert res["lse_max_abs"] <= LSE_ABS, f"{name}: lse {res['lse_max_abs']:.3g} > {LSE_ABS}"


def uniform_lengths(n: int, lo: int, hi: int, seed: int) -> list[int]:
    rng = np.random.default_rng(seed)
    return [int(x) for x in rng.integers(lo, hi + 1, size=n)]
