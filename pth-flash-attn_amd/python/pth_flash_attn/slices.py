"""The engine-side core of the vLLM backend: launch slices of one step.

The reference's vLLM backend (``python/pth_flash_attn/vllm_backend.py``) does
four engine-independent things around the op, and this module holds them
without importing vLLM, so they run and are tested where vLLM is absent:

* **Refusals** (``impl_refusals``, ``group_size``, ``SliceBuilder.__init__``,
  ``SliceBuilder.build``): what the kernels do not serve is refused with its
  reason, at layer construction or at build time (reference
  vllm_backend.py:185-211, 253-285, 330-352, 589-621).
* **Slicing** (``SliceBuilder.build``): a step's batch, ordered decode first,
  becomes at most two launches, the decode-like slice (every request with
  ``q_len <= reorder_batch_threshold``, speculative verify included) and the
  prefill slice, each planned with ``planner.plan_launch`` on its own
  descriptor (reference vllm_backend.py:287-446).
* **Device-side rebase**: the prefill slice's ``query_start_loc`` is the
  device copy minus the device value of its first request, written into one
  persistent buffer, so the step reads nothing on the host and allocates
  nothing (reference vllm_backend.py:304-352).
* **The forward** (``run_slices``): one op call per slice with workspace
  views of that launch's size, or the shared empty tensor when S = 1
  (reference vllm_backend.py:704-796).

Nothing here reads device data on the host, so a decode step can be captured
in a HIP graph (the plan depends on host integers only, and the kernels read
``seq_lens`` and ``query_start_loc`` on the device).

``split_decodes_and_prefills`` restates vLLM's helper of the same name
(``vllm/v1/attention/backends/utils.py``, vLLM 0.30; vLLM is not installed
here): the first request whose ``q_len`` exceeds the threshold starts the
prefill part; everything before it is decode-like.
"""

from __future__ import annotations

from collections.abc import Callable, Sequence
from dataclasses import dataclass

import torch

from . import planner

# The one KV-cache dtype the backend serves.
KV_CACHE_DTYPE = "int8_per_token_head"
# Kernel block sizes the backend accepts are multiples of this (the paged
# kernels take 16-key groups from one page).
KERNEL_BLOCK_MULTIPLE = 16
# Query length of a decode request without speculation.
NO_SPEC_QUERY_LEN = 1


def verify_query_len(num_speculative_tokens: int | None) -> int:
    """q_dec_max = 1 + k: the verify length that sizes the workspace
    (reference vllm_backend.py:111-124)."""
    k = int(num_speculative_tokens) if num_speculative_tokens else 0
    if k < 0:
        raise ValueError(f"num_speculative_tokens must be >= 0, got {k}")
    return NO_SPEC_QUERY_LEN + k


def group_size(num_heads_q: int, num_kv_heads: int) -> int:
    """G = Hq / Hkv, refused when not a whole number or larger than one row
    tile (reference vllm_backend.py:185-197)."""
    if num_kv_heads < 1 or num_heads_q % num_kv_heads != 0:
        raise ValueError(
            f"pth_flash_attn: Hq = {num_heads_q} must be a positive multiple of "
            f"Hkv = {num_kv_heads}"
        )
    g = num_heads_q // num_kv_heads
    if g > planner.MAX_ROWS_PER_CTA:
        raise ValueError(f"pth_flash_attn: G = Hq/Hkv = {g} exceeds {planner.MAX_ROWS_PER_CTA}")
    return g


def no_windowed_kernel(what: str, head_size: int) -> str:
    """Reason text for a windowed or non-causal layer at a head size without
    that kernel (reference vllm_backend.py:200-205)."""
    sizes = ", ".join(map(str, planner.WINDOWED_HEAD_SIZES))
    return f"{what} at head size {head_size} (the windowed kernels exist for D = {sizes} only)"


def decode_threshold(G: int, q_verify: int) -> int:
    """reorder_batch_threshold: the query tokens one 64-row tile holds
    (floor(64 / G)), raised to the verify length (spec-as-decode)."""
    return max(planner.max_tokens_per_tile(G), int(q_verify))


def impl_refusals(
    *,
    head_size: int,
    sliding_window: int | None = None,
    alibi: bool = False,
    logits_soft_cap: float | None = None,
    sinks: bool = False,
    chunk_lookback: int = -1,
    is_decoder: bool = True,
    kv_cache_dtype: str = KV_CACHE_DTYPE,
) -> list[str]:
    """What a layer asks for that the kernels do not serve, one reason each
    (reference vllm_backend.py:589-621, in the same order)."""
    out: list[str] = []
    if alibi:
        out.append("ALiBi")
    if sliding_window is not None:
        if sliding_window < 1:
            out.append(f"sliding window {sliding_window}")
        elif head_size not in planner.WINDOWED_HEAD_SIZES:
            out.append(no_windowed_kernel("sliding window", head_size))
    if logits_soft_cap:
        out.append("logits soft cap")
    if sinks:
        out.append("attention sinks")
    if chunk_lookback != -1:
        out.append("chunk lookback")
    if not is_decoder:
        out.append("attention type other than decoder self-attention")
    if kv_cache_dtype != KV_CACHE_DTYPE:
        out.append(f"kv_cache_dtype {kv_cache_dtype}")
    if head_size not in planner.SUPPORTED_HEAD_SIZES:
        out.append(f"head size {head_size}")
    return out


def split_decodes_and_prefills(
    query_start_loc_cpu: torch.Tensor, *, num_reqs: int, num_tokens: int, max_query_len: int,
    threshold: int,
) -> tuple[int, int, int, int]:
    """(num_decodes, num_prefills, num_decode_tokens, num_prefill_tokens).

    The batch is expected decode first: the first request with
    q_len > threshold and every request after it form the prefill part. A
    batch in another order stays correct (the prefill launch serves any
    q_len), it is only planned less tightly.
    """
    if max_query_len <= threshold:
        return num_reqs, 0, num_tokens, 0
    q = query_start_loc_cpu[1 : num_reqs + 1] - query_start_loc_cpu[:num_reqs]
    long_q = (q > threshold).tolist()
    if long_q and long_q[0]:
        return 0, num_reqs, 0, num_tokens
    if not any(long_q):
        return num_reqs, 0, num_tokens, 0
    first = long_q.index(True)
    dec_tokens = int(query_start_loc_cpu[first])
    return first, num_reqs - first, dec_tokens, num_tokens - dec_tokens


@dataclass(frozen=True)
class LaunchSlice:
    """One op call: a contiguous run of requests and of their tokens.

    The tensors are views of the step's persistent device buffers (or of the
    builder's rebase buffer), made once per step, so the forward only slices
    ``query``/``output`` by the token range.
    """

    plan: planner.LaunchPlan
    token_start: int
    token_end: int
    max_query_len: int
    query_start_loc: torch.Tensor  # int32 [num_reqs + 1], starts at 0
    seq_lens: torch.Tensor  # int32 [num_reqs]
    block_table: torch.Tensor  # int32 [>= num_reqs, max_blocks]


@dataclass
class StepSlices:
    """The launches of one step (reference PthAttnMetadata's two slices)."""

    num_actual_tokens: int
    max_query_len: int
    causal: bool
    decode: LaunchSlice | None
    prefill: LaunchSlice | None


class SliceBuilder:
    """Plans the decode-like and prefill slices of a step for one group of
    layers (one KV-cache spec: heads, head size, window)."""

    def __init__(
        self,
        *,
        num_heads_q: int,
        num_kv_heads: int,
        head_size: int,
        window: int,
        max_num_seqs: int,
        q_verify: int,
        num_cus: int,
        device: torch.device | str,
    ) -> None:
        self.num_kv_heads = int(num_kv_heads)
        self.head_size = int(head_size)
        self.group = group_size(int(num_heads_q), self.num_kv_heads)
        if self.head_size not in planner.SUPPORTED_HEAD_SIZES:
            raise NotImplementedError(
                f"pth_flash_attn: head size {self.head_size} is not one of "
                f"{planner.SUPPORTED_HEAD_SIZES}"
            )
        self.window = int(window) if window else 0
        if self.window and self.head_size not in planner.WINDOWED_HEAD_SIZES:
            raise NotImplementedError(
                "pth_flash_attn: " + no_windowed_kernel("sliding window", self.head_size)
            )
        self.num_cus = int(num_cus)
        self.q_verify = int(q_verify)
        self.reorder_batch_threshold = decode_threshold(self.group, self.q_verify)
        self.ws_token_splits = planner.workspace_token_splits(
            max_num_seqs=int(max_num_seqs), q_dec_max=self.q_verify, Hkv=self.num_kv_heads,
            D=self.head_size, num_sms=self.num_cus,
        )
        # The prefill slice's query_start_loc, rebased on the device: one int32
        # per request plus one, kept for the builder's lifetime.
        self.prefill_qsl = torch.zeros(int(max_num_seqs) + 1, dtype=torch.int32, device=device)

    def _slice(
        self, query_start_loc: torch.Tensor, seq_lens: torch.Tensor, block_table: torch.Tensor, *,
        req_start: int, req_end: int, token_start: int, token_end: int, max_query_len: int,
        is_prefill: bool,
    ) -> LaunchSlice:
        plan = planner.plan_launch(
            num_tokens=token_end - token_start, num_reqs=req_end - req_start,
            max_query_len=max_query_len, G=self.group, Hkv=self.num_kv_heads, D=self.head_size,
            num_sms=self.num_cus, is_prefill=is_prefill, ws_token_splits=self.ws_token_splits,
            window=self.window,
        )
        n = req_end - req_start
        if req_start == 0:
            qsl = query_start_loc if query_start_loc.shape[0] == n + 1 else query_start_loc[: n + 1]
        else:
            if n + 1 > self.prefill_qsl.shape[0]:
                raise RuntimeError(
                    f"pth_flash_attn: {n} prefill requests exceed max_num_seqs = "
                    f"{self.prefill_qsl.shape[0] - 1}"
                )
            qsl = self.prefill_qsl[: n + 1]
            # The device value of the first prefill request is subtracted: under
            # adaptive verification the host copy can differ from it.
            torch.sub(query_start_loc[req_start : req_end + 1],
                      query_start_loc[req_start : req_start + 1], out=qsl)
        return LaunchSlice(
            plan=plan, token_start=token_start, token_end=token_end, max_query_len=max_query_len,
            query_start_loc=qsl, seq_lens=seq_lens[req_start:req_end],
            block_table=block_table[req_start:req_end],
        )

    def build(
        self,
        *,
        query_start_loc: torch.Tensor,
        query_start_loc_cpu: torch.Tensor,
        seq_lens: torch.Tensor,
        block_table: torch.Tensor,
        num_reqs: int,
        num_actual_tokens: int,
        max_query_len: int,
        causal: object = True,
        common_prefix_len: int = 0,
        rswa_prefix_lens: object = None,
        mm_req_doc_ranges: dict | None = None,
    ) -> StepSlices:
        """The step's slices (reference vllm_backend.py:367-446)."""
        if common_prefix_len > 0:
            raise NotImplementedError("pth_flash_attn: cascade attention")
        if not isinstance(causal, bool):
            raise NotImplementedError(
                "pth_flash_attn: per-request causal masks are not supported (got "
                f"{type(causal).__name__}); causal must be one bool per group"
            )
        if not causal and self.head_size not in planner.WINDOWED_HEAD_SIZES:
            raise NotImplementedError(
                "pth_flash_attn: " + no_windowed_kernel("non-causal attention", self.head_size)
            )
        if rswa_prefix_lens is not None:
            raise NotImplementedError("pth_flash_attn: R-SWA is not supported")
        if mm_req_doc_ranges and any(mm_req_doc_ranges.values()):
            raise NotImplementedError(
                "pth_flash_attn: bidirectional multimodal prefix ranges are not supported"
            )
        num_reqs, num_tokens, max_q = int(num_reqs), int(num_actual_tokens), int(max_query_len)
        n_dec, n_pre, dec_tokens, _ = split_decodes_and_prefills(
            query_start_loc_cpu, num_reqs=num_reqs, num_tokens=num_tokens, max_query_len=max_q,
            threshold=self.reorder_batch_threshold or 1,
        )
        decode = prefill = None
        if n_dec > 0 and dec_tokens > 0:
            if n_pre == 0:
                q_dec = max_q
            else:
                # Host bound of the decode part alone, from the host copy.
                q_dec = int((query_start_loc_cpu[1 : n_dec + 1] - query_start_loc_cpu[:n_dec]).max())
            decode = self._slice(
                query_start_loc, seq_lens, block_table, req_start=0, req_end=n_dec, token_start=0,
                token_end=dec_tokens, max_query_len=max(q_dec, 1), is_prefill=False,
            )
        if n_pre > 0 and num_tokens - dec_tokens > 0:
            prefill = self._slice(
                query_start_loc, seq_lens, block_table, req_start=n_dec, req_end=num_reqs,
                token_start=dec_tokens, token_end=num_tokens, max_query_len=max_q, is_prefill=True,
            )
        return StepSlices(num_actual_tokens=num_tokens, max_query_len=max_q, causal=causal,
                          decode=decode, prefill=prefill)

    def build_for_graph_capture(self, **kw) -> StepSlices:
        """As ``build``, then ``seq_lens = 1``: a capture run walks one key per
        request instead of the whole cache; the plan does not depend on it
        (reference vllm_backend.py:448-456)."""
        step = self.build(**kw)
        kw["seq_lens"].fill_(1)
        return step


# The workspace provider: (o_shape, lse_shape) -> (ws_o, ws_lse) fp32 views.
WorkspaceFn = Callable[[tuple, tuple], tuple[torch.Tensor, torch.Tensor]]


def run_slices(
    step: StepSlices,
    *,
    query: torch.Tensor,
    output: torch.Tensor,
    caches: Sequence[torch.Tensor],
    scale: float,
    window: int,
    workspace: WorkspaceFn,
    no_workspace: torch.Tensor,
    reserved_token_splits: int = 0,
    op: Callable | None = None,
) -> torch.Tensor:
    """The forward: one op call per slice, decode first (at most two calls;
    reference vllm_backend.py:704-796). ``caches`` are the op's (k_cache,
    v_cache, k_scale, v_scale) views."""
    if op is None:
        from . import ops

        op = ops.pth_flash_attn_fwd
    k, v, ks, vs = caches
    for part in (step.decode, step.prefill):
        if part is None:
            continue
        plan = part.plan
        if plan.num_splits > 1:
            need = plan.num_splits * plan.num_tokens
            if reserved_token_splits and need > reserved_token_splits:
                raise RuntimeError(
                    f"pth_flash_attn: launch needs {need} token-splits, "
                    f"{reserved_token_splits} were reserved"
                )
            ws_o, ws_lse = workspace(plan.ws_o_shape, plan.ws_lse_shape)
        else:
            ws_o = ws_lse = no_workspace
        t0, t1 = part.token_start, part.token_end
        whole = t0 == 0 and t1 == output.shape[0]
        op(output if whole else output[t0:t1], query if whole else query[t0:t1], k, v, ks, vs,
           part.block_table, part.seq_lens, part.query_start_loc, part.max_query_len, plan.wm,
           plan.num_splits, scale, ws_o, ws_lse, window, step.causal)
    return output
