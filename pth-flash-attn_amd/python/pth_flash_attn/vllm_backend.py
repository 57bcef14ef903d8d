"""vLLM attention backend ``CUSTOM`` that runs ``pth_flash_attn_fwd`` on MI355X.

The adapter between vLLM's backend interfaces and ``slices`` (which holds the
engine-independent logic and is tested without vLLM). Class names, the
backend name, the capability queries and the refusals follow the reference
backend (``python/pth_flash_attn/vllm_backend.py``), so a deployment selects
it the same way (``--attention-backend CUSTOM`` after ``plugin.register``):

* the cache spec, page layout and cache writer stay vLLM's Triton backend's
  (``PthFlashAttnBackend`` subclasses ``TritonAttentionBackend``,
  ``PthFlashAttnImpl`` subclasses ``TritonAttentionImpl``); only the read side
  changes;
* ``PthFlashAttnMetadataBuilder`` plans at most two launches per step
  (``slices.SliceBuilder``) and allocates one small persistent buffer;
* the Impl reserves the split workspace at model load, inside the memory
  window that sizes the KV cache, and its forward makes at most two op calls
  (``slices.run_slices``) and allocates nothing.

The op's four cache views are carved from vLLM's packed layer cache by
``cache.vllm_packed_views`` (no copy). The accepted GPU is gfx950 (vLLM's
ROCm platform reports it as capability 9.5).

Importing this module imports vLLM; on a host without vLLM it raises
ImportError (``plugin.register`` imports it only when the backend is
selected). vLLM is not installed where this library is built and tested:
``tests/test_vllm_backend.py`` executes every class here against stand-ins
for the vLLM names imported below (``tests/vllm_stub.py``) with a recording
op, and ``tests/test_slices.py`` covers the logic it delegates to.
"""

from __future__ import annotations

import inspect
from typing import Any, ClassVar

import torch
from vllm.config import VllmConfig, get_current_vllm_config_or_none
from vllm.config.cache import CacheDType
from vllm.platforms import current_platform
from vllm.platforms.interface import DeviceCapability
from vllm.v1.attention.backend import (
    AttentionCGSupport,
    AttentionMetadataBuilder,
    AttentionType,
    CommonAttentionMetadata,
    MultipleOf,
)
from vllm.v1.attention.backends.triton_attn import TritonAttentionBackend, TritonAttentionImpl
from vllm.v1.attention.backends.utils import get_num_attention_heads_from_layers
from vllm.v1.kv_cache_interface import AttentionSpec
from vllm.v1.worker.ubatch_utils import get_num_ubatches
from vllm.v1.worker.workspace import current_workspace_manager, is_workspace_manager_initialized

from . import ops, planner, slices
from .cache import vllm_packed_views

BACKEND_NAME = "CUSTOM"
# gfx950 as vLLM's ROCm platform reports it.
SUPPORTED_CAPABILITY = (9, 5)


def _num_cus(device: torch.device | None = None) -> int:
    """The CU count (a planner input) from vLLM's platform, never torch.cuda."""
    index = device.index if device is not None else None
    if index is None:
        index = torch.accelerator.current_device_index()
    return int(current_platform.num_compute_units(index))


def _speculative_tokens(vllm_config: VllmConfig) -> int:
    spec = vllm_config.speculative_config
    return int(spec.num_speculative_tokens) if spec is not None and spec.num_speculative_tokens else 0


def verify_query_len(vllm_config: VllmConfig) -> int:
    """q_dec_max = 1 + k (reference vllm_backend.py:111-124)."""
    return slices.verify_query_len(_speculative_tokens(vllm_config))


def reserved_token_splits(vllm_config: VllmConfig, *, num_kv_heads: int, head_size: int,
                          num_sms: int) -> int:
    """W_ts the Impl reserves and the builder clamps to (the same inputs)."""
    return planner.workspace_token_splits(
        max_num_seqs=int(vllm_config.scheduler_config.max_num_seqs),
        q_dec_max=verify_query_len(vllm_config), Hkv=num_kv_heads, D=head_size, num_sms=num_sms,
    )


def group_window(kv_cache_spec: AttentionSpec) -> int:
    """The group's sliding window (0 for none); it caps the split count."""
    window = getattr(kv_cache_spec, "sliding_window", None)
    return int(window) if window else 0


class PthFlashAttnMetadataBuilder(AttentionMetadataBuilder[slices.StepSlices]):
    """Builds the decode-like and prefill launch slices of a step."""

    _cudagraph_support: ClassVar[AttentionCGSupport] = AttentionCGSupport.UNIFORM_BATCH
    supports_draft_decode_metadata_update = True

    def __init__(self, kv_cache_spec: AttentionSpec, layer_names: list[str],
                 vllm_config: VllmConfig, device: torch.device) -> None:
        super().__init__(kv_cache_spec, layer_names, vllm_config, device)
        model_config = vllm_config.model_config
        if get_num_ubatches(vllm_config.parallel_config) > 1:
            raise NotImplementedError(
                "pth_flash_attn: dual-batch overlap (DBO) is not supported: the "
                "workspace is one buffer per ubatch lane"
            )
        if model_config.rswa_window is not None:
            raise NotImplementedError("pth_flash_attn: R-SWA is not supported")
        num_heads_q = get_num_attention_heads_from_layers(
            vllm_config, layer_names
        ) or model_config.get_num_attention_heads(vllm_config.parallel_config)
        self.core = slices.SliceBuilder(
            num_heads_q=num_heads_q, num_kv_heads=int(kv_cache_spec.num_kv_heads),
            head_size=int(kv_cache_spec.head_size), window=group_window(kv_cache_spec),
            max_num_seqs=int(vllm_config.scheduler_config.max_num_seqs),
            q_verify=verify_query_len(vllm_config), num_cus=_num_cus(device), device=device,
        )
        self.ws_token_splits = self.core.ws_token_splits
        self._init_reorder_batch_threshold(
            planner.max_tokens_per_tile(self.core.group), supports_spec_as_decode=True
        )

    @classmethod
    def get_varlen_cudagraph_max_query_len(cls, vllm_config: VllmConfig,
                                           kv_cache_spec: AttentionSpec) -> int:
        heads = vllm_config.model_config.get_num_attention_heads(vllm_config.parallel_config)
        g = slices.group_size(heads, int(kv_cache_spec.num_kv_heads))
        return slices.decode_threshold(g, verify_query_len(vllm_config))

    def _core_args(self, common_prefix_len: int, cam: CommonAttentionMetadata) -> dict:
        return dict(
            query_start_loc=cam.query_start_loc, query_start_loc_cpu=cam.query_start_loc_cpu,
            seq_lens=cam.seq_lens, block_table=cam.block_table_tensor, num_reqs=int(cam.num_reqs),
            num_actual_tokens=int(cam.num_actual_tokens), max_query_len=int(cam.max_query_len),
            causal=cam.causal, common_prefix_len=common_prefix_len,
            rswa_prefix_lens=getattr(cam, "rswa_prefix_lens", None),
            mm_req_doc_ranges=getattr(cam, "mm_req_doc_ranges", None),
        )

    def build(self, common_prefix_len: int, common_attn_metadata: CommonAttentionMetadata,
              fast_build: bool = False) -> slices.StepSlices:
        # vLLM's own threshold (set by _init_reorder_batch_threshold) decides
        # the split, as its runner reorders the batch with it.
        self.core.reorder_batch_threshold = self.reorder_batch_threshold or 1
        step = self.core.build(**self._core_args(common_prefix_len, common_attn_metadata))
        cam = common_attn_metadata
        # Field names vLLM's runners and speculators read.
        step.query_start_loc = cam.query_start_loc
        step.seq_lens = cam.seq_lens
        step.block_table = cam.block_table_tensor
        step.slot_mapping = cam.slot_mapping
        step.max_seq_len = int(cam.max_seq_len)
        step.use_cascade = False
        step.common_prefix_len = 0
        return step

    def build_for_cudagraph_capture(self, common_attn_metadata: CommonAttentionMetadata
                                    ) -> slices.StepSlices:
        step = self.build(0, common_attn_metadata)
        step.seq_lens.fill_(1)
        return step

    def update_draft_decode_metadata(self, _metadata: slices.StepSlices) -> None:
        """Nothing to update: every step-dependent field is a persistent buffer."""


class PthFlashAttnBackend(TritonAttentionBackend):
    """``CUSTOM``: Triton's cache and writer, this library's kernels and builder."""

    supported_dtypes: ClassVar[list[torch.dtype]] = [torch.float16, torch.bfloat16]
    supported_kv_cache_dtypes: ClassVar[list[CacheDType]] = [slices.KV_CACHE_DTYPE]  # type: ignore[list-item]

    @staticmethod
    def get_name() -> str:
        return BACKEND_NAME

    @staticmethod
    def get_impl_cls() -> type[PthFlashAttnImpl]:
        return PthFlashAttnImpl

    @staticmethod
    def get_builder_cls() -> type[PthFlashAttnMetadataBuilder]:  # type: ignore[override]
        return PthFlashAttnMetadataBuilder

    @staticmethod
    def get_supported_kernel_block_sizes(kv_cache_spec: AttentionSpec | None = None
                                         ) -> list[int | MultipleOf]:  # type: ignore[override]
        return [MultipleOf(slices.KERNEL_BLOCK_MULTIPLE)]

    @classmethod
    def supports_block_size(cls, block_size: int | None) -> bool:
        return block_size is None or block_size % slices.KERNEL_BLOCK_MULTIPLE == 0

    @classmethod
    def supports_head_size(cls, head_size: int) -> bool:
        return head_size in planner.SUPPORTED_HEAD_SIZES

    @classmethod
    def supports_attn_type(cls, attn_type: str) -> bool:
        return attn_type == AttentionType.DECODER

    @classmethod
    def supports_non_causal(cls) -> bool:
        return True  # at D = 128; validate_configuration refuses other sizes

    @classmethod
    def supports_sliding_window(cls) -> bool:
        return True  # at D = 128; validate_configuration refuses other sizes

    @classmethod
    def supports_rswa(cls) -> bool:
        return False

    @classmethod
    def validate_configuration(cls, *args: Any, **kwargs: Any) -> list[str]:
        """vLLM's reasons plus: a windowed or non-causal layer needs D = 128."""
        reasons = super().validate_configuration(*args, **kwargs)
        bound = inspect.signature(super().validate_configuration).bind(*args, **kwargs)
        bound.apply_defaults()
        arg = bound.arguments
        head_size = arg["head_size"]
        if head_size in planner.SUPPORTED_HEAD_SIZES and head_size not in planner.WINDOWED_HEAD_SIZES:
            if arg["has_sliding_window"]:
                reasons.append(slices.no_windowed_kernel("sliding window", head_size))
            if arg["use_non_causal"]:
                reasons.append(slices.no_windowed_kernel("non-causal attention", head_size))
        return reasons

    @classmethod
    def supports_sink(cls) -> bool:
        return False

    @classmethod
    def supports_mm_prefix(cls) -> bool:
        return False

    @classmethod
    def supports_alibi_sqrt(cls) -> bool:
        return False

    @classmethod
    def supports_batch_invariance(cls) -> bool:
        return False  # the split count depends on the batch shape

    @classmethod
    def supports_compute_capability(cls, capability: DeviceCapability) -> bool:
        """gfx950 with the op library built."""
        return (capability.major, capability.minor) == SUPPORTED_CAPABILITY and ops.is_available()


class PthFlashAttnImpl(TritonAttentionImpl):
    """Reads the int8 cache with ``pth_flash_attn_fwd``; writes it as Triton does."""

    def __init__(self, num_heads: int, head_size: int, scale: float, num_kv_heads: int,
                 alibi_slopes: list[float] | None, sliding_window: int | None,
                 kv_cache_dtype: str, logits_soft_cap: float | None = None,
                 attn_type: AttentionType = AttentionType.DECODER,
                 kv_sharing_target_layer_name: int | None = None,
                 sinks: torch.Tensor | None = None, use_alibi_sqrt: bool = False,
                 chunk_lookback: int = -1) -> None:
        unsupported = slices.impl_refusals(
            head_size=head_size, sliding_window=sliding_window,
            alibi=alibi_slopes is not None or use_alibi_sqrt, logits_soft_cap=logits_soft_cap,
            sinks=sinks is not None, chunk_lookback=chunk_lookback,
            is_decoder=attn_type == AttentionType.DECODER, kv_cache_dtype=kv_cache_dtype,
        )
        if unsupported:
            raise NotImplementedError("pth_flash_attn does not support: " + ", ".join(unsupported))
        slices.group_size(num_heads, num_kv_heads)
        super().__init__(num_heads, head_size, scale, num_kv_heads, alibi_slopes, sliding_window,
                         kv_cache_dtype, logits_soft_cap, attn_type, kv_sharing_target_layer_name,
                         sinks, use_alibi_sqrt, chunk_lookback)
        if getattr(self, "dcp_world_size", 1) > 1 or getattr(self, "pcp_world_size", 1) > 1:
            raise NotImplementedError("pth_flash_attn: DCP/PCP are not supported")
        self.supports_quant_query_input = False
        self.window = 0 if sliding_window is None else int(sliding_window)
        self._cache_views: tuple[int, tuple[torch.Tensor, ...]] | None = None
        self._ws_token_splits = 0
        self._no_workspace: torch.Tensor | None = None
        self._reserve_workspace(get_current_vllm_config_or_none())

    def _reserve_workspace(self, vllm_config: VllmConfig | None) -> None:
        """Reserve W_ts token-splits of fp32 partials at model load."""
        if vllm_config is None or not is_workspace_manager_initialized():
            return
        self._ws_token_splits = reserved_token_splits(
            vllm_config, num_kv_heads=self.num_kv_heads, head_size=self.head_size,
            num_sms=_num_cus(),
        )
        o_shape, lse_shape = planner.workspace_shapes(
            ws_token_splits=self._ws_token_splits, Hq=self.num_heads, D=self.head_size
        )
        ws_o, _ = current_workspace_manager().get_simultaneous(
            (o_shape, torch.float32), (lse_shape, torch.float32)
        )
        self._no_workspace = torch.empty(0, dtype=torch.float32, device=ws_o.device)

    def _caches(self, kv_cache: torch.Tensor) -> tuple[torch.Tensor, ...]:
        """The op's four views of this layer's cache, carved once per tensor."""
        ptr = kv_cache.data_ptr()
        if self._cache_views is not None and self._cache_views[0] == ptr:
            return self._cache_views[1]
        views = vllm_packed_views(kv_cache)
        self._cache_views = (ptr, views)
        return views

    @staticmethod
    def _workspace(o_shape: tuple, lse_shape: tuple) -> tuple[torch.Tensor, torch.Tensor]:
        return current_workspace_manager().get_simultaneous(
            (o_shape, torch.float32), (lse_shape, torch.float32)
        )

    def forward(self, layer: torch.nn.Module, query: torch.Tensor, key: torch.Tensor,
                value: torch.Tensor, kv_cache: torch.Tensor, attn_metadata: slices.StepSlices,
                output: torch.Tensor, output_scale: torch.Tensor | None = None,
                output_block_scale: torch.Tensor | None = None) -> torch.Tensor:
        """The decode slice, then the prefill slice (at most two op calls)."""
        if output_scale is not None or output_block_scale is not None:
            raise NotImplementedError("pth_flash_attn: fused output quantisation is not supported")
        if attn_metadata is None:  # memory-profile run
            return output.fill_(0)
        if self._no_workspace is None:
            self._no_workspace = torch.empty(0, dtype=torch.float32, device=output.device)
        return slices.run_slices(
            attn_metadata, query=query, output=output, caches=self._caches(kv_cache),
            scale=self.scale, window=self.window, workspace=self._workspace,
            no_workspace=self._no_workspace, reserved_token_splits=self._ws_token_splits,
        )
