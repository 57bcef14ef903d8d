"""Stand-in modules for the part of vLLM's API that ``pth_flash_attn.vllm_backend``
and ``pth_flash_attn.plugin`` import, so the adapter runs on the CPU where vLLM
is absent (vLLM is not installed in this image or on the GPU boxes).

Only the names and behaviours the adapter relies on are provided, each
restated from how the reference's own backend tests drive vLLM
(``tests/cpu/test_backend_builder.py`` of the reference: the config fields it
builds with ``SimpleNamespace``, the reorder threshold ``max(floor(64 / G),
1 + k)`` with spec-as-decode, ``UNIFORM_BATCH`` = 2, a workspace manager whose
``get_simultaneous`` hands out views of one growing buffer and refuses to
grow once locked). Nothing here is vLLM code; a test that passes against
these stand-ins shows that the adapter drives this surface as intended, not
that a given vLLM release matches it.

``installed()`` is a context manager that puts the modules into
``sys.modules`` and removes them (and any module imported under them)
afterwards.
"""

from __future__ import annotations

import contextlib
import dataclasses
import enum
import sys
import types
from collections import namedtuple
from typing import Any, Generic, TypeVar

import torch

# --------------------------------------------------------------- vllm.config
_current_config: list[Any] = [None]


class VllmConfig:
    """Type name only: the tests pass ``SimpleNamespace`` configs."""


def get_current_vllm_config_or_none() -> Any:
    return _current_config[0]


@contextlib.contextmanager
def current_config(cfg: Any):
    """Stand-in for vLLM's ``set_current_vllm_config`` (model load scope)."""
    old = _current_config[0]
    _current_config[0] = cfg
    try:
        yield cfg
    finally:
        _current_config[0] = old


# ------------------------------------------------------------ vllm.platforms
DeviceCapability = namedtuple("DeviceCapability", ["major", "minor"])


class _Platform:
    compute_units = 256  # MI355X

    def num_compute_units(self, index: int | None = None) -> int:
        return self.compute_units


current_platform = _Platform()


# ------------------------------------------------------ vllm.v1.attention.*
class AttentionCGSupport(enum.Enum):
    NEVER = 0
    UNIFORM_SINGLE_TOKEN_DECODE = 1
    UNIFORM_BATCH = 2
    ALWAYS = 3


class AttentionType:
    DECODER = "decoder"
    ENCODER = "encoder"
    ENCODER_ONLY = "encoder_only"
    ENCODER_DECODER = "encoder_decoder"


@dataclasses.dataclass(frozen=True)
class MultipleOf:
    base: int


@dataclasses.dataclass
class CommonAttentionMetadata:
    query_start_loc: torch.Tensor
    query_start_loc_cpu: torch.Tensor
    seq_lens: torch.Tensor
    num_reqs: int
    num_actual_tokens: int
    max_query_len: int
    max_seq_len: int
    block_table_tensor: torch.Tensor
    slot_mapping: torch.Tensor
    causal: bool = True


M = TypeVar("M")


class AttentionMetadataBuilder(Generic[M]):
    reorder_batch_threshold: int | None = None

    def __init__(self, kv_cache_spec: Any, layer_names: list[str], vllm_config: Any,
                 device: torch.device) -> None:
        self.kv_cache_spec = kv_cache_spec
        self.layer_names = layer_names
        self.vllm_config = vllm_config
        self.device = device

    def _init_reorder_batch_threshold(self, reorder_batch_threshold: int | None = 1,
                                      supports_spec_as_decode: bool = False) -> None:
        self.reorder_batch_threshold = reorder_batch_threshold
        if reorder_batch_threshold is not None and supports_spec_as_decode:
            spec = self.vllm_config.speculative_config
            if spec is not None and spec.num_speculative_tokens:
                self.reorder_batch_threshold = max(reorder_batch_threshold,
                                                   1 + int(spec.num_speculative_tokens))


class TritonAttentionBackend:
    """The base the adapter subclasses: generic validation over the
    ``supports_*`` queries, in one reason string per refusal."""

    supported_dtypes: list[torch.dtype] = [torch.float16, torch.bfloat16, torch.float32]
    supported_kv_cache_dtypes: list[str] = ["auto"]

    @classmethod
    def supports_head_size(cls, head_size: int) -> bool:
        return True

    @classmethod
    def supports_block_size(cls, block_size: int | None) -> bool:
        return True

    @classmethod
    def supports_attn_type(cls, attn_type: str) -> bool:
        return attn_type == AttentionType.DECODER

    @classmethod
    def supports_non_causal(cls) -> bool:
        return False

    @classmethod
    def supports_sliding_window(cls) -> bool:
        return True

    @classmethod
    def supports_sink(cls) -> bool:
        return False

    @classmethod
    def supports_mm_prefix(cls) -> bool:
        return False

    @classmethod
    def supports_compute_capability(cls, capability: DeviceCapability) -> bool:
        return True

    @classmethod
    def validate_configuration(cls, head_size: int, dtype: torch.dtype, kv_cache_dtype: str,
                               block_size: int | None, use_mla: bool, has_sink: bool,
                               use_sparse: bool, device_capability: DeviceCapability,
                               use_mm_prefix: bool = False, has_sliding_window: bool = False,
                               use_non_causal: bool = False,
                               attn_type: str = AttentionType.DECODER) -> list[str]:
        reasons = []
        if not cls.supports_head_size(head_size):
            reasons.append("head_size not supported")
        if dtype not in cls.supported_dtypes:
            reasons.append("dtype not supported")
        if kv_cache_dtype not in cls.supported_kv_cache_dtypes:
            reasons.append("kv_cache_dtype not supported")
        if not cls.supports_block_size(block_size):
            reasons.append("block_size not supported")
        if use_mla:
            reasons.append("MLA not supported")
        if has_sink and not cls.supports_sink():
            reasons.append("sink setting not supported")
        if use_sparse:
            reasons.append("sparse not supported")
        if use_mm_prefix and not cls.supports_mm_prefix():
            reasons.append("partial multimodal token full attention not supported")
        if has_sliding_window and not cls.supports_sliding_window():
            reasons.append("sliding window not supported")
        if use_non_causal and not cls.supports_non_causal():
            reasons.append("non-causal attention not supported")
        if not cls.supports_compute_capability(device_capability):
            reasons.append("compute capability not supported")
        if not cls.supports_attn_type(attn_type):
            reasons.append(f"attention type {attn_type} not supported")
        return reasons


class TritonAttentionImpl:
    def __init__(self, num_heads: int, head_size: int, scale: float, num_kv_heads: int,
                 alibi_slopes: Any, sliding_window: int | None, kv_cache_dtype: str,
                 logits_soft_cap: float | None = None, attn_type: str = AttentionType.DECODER,
                 kv_sharing_target_layer_name: Any = None, sinks: Any = None,
                 use_alibi_sqrt: bool = False, chunk_lookback: int = -1) -> None:
        self.num_heads = num_heads
        self.head_size = head_size
        self.scale = float(scale)
        self.num_kv_heads = num_kv_heads
        self.kv_cache_dtype = kv_cache_dtype
        self.attn_type = attn_type
        self.dcp_world_size = 1
        self.pcp_world_size = 1


def get_num_attention_heads_from_layers(vllm_config: Any, layer_names: list[str]) -> int | None:
    """The q heads of the group's layers from the forward context, if recorded."""
    ctx = getattr(getattr(vllm_config, "compilation_config", None), "static_forward_context", {})
    heads = {getattr(ctx[n], "num_heads", None) for n in layer_names if n in ctx}
    heads.discard(None)
    return heads.pop() if len(heads) == 1 else None


@dataclasses.dataclass
class AttentionSpec:
    num_kv_heads: int
    head_size: int
    block_size: int = 16
    sliding_window: int | None = None


class AttentionBackendEnum(enum.Enum):
    TRITON_ATTN = "vllm.v1.attention.backends.triton_attn.TritonAttentionBackend"
    CUSTOM = ""

    def get_path(self) -> str:
        return _registry.get(self, self.value)

    def is_overridden(self) -> bool:
        return self in _registry


_registry: dict[AttentionBackendEnum, str] = {}


def register_backend(backend: AttentionBackendEnum, class_path: str) -> None:
    _registry[backend] = class_path


# ------------------------------------------------------------ vllm.v1.worker
def get_num_ubatches(parallel_config: Any) -> int:
    return int(parallel_config.num_ubatches) if getattr(parallel_config, "use_ubatching", False) else 1


class WorkspaceManager:
    """One device buffer; get_simultaneous returns disjoint views of it
    (256-byte aligned), growing it while unlocked and refusing to once locked."""

    def __init__(self, device: torch.device | str) -> None:
        self.device = torch.device(device)
        self.buffer = torch.empty(0, dtype=torch.uint8, device=self.device)
        self.locked = False
        self.grows = 0

    def get_simultaneous(self, *specs: tuple[tuple, torch.dtype]) -> list[torch.Tensor]:
        offs, total = [], 0
        for shape, dtype in specs:
            n = 1
            for s in shape:
                n *= int(s)
            offs.append(total)
            total += (n * torch.empty(0, dtype=dtype).element_size() + 255) // 256 * 256
        if total > self.buffer.numel():
            if self.locked:
                raise AssertionError(
                    f"workspace is locked: {total} bytes requested, {self.buffer.numel()} reserved")
            self.buffer = torch.empty(total, dtype=torch.uint8, device=self.device)
            self.grows += 1
        out = []
        for (shape, dtype), o in zip(specs, offs):
            n = 1
            for s in shape:
                n *= int(s)
            nb = n * torch.empty(0, dtype=dtype).element_size()
            out.append(self.buffer[o:o + nb].view(dtype).view(shape))
        return out

    def lock(self) -> None:
        self.locked = True


_manager: list[WorkspaceManager | None] = [None]


def init_workspace_manager(device: torch.device | str) -> WorkspaceManager:
    _manager[0] = WorkspaceManager(device)
    return _manager[0]


def reset_workspace_manager() -> None:
    _manager[0] = None


def current_workspace_manager() -> WorkspaceManager:
    if _manager[0] is None:
        raise AssertionError("workspace manager is not initialized")
    return _manager[0]


def is_workspace_manager_initialized() -> bool:
    return _manager[0] is not None


# ----------------------------------------------------------------- install
def _module(name: str, **attrs: Any) -> types.ModuleType:
    m = types.ModuleType(name)
    m.__dict__.update(attrs)
    m.__path__ = []  # every stand-in can be a package
    return m


def modules() -> dict[str, types.ModuleType]:
    return {
        "vllm": _module("vllm", __pth_stub__=True),
        "vllm.config": _module("vllm.config", VllmConfig=VllmConfig,
                               get_current_vllm_config_or_none=get_current_vllm_config_or_none),
        "vllm.config.cache": _module("vllm.config.cache", CacheDType=str),
        "vllm.platforms": _module("vllm.platforms", current_platform=current_platform),
        "vllm.platforms.interface": _module("vllm.platforms.interface",
                                            DeviceCapability=DeviceCapability),
        "vllm.v1": _module("vllm.v1"),
        "vllm.v1.attention": _module("vllm.v1.attention"),
        "vllm.v1.attention.backend": _module(
            "vllm.v1.attention.backend", AttentionCGSupport=AttentionCGSupport,
            AttentionMetadataBuilder=AttentionMetadataBuilder, AttentionType=AttentionType,
            CommonAttentionMetadata=CommonAttentionMetadata, MultipleOf=MultipleOf),
        "vllm.v1.attention.backends": _module("vllm.v1.attention.backends"),
        "vllm.v1.attention.backends.triton_attn": _module(
            "vllm.v1.attention.backends.triton_attn",
            TritonAttentionBackend=TritonAttentionBackend, TritonAttentionImpl=TritonAttentionImpl),
        "vllm.v1.attention.backends.utils": _module(
            "vllm.v1.attention.backends.utils",
            get_num_attention_heads_from_layers=get_num_attention_heads_from_layers),
        "vllm.v1.attention.backends.registry": _module(
            "vllm.v1.attention.backends.registry", AttentionBackendEnum=AttentionBackendEnum,
            register_backend=register_backend),
        "vllm.v1.kv_cache_interface": _module("vllm.v1.kv_cache_interface",
                                              AttentionSpec=AttentionSpec),
        "vllm.v1.worker": _module("vllm.v1.worker"),
        "vllm.v1.worker.ubatch_utils": _module("vllm.v1.worker.ubatch_utils",
                                               get_num_ubatches=get_num_ubatches),
        "vllm.v1.worker.workspace": _module(
            "vllm.v1.worker.workspace", current_workspace_manager=current_workspace_manager,
            is_workspace_manager_initialized=is_workspace_manager_initialized),
    }


@contextlib.contextmanager
def installed():
    """The stand-ins in sys.modules for the duration; the adapter modules
    imported under them are dropped afterwards."""
    saved = {k: v for k, v in sys.modules.items() if k == "vllm" or k.startswith("vllm.")}
    for k in saved:
        del sys.modules[k]
    sys.modules.update(modules())
    _registry.clear()
    try:
        yield
    finally:
        for k in [k for k in sys.modules if k == "vllm" or k.startswith("vllm.")
                  or k == "pth_flash_attn.vllm_backend"]:
            del sys.modules[k]
        sys.modules.update(saved)
        reset_workspace_manager()
