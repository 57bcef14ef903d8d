"""The ``vllm.general_plugins`` entry point: registers the ``CUSTOM`` backend.

vLLM runs every ``vllm.general_plugins`` entry point in each process it
starts, before it selects an attention backend. ``register`` records this
library's backend class path under ``AttentionBackendEnum.CUSTOM`` (the one
member vLLM reserves for out-of-tree backends) and imports nothing else: the
op library and the backend module load only when ``--attention-backend
CUSTOM`` selects it. If another plugin already registered a different class
there, it is left in place with a warning (reference python/pth_flash_attn/
plugin.py:28-45).
"""

from __future__ import annotations

import logging

BACKEND_CLASS_PATH = "pth_flash_attn.vllm_backend.PthFlashAttnBackend"

logger = logging.getLogger(__name__)


def register() -> None:
    """Register ``PthFlashAttnBackend`` as ``AttentionBackendEnum.CUSTOM``."""
    from vllm.v1.attention.backends.registry import AttentionBackendEnum, register_backend

    custom = AttentionBackendEnum.CUSTOM
    if custom.is_overridden() and custom.get_path() != BACKEND_CLASS_PATH:
        logger.warning("pth_flash_attn: AttentionBackendEnum.CUSTOM is already registered as "
                       "%s; leaving it unchanged", custom.get_path())
        return
    register_backend(custom, BACKEND_CLASS_PATH)
