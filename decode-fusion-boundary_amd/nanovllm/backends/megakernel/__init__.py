"""MI355X task-graph decode backend (``decode_backend="megakernel"``)."""

from .backend import (
    Compatibility,
    MegakernelBackend,
    gcn_arch_supported,
    is_megakernel_backend,
    qwen3_contract_mismatch,
)
from .cache import PagedKVCacheSpec
from .taskgraph import TG_MAX_BATCH, TaskGraphCompatibility, taskgraph_compatibility

__all__ = [
    "Compatibility",
    "MegakernelBackend",
    "PagedKVCacheSpec",
    "TG_MAX_BATCH",
    "TaskGraphCompatibility",
    "gcn_arch_supported",
    "is_megakernel_backend",
    "qwen3_contract_mismatch",
    "taskgraph_compatibility",
]
