"""Engine configuration with the ``decode_backend`` plugin switch.

Same fields, defaults and validation messages as the reference
``src/nanovllm/config.py:13-110``. ``decode_backend="megakernel"`` selects the
MI355X persistent task-graph decoder; ``"torch"`` is the standard path.

Two knobs are specific to this build and documented here:

* ``megakernel_launch``: ``"persistent"`` (one persistent launch per step, the
  task graph with dependency counters) or ``"graph"`` (the same kernels
  launched one per op and replayed as a captured hipGraph). Default
  ``"persistent"``.
* ``megakernel_attn_splits``: minimum split-KV factor. The decoder raises it
  with context length (one split per 256 positions, capped at 16) because a
  static single split leaves most CUs idle at long context.
"""

from __future__ import annotations

import os
from dataclasses import dataclass
from typing import Any

VALID_DECODE_BACKENDS = {"torch", "megakernel"}
VALID_MEGAKERNEL_LAUNCH = {"persistent", "graph"}


def validate_decode_backend(value: str) -> str:
    if value not in VALID_DECODE_BACKENDS:
        options = ", ".join(sorted(VALID_DECODE_BACKENDS))
        raise ValueError(f"decode_backend must be one of: {options}; got {value!r}")
    return value


@dataclass(slots=True)
class Config:
    model: str
    max_num_batched_tokens: int = 16384
    max_prefill_tokens_per_step: int = 0
    prefill_decode_ratio: int = 1
    max_num_seqs: int = 512
    max_model_len: int = 4096
    gpu_memory_utilization: float = 0.9
    tensor_parallel_size: int = 1
    enforce_eager: bool = False
    decode_backend: str = "torch"
    megakernel_attn_splits: int = 1
    fusion_groups: int = 1
    megakernel_verbose: bool = False
    megakernel_debug_bounds: bool = False
    megakernel_launch: str = "persistent"
    hf_config: Any | None = None
    eos: int = -1
    kvcache_block_size: int = 256
    num_kvcache_blocks: int = -1

    def __post_init__(self):
        self.decode_backend = validate_decode_backend(self.decode_backend)
        if self.megakernel_launch not in VALID_MEGAKERNEL_LAUNCH:
            raise ValueError(
                "megakernel_launch must be one of: graph, persistent; got "
                f"{self.megakernel_launch!r}"
            )
        if self.max_prefill_tokens_per_step < 0:
            raise ValueError(
                "max_prefill_tokens_per_step must be >= 0; got "
                f"{self.max_prefill_tokens_per_step}"
            )
        if self.prefill_decode_ratio < 1:
            raise ValueError(
                f"prefill_decode_ratio must be >= 1; got {self.prefill_decode_ratio}"
            )
        if self.megakernel_attn_splits < 1:
            raise ValueError(
                f"megakernel_attn_splits must be >= 1; got {self.megakernel_attn_splits}"
            )
        if self.fusion_groups < 1:
            raise ValueError(f"fusion_groups must be >= 1; got {self.fusion_groups}")
        if not os.path.isdir(self.model):
            raise ValueError(f"model directory does not exist: {self.model}")
        if self.max_num_batched_tokens < 1:
            raise ValueError(
                f"max_num_batched_tokens must be >= 1; got {self.max_num_batched_tokens}"
            )
        if self.max_num_seqs < 1:
            raise ValueError(f"max_num_seqs must be >= 1; got {self.max_num_seqs}")
        if self.max_model_len < 1:
            raise ValueError(f"max_model_len must be >= 1; got {self.max_model_len}")
        if not 0.0 < self.gpu_memory_utilization <= 1.0:
            raise ValueError(
                "gpu_memory_utilization must be in (0, 1]; got "
                f"{self.gpu_memory_utilization}"
            )
        if self.kvcache_block_size < 256 or self.kvcache_block_size % 256:
            raise ValueError(
                "kvcache_block_size must be a multiple of 256 and >= 256; got "
                f"{self.kvcache_block_size}"
            )
        if not 1 <= self.tensor_parallel_size <= 8:
            raise ValueError(
                f"tensor_parallel_size must be in [1, 8]; got {self.tensor_parallel_size}"
            )
        if self.hf_config is None:
            from transformers import AutoConfig

            self.hf_config = AutoConfig.from_pretrained(self.model)
        self.max_model_len = min(
            self.max_model_len, self.hf_config.max_position_embeddings
        )
