"""``decode_backend="megakernel"`` adapter (reference ``backends/megakernel/backend.py:104-258``).

Same public surface as the reference: ``compatibility`` (admission with the
same reason strings), ``set_kv_cache``, ``ensure_ready``, ``disable``,
``ready``, ``decode`` (batch 1, host block table) and ``decode_batch``. The
decoder is built lazily and needs a ROCm device with the HIP library built
for gfx950; any failure before it exists is reported to the caller, which
disables the backend and falls back to the torch path.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Any

from nanovllm.engine.kv_layout import decode_position

from .taskgraph import taskgraph_compatibility

MAX_BATCH_SIZE = 8
MEGAKERNEL_BACKENDS = ("megakernel",)
SUPPORTED_GCN_ARCH = "gfx950"

QWEN3_CONTRACT = {
    "model_type": "qwen3",
    "hidden_size": 1024,
    "intermediate_size": 3072,
    "num_hidden_layers": 28,
    "num_attention_heads": 16,
    "num_key_value_heads": 8,
    "vocab_size": 151936,
    "max_model_len": 2048,
    "head_dim": 128,
}


def is_megakernel_backend(value: Any) -> bool:
    return value in MEGAKERNEL_BACKENDS


def _attr(obj: Any, name: str, default: Any = None) -> Any:
    return getattr(obj, name, default)


def qwen3_contract_mismatch(config) -> str | None:
    """Name of the first contract field the config violates (None when it matches)."""

    hf = _attr(config, "hf_config")
    if _attr(hf, "tie_word_embeddings", True) is not True:
        return "tie_word_embeddings"
    if _attr(hf, "attention_bias", False) is not False:
        return "attention_bias"
    for name, expected in QWEN3_CONTRACT.items():
        if name == "max_model_len":
            actual = _attr(config, "max_model_len", 2048)
            if actual > expected:
                return name
            continue
        if name == "head_dim":
            actual = _attr(hf, "head_dim", None) or hf.hidden_size // hf.num_attention_heads
        else:
            actual = _attr(hf, name)
        if actual != expected:
            return name
    return None


@dataclass(frozen=True)
class Compatibility:
    supported: bool
    reason: str = ""


def gcn_arch_supported(arch_name: str) -> bool:
    """Whether a ROCm ``gcnArchName`` (e.g. ``gfx950:sramecc+:xnack-``) runs the library."""

    return arch_name.split(":")[0] == SUPPORTED_GCN_ARCH


class MegakernelBackend:
    """Lazy adapter around the task-graph decoder."""

    def __init__(self, config, model):
        self.config = config
        self.model = model
        self.decoder = None
        self.kv_cache = None
        self.disabled_reason = None

    @staticmethod
    def compatibility(config, seqs, is_prefill: bool) -> Compatibility:
        decision = taskgraph_compatibility(config, seqs, is_prefill)
        if not decision.supported:
            return Compatibility(False, decision.reason)
        mismatch = qwen3_contract_mismatch(config)
        if mismatch is not None:
            return Compatibility(False, f"unsupported Qwen config: {mismatch}")
        return Compatibility(True)

    def set_kv_cache(self, kv_cache) -> None:
        if kv_cache is None or kv_cache.dim() != 6 or kv_cache.shape[0] != 2:
            raise ValueError("kv_cache must have shape [2, layers, blocks, tokens, heads, dim]")
        self.kv_cache = kv_cache

    def disable(self, reason: str) -> None:
        self.disabled_reason = reason

    @property
    def ready(self) -> bool:
        return self.decoder is not None

    def ensure_ready(self) -> None:
        self._ensure_decoder()

    def _validate_cache_layout(self) -> None:
        from .cache import PagedKVCacheSpec

        kv = self.kv_cache
        hf = self.config.hf_config
        head_dim = _attr(hf, "head_dim", None) or hf.hidden_size // hf.num_attention_heads
        spec = PagedKVCacheSpec(
            num_layers=hf.num_hidden_layers, num_blocks=kv.shape[2],
            block_size=self.config.kvcache_block_size, num_kv_heads=kv.shape[4],
            head_dim=kv.shape[5], dtype_itemsize=kv.element_size(),
        )
        if tuple(kv.shape) != spec.shape:
            raise RuntimeError(
                f"paged KV cache shape {tuple(kv.shape)} does not match the megakernel contract {spec.shape}")
        if not (kv[0].is_contiguous() and kv[1].is_contiguous()):
            raise RuntimeError("paged KV cache views must be contiguous for the megakernel layer-stride offset math")
        if kv[0].size(0) * spec.layer_stride != kv[0].numel():
            raise RuntimeError("paged KV cache layer stride does not match the megakernel offset contract")
        if head_dim != QWEN3_CONTRACT["head_dim"]:
            raise RuntimeError("Qwen head_dim differs from the megakernel contract")

    def _ensure_decoder(self):
        if self.disabled_reason:
            raise RuntimeError(self.disabled_reason)
        if self.decoder is not None:
            return
        if self.kv_cache is None:
            raise RuntimeError("nano-vLLM KV cache has not been attached")
        import torch

        if not torch.cuda.is_available() or torch.version.hip is None:
            raise RuntimeError("Megakernel requires a ROCm (HIP) device")
        arch = torch.cuda.get_device_properties(self.kv_cache.device).gcnArchName
        if not gcn_arch_supported(arch):
            raise RuntimeError(f"Megakernel is built for {SUPPORTED_GCN_ARCH}; detected {arch}")
        self._validate_cache_layout()
        from .build import get_extension
        from .taskgraph import TaskGraphDecoder
        from .weights import weights_from_nano_model

        get_extension()
        weights = weights_from_nano_model(self.model, self.config.hf_config)
        self.decoder = TaskGraphDecoder(
            weights,
            k_cache=self.kv_cache[0], v_cache=self.kv_cache[1],
            block_size=self.config.kvcache_block_size, num_cache_blocks=self.kv_cache.shape[2],
            max_model_len=_attr(self.config, "max_model_len", 2048),
            attn_splits=int(_attr(self.config, "megakernel_attn_splits", 1)),
            fusion_groups=int(_attr(self.config, "fusion_groups", 1)),
            launch=_attr(self.config, "megakernel_launch", "persistent"),
            verbose=bool(_attr(self.config, "megakernel_verbose", False)),
            debug_bounds=bool(_attr(self.config, "megakernel_debug_bounds", False)),
        )

    def decode_batch(self, input_ids, positions, block_tables) -> list[int]:
        self._ensure_decoder()
        return self.decoder.decode_rows(input_ids, positions, block_tables)

    def decode_seqs(self, seqs) -> list[int]:
        """Batch step straight from the sequences (host values, pinned staging):
        the runner's batch path. ``decode_batch`` keeps the device-tensor signature."""

        self._ensure_decoder()
        return self.decoder.decode_rows_host([s.last_token for s in seqs],
                                             [decode_position(len(s)) for s in seqs],
                                             [list(s.block_table) for s in seqs])

    def decode(self, seq, block_table) -> list[int]:
        self._ensure_decoder()
        return [int(self.decoder.step(seq.last_token, position=decode_position(len(seq)),
                                      block_table=block_table))]
