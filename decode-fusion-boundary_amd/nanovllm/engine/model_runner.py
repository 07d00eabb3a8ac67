"""Model runner: owns the torch model and the paged KV cache, dispatches decode.

Dispatch and fallback follow the reference ``engine/model_runner.py:315-376``:
a greedy decode batch the megakernel admits goes to ``MegakernelBackend``
(batch 1 through ``decode`` with the host block table, larger batches through
``decode_batch``); everything else runs the torch path with
``last_fallback_reason`` set. A failure before the decoder exists disables the
backend with a ``RuntimeWarning``; a failure after it exists is fatal, because
the shared KV cache may already have been written.

Single GPU only: ``tensor_parallel_size > 1`` is rejected here (the reference's
spawned-worker tensor parallelism is not built; the megakernel requires TP=1).
"""

from __future__ import annotations

import os
import warnings

import torch

from nanovllm.backends.megakernel import MegakernelBackend
from nanovllm.backends.megakernel.backend import is_megakernel_backend
from nanovllm.config import Config
from nanovllm.engine.kv_layout import (
    decode_cache_len, decode_position, decode_slot_mapping, pad_block_table, prefill_cache_len,
    prefill_positions, prefill_slot_mapping,
)
from nanovllm.engine.sequence import Sequence
from nanovllm.qwen3_torch import AttentionMetadata, Qwen3ForCausalLM, load_synthetic, sample
from nanovllm.synthetic import make_weights, synthetic_marker


def load_model(model: Qwen3ForCausalLM, path: str) -> None:
    """Fill the model from ``path``: a synthetic marker (random init) or safetensors files."""

    marker = synthetic_marker(path)
    if marker is not None:
        weights = make_weights(seed=int(marker.get("seed", 0)), num_layers=len(model.model.layers))
        load_synthetic(model, weights)
        return
    from safetensors import safe_open

    params = dict(model.named_parameters())
    packed = {"q_proj": ("qkv_proj", 0), "k_proj": ("qkv_proj", 1), "v_proj": ("qkv_proj", 2),
              "gate_proj": ("gate_up_proj", 0), "up_proj": ("gate_up_proj", 1)}
    files = sorted(f for f in os.listdir(path) if f.endswith(".safetensors"))
    if not files:
        raise FileNotFoundError(f"no safetensors and no synthetic.json in {path}")
    with torch.no_grad():
        for name in files:
            with safe_open(os.path.join(path, name), "pt", "cpu") as f:
                for key in f.keys():
                    tensor = f.get_tensor(key)
                    for short, (fused, idx) in packed.items():
                        if short in key:
                            target = params[key.replace(short, fused)]
                            attn = model.model.layers[0].self_attn
                            sizes = ([attn.q_size, attn.kv_size, attn.kv_size] if fused == "qkv_proj"
                                     else [target.shape[0] // 2] * 2)
                            start = sum(sizes[:idx])
                            target.data[start:start + sizes[idx]].copy_(tensor)
                            break
                    else:
                        if key == "lm_head.weight" and key not in params:
                            continue
                        params[key].data.copy_(tensor)


class ModelRunner:
    def __init__(self, config: Config, rank: int = 0, event=None, init_method: str | None = None):
        if config.tensor_parallel_size != 1:
            raise NotImplementedError(
                "tensor_parallel_size > 1 is not built: the MI355X engine runs one GPU per process")
        self.config = config
        hf = config.hf_config
        self.block_size = config.kvcache_block_size
        self.enforce_eager = config.enforce_eager
        self.world_size = 1
        self.rank = rank
        self.device = torch.device("cuda" if torch.cuda.is_available() else "cpu")
        default_dtype = torch.get_default_dtype()
        torch.set_default_dtype(torch.bfloat16)
        try:
            self.model = Qwen3ForCausalLM(hf)
        finally:
            torch.set_default_dtype(default_dtype)
        load_model(self.model, config.model)
        self.model.to(self.device)
        self.megakernel = None
        self.last_backend_used = "torch"
        self.last_fallback_reason = None
        self._cuda_poisoned = False
        self.allocate_kv_cache()
        if is_megakernel_backend(config.decode_backend):
            self.megakernel = MegakernelBackend(config, self.model)
            self.megakernel.set_kv_cache(self.kv_cache)
            try:
                self.megakernel.ensure_ready()
            except Exception as exc:  # noqa: BLE001 - the torch path stays available
                warnings.warn(f"Megakernel disabled at startup; using the standard backend: {exc}",
                              RuntimeWarning, stacklevel=2)
                self.megakernel.disable(str(exc))

    def exit(self):
        if self.megakernel is not None and self.megakernel.decoder is not None:
            self.megakernel.decoder.close()
        if self.device.type == "cuda" and not self._cuda_poisoned:
            torch.cuda.synchronize()

    def call(self, method_name, *args):
        return getattr(self, method_name)(*args)

    def allocate_kv_cache(self):
        config, hf = self.config, self.config.hf_config
        num_kv_heads = hf.num_key_value_heads
        head_dim = getattr(hf, "head_dim", None) or hf.hidden_size // hf.num_attention_heads
        block_bytes = 2 * hf.num_hidden_layers * self.block_size * num_kv_heads * head_dim * 2
        if config.num_kvcache_blocks > 0:
            blocks = config.num_kvcache_blocks
        elif self.device.type == "cuda":
            free, total = torch.cuda.mem_get_info()
            used = total - free
            blocks = int(total * config.gpu_memory_utilization - used) // block_bytes
        else:
            per_seq = -(-config.max_model_len // self.block_size)
            blocks = min(config.max_num_seqs, 16) * per_seq
        if blocks <= 0:
            raise RuntimeError(
                f"Insufficient free memory for the KV cache: block_bytes={block_bytes}, "
                f"gpu_memory_utilization={config.gpu_memory_utilization:.2f}")
        config.num_kvcache_blocks = blocks
        self.kv_cache = torch.zeros(2, hf.num_hidden_layers, blocks, self.block_size, num_kv_heads,
                                    head_dim, dtype=torch.bfloat16, device=self.device)
        for layer_id, layer in enumerate(self.model.model.layers):
            layer.self_attn.attn.k_cache = self.kv_cache[0, layer_id]
            layer.self_attn.attn.v_cache = self.kv_cache[1, layer_id]

    def prepare_block_tables(self, seqs: list[Sequence]) -> torch.Tensor:
        width = max(len(seq.block_table) for seq in seqs)
        tables = [pad_block_table(seq.block_table, width) for seq in seqs]
        return torch.tensor(tables, dtype=torch.int32, device=self.device)

    def prepare_prefill(self, seqs: list[Sequence]):
        input_ids, positions, slots = [], [], []
        cu_q, cu_k = [0], [0]
        prefix_hit = False
        for seq in seqs:
            start = seq.num_cached_tokens
            n = seq.num_scheduled_tokens
            end = start + n
            input_ids.extend(seq[start:end])
            positions.extend(prefill_positions(start, n))
            cu_q.append(cu_q[-1] + n)
            cu_k.append(cu_k[-1] + prefill_cache_len(start, n))
            prefix_hit |= start > 0
            if seq.block_table:
                slots.extend(prefill_slot_mapping(seq.block_table, start, end, self.block_size))
        meta = AttentionMetadata(
            is_prefill=True,
            slot_mapping=torch.tensor(slots, dtype=torch.int32, device=self.device) if slots else None,
            cu_seqlens_q=cu_q, cu_seqlens_k=cu_k,
            block_tables=self.prepare_block_tables(seqs) if prefix_hit else None,
        )
        ids = torch.tensor(input_ids, dtype=torch.int64, device=self.device)
        pos = torch.tensor(positions, dtype=torch.int64, device=self.device)
        return ids, pos, meta

    def prepare_decode(self, seqs: list[Sequence]):
        input_ids, positions, slots, lens = [], [], [], []
        for seq in seqs:
            n = len(seq)
            input_ids.append(seq.last_token)
            positions.append(decode_position(n))
            lens.append(decode_cache_len(n))
            slots.append(decode_slot_mapping(seq.block_table, n, self.block_size))
        meta = AttentionMetadata(
            is_prefill=False,
            slot_mapping=torch.tensor(slots, dtype=torch.int32, device=self.device),
            context_lens=torch.tensor(lens, dtype=torch.int32, device=self.device),
            context_lens_host=lens,
            block_tables=self.prepare_block_tables(seqs),
        )
        ids = torch.tensor(input_ids, dtype=torch.int64, device=self.device)
        pos = torch.tensor(positions, dtype=torch.int64, device=self.device)
        return ids, pos, meta

    @torch.inference_mode()
    def run_model(self, input_ids, positions, meta):
        hidden = self.model(input_ids, positions, meta)
        return self.model.compute_logits(hidden, meta)

    def run(self, seqs: list[Sequence], is_prefill: bool) -> list[int]:
        self.last_backend_used = "torch"
        self.last_fallback_reason = None
        if self.megakernel is not None and not self.megakernel.disabled_reason:
            decision = MegakernelBackend.compatibility(self.config, seqs, is_prefill)
            if not decision.supported and not is_prefill:
                self.last_fallback_reason = decision.reason
            if decision.supported:
                try:
                    if len(seqs) == 1:
                        token_ids = self.megakernel.decode(seqs[0], seqs[0].block_table)
                    else:
                        token_ids = self.megakernel.decode_seqs(seqs)
                except Exception as exc:
                    if self.megakernel.decoder is not None:
                        self._cuda_poisoned = True
                        raise RuntimeError(
                            f"Megakernel decode failed after initialization: {exc}; "
                            'restart with decode_backend="torch"') from exc
                    self.megakernel.disable(str(exc))
                    self.last_fallback_reason = str(exc)
                    warnings.warn(f"Megakernel unavailable; falling back to the standard backend: {exc}",
                                  RuntimeWarning, stacklevel=2)
                else:
                    self.last_backend_used = self.config.decode_backend
                    return token_ids
        elif self.megakernel is not None and not is_prefill:
            self.last_fallback_reason = self.megakernel.disabled_reason
        ids, pos, meta = self.prepare_prefill(seqs) if is_prefill else self.prepare_decode(seqs)
        temperatures = torch.tensor([seq.temperature for seq in seqs], dtype=torch.float32,
                                    device=self.device)
        logits = self.run_model(ids, pos, meta)
        return sample(logits, temperatures).tolist()
