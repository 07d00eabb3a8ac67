"""Helpers shared by the GPU parity tests: build a decoder on synthetic weights
and run the CPU oracle on the same inputs."""

from __future__ import annotations

import torch

from conftest import synthetic_weights

VOCAB = 151936
BS = 256


class Harness:
    """A decoder + a paged KV cache on cuda:0, and the oracle with its own CPU cache copy."""

    def __init__(self, num_layers: int, num_blocks: int, *, launch="persistent", attn_splits=1,
                 fusion_groups=1, max_model_len=2048, kv_fill_seed: int | None = None,
                 variant: str = "lds_dma", **decoder_options):
        from nanovllm.backends.megakernel.taskgraph import TaskGraphDecoder
        from nanovllm.backends.megakernel.weights import weights_from_synthetic
        from oracle.qwen3_oracle import Oracle

        self.synth = synthetic_weights(num_layers)
        self.num_layers = num_layers
        self.w = weights_from_synthetic(self.synth, device="cuda")
        shape = (2, num_layers, num_blocks, BS, 8, 128)
        if kv_fill_seed is None:
            kv_cpu = torch.zeros(shape, dtype=torch.bfloat16)
        else:
            g = torch.Generator().manual_seed(kv_fill_seed)
            kv_cpu = torch.randn(shape, generator=g, dtype=torch.float32).to(torch.bfloat16)
        self.kv_cpu = kv_cpu
        self.kv = kv_cpu.to("cuda")
        self.dec = TaskGraphDecoder(self.w, k_cache=self.kv[0], v_cache=self.kv[1], block_size=BS,
                                    num_cache_blocks=num_blocks, max_model_len=max_model_len,
                                    attn_splits=attn_splits, fusion_groups=fusion_groups, launch=launch,
                                    persistent_variant=variant, **decoder_options)
        self.oracle = Oracle(self.synth)

    def step(self, ids, positions, tables, active=None, mode=None):
        rows = len(ids)
        width = max(len(t) for t in tables)
        padded = [list(t) + [0] * (width - len(t)) for t in tables]
        logits = torch.zeros(rows, VOCAB, dtype=torch.bfloat16, device="cuda")
        toks = self.dec.decode_rows(
            torch.tensor(ids, dtype=torch.int64, device="cuda"),
            torch.tensor(positions, dtype=torch.int64, device="cuda"),
            torch.tensor(padded, dtype=torch.int32, device="cuda"),
            active_rows=active, logits=logits, mode=mode)
        return toks, logits.float().cpu()

    def oracle_step(self, ids, positions, tables, active=None):
        logits, toks = self.oracle.decode_step(ids, positions, tables, self.kv_cpu[0], self.kv_cpu[1],
                                               row_active=active)
        return toks, logits.float()

    def close(self):
        self.dec.close()


def max_abs(a: torch.Tensor, b: torch.Tensor) -> float:
    return (a - b).abs().max().item()
