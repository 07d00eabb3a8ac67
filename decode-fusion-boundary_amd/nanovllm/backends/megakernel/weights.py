"""Weight views, the per-layer pointer table and the RoPE tables of the decoder.

Follows the reference ``backends/megakernel/weights.py``:
``weights_from_nano_model`` (:120-169) splits the fused ``qkv_proj`` and
``gate_up_proj`` weights into row views (no copies), checks bf16 and the tied
``lm_head``/``embed_tokens`` storage, and ``_pack_layer_weights`` (:172-183)
packs 28 x 11 device pointers in ``MkdLayerWeight`` order. The RoPE tables
differ on purpose: the HIP kernels read fp32 cos/sin ``[2048, 64]`` (the
reference kernel used bf16 ``[2048, 128]``) because the torch path they are
compared with rotates with an fp32 cache.
"""

from __future__ import annotations

import torch

from nanovllm.rope_config import QWEN3_DEFAULT_ROPE_THETA, assert_supported_rope_type, resolve_rope_theta

from .schedule import HEAD_DIM, INTERMEDIATE, KV_SIZE, NUM_LAYERS, Q_SIZE

LAYER_POINTER_ORDER = ("ln_in", "q", "k", "v", "q_norm", "k_norm", "o", "ln_post", "gate", "up", "down")
MAX_POSITION = 2048


def rope_tables(theta: float = QWEN3_DEFAULT_ROPE_THETA, device="cuda"):
    """fp32 ``(cos, sin)`` of shape ``[2048, 64]``: ``angle[p, i] = p * theta^(-2i/128)``."""

    inv_freq = 1.0 / (theta ** (torch.arange(0, HEAD_DIM, 2, dtype=torch.float32) / HEAD_DIM))
    angles = torch.einsum("i,j->ij", torch.arange(MAX_POSITION, dtype=torch.float32), inv_freq)
    return angles.cos().contiguous().to(device), angles.sin().contiguous().to(device)


def weights_from_nano_model(model, hf_config) -> dict:
    inner = model.model
    if inner.embed_tokens.weight.dtype != torch.bfloat16:
        raise RuntimeError("Qwen Megakernel requires BF16 model weights")
    if getattr(hf_config, "attention_bias", False):
        raise RuntimeError("Qwen Megakernel requires Qwen QK normalization")
    if model.lm_head.weight.data_ptr() != inner.embed_tokens.weight.data_ptr():
        raise RuntimeError("Qwen Megakernel requires tied lm_head and embed_tokens storage")
    layers = []
    for layer in inner.layers:
        attn = layer.self_attn
        q, k, v = attn.qkv_proj.weight.split([Q_SIZE, KV_SIZE, KV_SIZE], dim=0)
        gate, up = layer.mlp.gate_up_proj.weight.split([INTERMEDIATE, INTERMEDIATE], dim=0)
        layers.append({
            "ln_in": layer.input_layernorm.weight, "q": q, "k": k, "v": v,
            "q_norm": attn.q_norm.weight, "k_norm": attn.k_norm.weight,
            "o": attn.o_proj.weight, "ln_post": layer.post_attention_layernorm.weight,
            "gate": gate, "up": up, "down": layer.mlp.down_proj.weight,
        })
    assert_supported_rope_type(hf_config)
    device = inner.embed_tokens.weight.device
    cos, sin = rope_tables(resolve_rope_theta(hf_config), device=device)
    return {"layers": layers, "embed": inner.embed_tokens.weight, "final_norm": inner.norm.weight,
            "cos": cos, "sin": sin}


def weights_from_synthetic(synth, device="cuda") -> dict:
    """Device copies of :class:`nanovllm.synthetic.SyntheticWeights` (bench / tests)."""

    layers = []
    for layer in synth.layers:
        layers.append({k: v.to(device).contiguous() for k, v in layer.items()})
    cos, sin = rope_tables(device=device)
    return {"layers": layers, "embed": synth.embed.to(device).contiguous(),
            "final_norm": synth.final_norm.to(device).contiguous(), "cos": cos, "sin": sin}


def pack_layer_pointers(layers: list[dict], device="cuda") -> torch.Tensor:
    """``int64 [num_layers, 11]`` device table of the layers' weight pointers."""

    if not 1 <= len(layers) <= NUM_LAYERS:
        raise ValueError(f"expected 1..{NUM_LAYERS} layers, got {len(layers)}")
    rows = []
    for layer in layers:
        row = []
        for key in LAYER_POINTER_ORDER:
            t = layer[key]
            if t.dtype != torch.bfloat16 or not t.is_contiguous():
                raise RuntimeError(f"layer weight {key} must be a contiguous bf16 tensor")
            row.append(t.data_ptr())
        rows.append(row)
    return torch.tensor(rows, dtype=torch.int64).to(device)
