"""Random-init Qwen3-0.6B weights and a local model directory.

There is no checkpoint on the GPU boxes and no network, so every run uses the
random-init model the benchmark configs describe: seed 0; every weight matrix
and the (tied) embedding drawn N(0, 0.02); every RMSNorm vector
(input/post-attention, q_norm/k_norm, final) drawn N(1, 0.02), i.e. the
Hugging Face init of ones perturbed by the same std so a kernel that skips a
norm weight cannot pass unnoticed.

Generation order is fixed (it defines the bytes): for each layer the eleven
tensors in weight-ABI order -- input_layernorm, q, k, v, q_norm, k_norm, o,
post_attention_layernorm, gate, up, down (reference
``backends/megakernel/weights.py:143-157``) -- then the embedding, then the
final norm. Values are drawn in fp32 on the CPU from one ``torch.Generator``
and rounded to bf16.
"""

from __future__ import annotations

import json
import os
from dataclasses import dataclass

from nanovllm.model_spec import QWEN3_06B, ModelSpec

WEIGHT_STD = 0.02
LAYER_KEYS = (
    "ln_in", "q", "k", "v", "q_norm", "k_norm", "o", "ln_post", "gate", "up", "down",
)


def layer_shapes(spec: ModelSpec = QWEN3_06B) -> dict[str, tuple[int, ...]]:
    h, i, hd = spec.hidden_size, spec.intermediate_size, spec.head_dim
    return {
        "ln_in": (h,),
        "q": (spec.q_size, h),
        "k": (spec.kv_size, h),
        "v": (spec.kv_size, h),
        "q_norm": (hd,),
        "k_norm": (hd,),
        "o": (h, spec.q_size),
        "ln_post": (h,),
        "gate": (i, h),
        "up": (i, h),
        "down": (h, i),
    }


@dataclass
class SyntheticWeights:
    """Host (CPU) bf16 tensors. ``layers[l][key]`` uses :data:`LAYER_KEYS`."""

    layers: list
    embed: object
    final_norm: object
    spec: ModelSpec = QWEN3_06B

    @property
    def num_layers(self) -> int:
        return len(self.layers)


def make_weights(
    seed: int = 0, num_layers: int | None = None, spec: ModelSpec = QWEN3_06B
) -> SyntheticWeights:
    """Generate the weights. ``num_layers`` < 28 gives the first layers of the
    same stream (layer ``l`` is bit-identical whatever ``num_layers`` is), but
    the embedding/final norm then come from a different point of the stream."""

    import torch

    gen = torch.Generator(device="cpu")
    gen.manual_seed(seed)
    n_layers = spec.num_layers if num_layers is None else int(num_layers)
    shapes = layer_shapes(spec)

    def draw(shape, mean):
        t = torch.empty(shape, dtype=torch.float32)
        t.normal_(mean=mean, std=WEIGHT_STD, generator=gen)
        return t.to(torch.bfloat16)

    layers = []
    for _ in range(n_layers):
        layer = {}
        for key in LAYER_KEYS:
            mean = 1.0 if len(shapes[key]) == 1 else 0.0
            layer[key] = draw(shapes[key], mean)
        layers.append(layer)
    embed = draw((spec.vocab_size, spec.hidden_size), 0.0)
    final_norm = draw((spec.hidden_size,), 1.0)
    return SyntheticWeights(layers=layers, embed=embed, final_norm=final_norm, spec=spec)


def hf_config_dict(spec: ModelSpec = QWEN3_06B, num_layers: int | None = None) -> dict:
    """``config.json`` of a Qwen3-0.6B-geometry model (what ``AutoConfig`` reads)."""

    return {
        "architectures": ["Qwen3ForCausalLM"],
        "model_type": "qwen3",
        "hidden_size": spec.hidden_size,
        "intermediate_size": spec.intermediate_size,
        "num_hidden_layers": spec.num_layers if num_layers is None else num_layers,
        "num_attention_heads": spec.num_q_heads,
        "num_key_value_heads": spec.num_kv_heads,
        "head_dim": spec.head_dim,
        "vocab_size": spec.vocab_size,
        "max_position_embeddings": 40960,
        "rms_norm_eps": spec.rms_norm_eps,
        "rope_theta": spec.rope_theta,
        "rope_scaling": None,
        "tie_word_embeddings": True,
        "attention_bias": False,
        "hidden_act": "silu",
        "torch_dtype": "bfloat16",
        "bos_token_id": 151643,
        "eos_token_id": 151645,
    }


def write_model_dir(path: str, num_layers: int | None = None, seed: int = 0) -> str:
    """Create a model directory holding ``config.json`` and a ``synthetic.json``
    marker that tells the loader to generate the weights instead of reading
    safetensors."""

    os.makedirs(path, exist_ok=True)
    with open(os.path.join(path, "config.json"), "w") as f:
        json.dump(hf_config_dict(num_layers=num_layers), f, indent=1)
    with open(os.path.join(path, "synthetic.json"), "w") as f:
        json.dump({"seed": seed, "std": WEIGHT_STD}, f)
    return path


def synthetic_marker(path: str) -> dict | None:
    marker = os.path.join(path, "synthetic.json")
    if not os.path.exists(marker):
        return None
    with open(marker) as f:
        return json.load(f)
