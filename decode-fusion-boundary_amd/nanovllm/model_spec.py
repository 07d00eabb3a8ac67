"""Qwen3-0.6B geometry: the single place the decode-step shapes are written down.

Follows the reference ``src/nanovllm/model_spec.py:399-411`` (``QWEN3_06B``) and
its byte accounting (``params_per_layer`` = 15,730,944 at ``:214-233``; tied
embedding streamed once per step). The HIP kernels are compiled for exactly
these numbers; ``csrc/mkd_common.h`` repeats them as ``constexpr`` and
``tests/test_spec_abi.py`` checks the two agree.
"""

from __future__ import annotations

from dataclasses import dataclass

BYTES_PER_PARAM_BF16 = 2


@dataclass(frozen=True)
class ModelSpec:
    name: str
    num_layers: int
    hidden_size: int
    intermediate_size: int
    num_q_heads: int
    num_kv_heads: int
    head_dim: int
    vocab_size: int
    max_model_len: int = 2048
    rms_norm_eps: float = 1e-6
    rope_theta: float = 1_000_000.0
    tie_word_embeddings: bool = True

    @property
    def q_size(self) -> int:
        return self.num_q_heads * self.head_dim

    @property
    def kv_size(self) -> int:
        return self.num_kv_heads * self.head_dim

    @property
    def qkv_size(self) -> int:
        return self.q_size + 2 * self.kv_size

    @property
    def group_size(self) -> int:
        return self.num_q_heads // self.num_kv_heads

    #: Device pointers per layer in the weight ABI, in this order:
    #: input_layernorm, q, k, v, q_norm, k_norm, o, post_attention_layernorm,
    #: gate, up, down (reference ``weights.py:143-157``).
    weight_pointer_count: int = 11

    def params_per_layer(self) -> int:
        h, i = self.hidden_size, self.intermediate_size
        qkv = h * self.qkv_size
        o = self.q_size * h
        norms = 2 * h + 2 * self.head_dim
        ffn = 3 * h * i
        return qkv + o + norms + ffn

    def total_params(self) -> int:
        """Parameters streamed per decode step (tied embedding counted once)."""

        return (
            self.num_layers * self.params_per_layer()
            + self.hidden_size
            + self.vocab_size * self.hidden_size
        )

    def weight_bytes(self) -> int:
        return self.total_params() * BYTES_PER_PARAM_BF16

    def kv_bytes_per_position(self) -> int:
        """K+V bytes of one token over all layers (read once per decode step)."""

        return self.num_layers * 2 * self.kv_size * BYTES_PER_PARAM_BF16


QWEN3_06B = ModelSpec(
    name="Qwen3-0.6B",
    num_layers=28,
    hidden_size=1024,
    intermediate_size=3072,
    num_q_heads=16,
    num_kv_heads=8,
    head_dim=128,
    vocab_size=151936,
)
