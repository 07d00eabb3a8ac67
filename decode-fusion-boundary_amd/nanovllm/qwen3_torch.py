"""The torch decode/prefill path: fallback and comparator of the megakernel.

Same computation, module layout and bf16 rounding points as the reference torch
path (``models/qwen3.py:74-187`` with ``layers/layernorm.py:16-40``,
``layers/rotary_embedding.py:6-48``, ``layers/activation.py:6-11``,
``layers/attention.py:59-75``, ``layers/embed_head.py:56-66``,
``layers/sampler.py:5-16``), written for PyTorch-ROCm without flash-attn,
Triton or a process group:

* tensors are bf16 between ops; RMSNorm computes in fp32 and rounds
  ``x * rsqrt(mean(x^2) + eps)`` to bf16 before multiplying by the weight;
  the residual is carried in bf16 and added in fp32;
* RoPE uses an fp32 cos/sin cache and rotate-half, rounded to bf16;
* SiLU-and-mul computes ``silu(g) * u`` in fp32 from the bf16 projections and
  rounds once (the reference compiles this op, which fuses the two roundings);
* paged KV: K/V are stored at ``slot_mapping`` (-1 skips), decode attends over
  ``context_lens`` entries gathered through ``block_tables``; attention is
  computed with fp32 scores and softmax and rounded to bf16;
* logits are bf16 (``F.linear`` on the tied embedding) and greedy sampling is
  ``logits.float().argmax(-1)`` (first maximal index).
"""

from __future__ import annotations

from dataclasses import dataclass

import torch
import torch.nn.functional as F
from torch import nn

from nanovllm.rope_config import assert_supported_rope_type, resolve_rope_theta


@dataclass
class AttentionMetadata:
    """Per-step attention inputs (the reference keeps these in a global Context)."""

    is_prefill: bool
    slot_mapping: torch.Tensor | None = None
    # prefill
    cu_seqlens_q: list[int] | None = None
    cu_seqlens_k: list[int] | None = None
    # decode (and prefix-cached prefill)
    context_lens: torch.Tensor | None = None
    block_tables: torch.Tensor | None = None
    # host copy of context_lens (saves each layer a device-to-host read)
    context_lens_host: list[int] | None = None


class RMSNorm(nn.Module):
    def __init__(self, hidden_size: int, eps: float = 1e-6):
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(hidden_size))

    def _normalize(self, x32: torch.Tensor, dtype) -> torch.Tensor:
        var = x32.pow(2).mean(dim=-1, keepdim=True)
        return (x32 * torch.rsqrt(var + self.eps)).to(dtype) * self.weight

    def forward(self, x: torch.Tensor, residual: torch.Tensor | None = None):
        if residual is None:
            return self._normalize(x.float(), x.dtype)
        s = x.float() + residual.float()
        return self._normalize(s, x.dtype), s.to(x.dtype)


def rope_cos_sin(head_dim: int, max_position: int, base: float, device=None):
    """fp32 ``(cos, sin)`` tables of shape ``[max_position, head_dim // 2]``."""

    inv_freq = 1.0 / (
        base ** (torch.arange(0, head_dim, 2, dtype=torch.float32, device=device) / head_dim)
    )
    t = torch.arange(max_position, dtype=torch.float32, device=device)
    freqs = torch.einsum("i,j->ij", t, inv_freq)
    return freqs.cos(), freqs.sin()


def apply_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    x1, x2 = torch.chunk(x.float(), 2, dim=-1)
    y = torch.cat((x1 * cos - x2 * sin, x2 * cos + x1 * sin), dim=-1)
    return y.to(x.dtype)


class RotaryEmbedding(nn.Module):
    def __init__(self, head_dim: int, max_position: int, base: float):
        super().__init__()
        cos, sin = rope_cos_sin(head_dim, max_position, base)
        self.register_buffer("cos", cos, persistent=False)
        self.register_buffer("sin", sin, persistent=False)

    def forward(self, positions, q, k):
        cos = self.cos[positions].unsqueeze(1)
        sin = self.sin[positions].unsqueeze(1)
        return apply_rope(q, cos, sin), apply_rope(k, cos, sin)


def _attend(q, k, v, scale, causal_offset: int | None):
    """q ``[Tq,Hq,D]``, k/v ``[Tk,Hkv,D]`` bf16 -> ``[Tq,Hq,D]`` bf16 (fp32 math)."""

    group = q.shape[1] // k.shape[1]
    kf = k.float().repeat_interleave(group, dim=1)
    vf = v.float().repeat_interleave(group, dim=1)
    scores = torch.einsum("qhd,khd->hqk", q.float(), kf) * scale
    if causal_offset is not None:
        tq, tk = q.shape[0], k.shape[0]
        qpos = torch.arange(tq, device=q.device).unsqueeze(1) + causal_offset
        kpos = torch.arange(tk, device=q.device).unsqueeze(0)
        scores = scores.masked_fill((kpos > qpos).unsqueeze(0), float("-inf"))
    probs = torch.softmax(scores, dim=-1)
    return torch.einsum("hqk,khd->qhd", probs, vf).to(q.dtype)


class Attention(nn.Module):
    def __init__(self, num_heads, head_dim, scale, num_kv_heads):
        super().__init__()
        self.num_heads = num_heads
        self.head_dim = head_dim
        self.scale = scale
        self.num_kv_heads = num_kv_heads
        self.k_cache = self.v_cache = torch.tensor([])

    def _gather(self, cache, table, length):
        bs = cache.shape[1]
        pos = torch.arange(length, device=cache.device)
        blocks = table[pos // bs].long()
        return cache[blocks, pos % bs]

    def forward(self, q, k, v, meta: AttentionMetadata):
        k_cache, v_cache = self.k_cache, self.v_cache
        has_cache = k_cache.numel() > 0
        if has_cache and meta.slot_mapping is not None:
            slots = meta.slot_mapping.long()
            keep = slots >= 0
            flat_k = k_cache.view(-1, self.num_kv_heads, self.head_dim)
            flat_v = v_cache.view(-1, self.num_kv_heads, self.head_dim)
            flat_k[slots[keep]] = k[keep]
            flat_v[slots[keep]] = v[keep]
        outs = []
        if meta.is_prefill:
            cq, ck = meta.cu_seqlens_q, meta.cu_seqlens_k
            for i in range(len(cq) - 1):
                qi = q[cq[i] : cq[i + 1]]
                len_k = ck[i + 1] - ck[i]
                if meta.block_tables is not None:
                    ki = self._gather(k_cache, meta.block_tables[i], len_k)
                    vi = self._gather(v_cache, meta.block_tables[i], len_k)
                else:
                    ki, vi = k[cq[i] : cq[i + 1]], v[cq[i] : cq[i + 1]]
                outs.append(_attend(qi, ki, vi, self.scale, len_k - qi.shape[0]))
        else:
            lens = meta.context_lens_host if meta.context_lens_host is not None else meta.context_lens.tolist()
            for b, length in enumerate(lens):
                kb = self._gather(k_cache, meta.block_tables[b], length)
                vb = self._gather(v_cache, meta.block_tables[b], length)
                outs.append(_attend(q[b : b + 1], kb, vb, self.scale, None))
        return torch.cat(outs, dim=0)


class Qwen3Attention(nn.Module):
    def __init__(self, cfg):
        super().__init__()
        self.num_heads = cfg.num_attention_heads
        self.num_kv_heads = cfg.num_key_value_heads
        self.head_dim = getattr(cfg, "head_dim", None) or cfg.hidden_size // self.num_heads
        self.q_size = self.num_heads * self.head_dim
        self.kv_size = self.num_kv_heads * self.head_dim
        self.scaling = self.head_dim ** -0.5
        h = cfg.hidden_size
        self.qkv_proj = nn.Linear(h, self.q_size + 2 * self.kv_size, bias=False)
        self.o_proj = nn.Linear(self.q_size, h, bias=False)
        self.rotary_emb = RotaryEmbedding(
            self.head_dim, cfg.max_position_embeddings, resolve_rope_theta(cfg)
        )
        self.attn = Attention(self.num_heads, self.head_dim, self.scaling, self.num_kv_heads)
        self.q_norm = RMSNorm(self.head_dim, eps=cfg.rms_norm_eps)
        self.k_norm = RMSNorm(self.head_dim, eps=cfg.rms_norm_eps)

    def forward(self, positions, x, meta):
        qkv = self.qkv_proj(x)
        q, k, v = qkv.split([self.q_size, self.kv_size, self.kv_size], dim=-1)
        q = self.q_norm(q.reshape(-1, self.num_heads, self.head_dim))
        k = self.k_norm(k.reshape(-1, self.num_kv_heads, self.head_dim))
        v = v.reshape(-1, self.num_kv_heads, self.head_dim)
        q, k = self.rotary_emb(positions, q, k)
        o = self.attn(q, k, v, meta)
        return self.o_proj(o.flatten(1))


class Qwen3MLP(nn.Module):
    def __init__(self, cfg):
        super().__init__()
        self.intermediate = cfg.intermediate_size
        self.gate_up_proj = nn.Linear(cfg.hidden_size, 2 * cfg.intermediate_size, bias=False)
        self.down_proj = nn.Linear(cfg.intermediate_size, cfg.hidden_size, bias=False)

    def forward(self, x):
        g, u = self.gate_up_proj(x).chunk(2, dim=-1)
        act = (F.silu(g.float()) * u.float()).to(x.dtype)
        return self.down_proj(act)


class Qwen3DecoderLayer(nn.Module):
    def __init__(self, cfg):
        super().__init__()
        self.self_attn = Qwen3Attention(cfg)
        self.mlp = Qwen3MLP(cfg)
        self.input_layernorm = RMSNorm(cfg.hidden_size, eps=cfg.rms_norm_eps)
        self.post_attention_layernorm = RMSNorm(cfg.hidden_size, eps=cfg.rms_norm_eps)

    def forward(self, positions, hidden, residual, meta):
        if residual is None:
            hidden, residual = self.input_layernorm(hidden), hidden
        else:
            hidden, residual = self.input_layernorm(hidden, residual)
        hidden = self.self_attn(positions, hidden, meta)
        hidden, residual = self.post_attention_layernorm(hidden, residual)
        return self.mlp(hidden), residual


class Qwen3Model(nn.Module):
    def __init__(self, cfg):
        super().__init__()
        assert_supported_rope_type(cfg)
        self.embed_tokens = nn.Embedding(cfg.vocab_size, cfg.hidden_size)
        self.layers = nn.ModuleList(Qwen3DecoderLayer(cfg) for _ in range(cfg.num_hidden_layers))
        self.norm = RMSNorm(cfg.hidden_size, eps=cfg.rms_norm_eps)

    def forward(self, input_ids, positions, meta):
        hidden = self.embed_tokens(input_ids)
        residual = None
        for layer in self.layers:
            hidden, residual = layer(positions, hidden, residual, meta)
        hidden, _ = self.norm(hidden, residual)
        return hidden


class Qwen3ForCausalLM(nn.Module):
    def __init__(self, cfg):
        super().__init__()
        if getattr(cfg, "attention_bias", False):
            raise NotImplementedError("Qwen3 with attention bias is not supported")
        self.model = Qwen3Model(cfg)
        self.lm_head = nn.Linear(cfg.hidden_size, cfg.vocab_size, bias=False)
        if getattr(cfg, "tie_word_embeddings", True):
            self.lm_head.weight = self.model.embed_tokens.weight

    def forward(self, input_ids, positions, meta):
        return self.model(input_ids, positions, meta)

    def compute_logits(self, hidden, meta: AttentionMetadata | None = None):
        if meta is not None and meta.is_prefill:
            last = torch.tensor(meta.cu_seqlens_q[1:], device=hidden.device) - 1
            hidden = hidden[last]
        return F.linear(hidden, self.lm_head.weight)


def greedy_sample(logits: torch.Tensor) -> torch.Tensor:
    """Greedy token = first index of the maximum of the fp32-cast logits."""

    return logits.float().argmax(dim=-1)


def sample(logits: torch.Tensor, temperatures: torch.Tensor, generator=None) -> torch.Tensor:
    """Greedy rows take the argmax; others sample by the Gumbel/exponential trick
    (reference ``layers/sampler.py:5-16``)."""

    logits = logits.float()
    greedy = temperatures <= 1e-10
    probs = torch.softmax(logits / temperatures.clamp_min(1e-10).unsqueeze(1), dim=-1)
    noise = torch.empty_like(probs).exponential_(1, generator=generator).clamp_min_(1e-10)
    sampled = (probs / noise).argmax(dim=-1)
    return torch.where(greedy, logits.argmax(dim=-1), sampled)


@torch.no_grad()
def load_synthetic(model: Qwen3ForCausalLM, weights) -> None:
    """Copy :class:`~nanovllm.synthetic.SyntheticWeights` into the modules."""

    inner = model.model
    inner.embed_tokens.weight.copy_(weights.embed)
    inner.norm.weight.copy_(weights.final_norm)
    for layer, w in zip(inner.layers, weights.layers):
        attn = layer.self_attn
        layer.input_layernorm.weight.copy_(w["ln_in"])
        attn.qkv_proj.weight.copy_(torch.cat([w["q"], w["k"], w["v"]], dim=0))
        attn.q_norm.weight.copy_(w["q_norm"])
        attn.k_norm.weight.copy_(w["k_norm"])
        attn.o_proj.weight.copy_(w["o"])
        layer.post_attention_layernorm.weight.copy_(w["ln_post"])
        layer.mlp.gate_up_proj.weight.copy_(torch.cat([w["gate"], w["up"]], dim=0))
        layer.mlp.down_proj.weight.copy_(w["down"])
