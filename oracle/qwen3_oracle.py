"""CPU restatement of the reference torch decode step -- TEST INFRASTRUCTURE.

This is the checker for the HIP decode step, not part of it: only ``tests/``,
``__graft_entry__.smoke()`` and the CPU-baseline leg of ``bench.py`` import it.

What it restates (reference paths, file:line):

* ``models/qwen3.py:147-160`` -- decoder layer: residual-carrying
  ``add_rms`` -> qkv -> per-head q/k RMSNorm -> RoPE -> KV store -> paged decode
  attention -> o_proj -> ``add_rms`` -> gate_up -> SiLU*mul -> down;
  ``models/qwen3.py:177-187`` -- embedding, layers, final norm;
* ``layers/layernorm.py:16-40`` -- RMSNorm: fp32 math, ``x*rsqrt(mean(x^2)+eps)``
  rounded to bf16, times the bf16 weight (bf16 result); with a residual the sum
  is taken in fp32 and the new residual is that sum rounded to bf16;
* ``layers/rotary_embedding.py:6-48`` -- rotate-half RoPE on an fp32 cos/sin
  cache, ``inv_freq = theta^(-2i/d)``, theta from ``rope_config.py:25-73``;
* ``layers/activation.py:6-11`` -- ``silu(gate) * up`` (fp32, one rounding, as
  the compiled op fuses it);
* ``layers/attention.py:59-75`` -- decode attention over ``context_lens =
  position + 1`` entries through the block table, GQA (2 query heads per KV
  head), scale ``head_dim**-0.5`` (``models/qwen3.py:39``), fp32 softmax;
* ``layers/linear.py`` / ``embed_head.py:56-66`` -- bf16 GEMMs with fp32
  accumulation, bf16 outputs; tied LM head; logits are bf16;
* ``layers/sampler.py:5-16`` -- greedy token = ``logits.float().argmax(-1)``,
  the first maximal index;
* ``engine/kv_layout.py`` + ``backends/megakernel/cache.py:94-119`` -- the slot
  and element-offset arithmetic (restated in :mod:`oracle.kv_oracle`).

Written as plain functions over a weight dict (no ``nn.Module``), independently
of the package's torch path. Pinned by ``tests/test_oracle.py`` (see there for
which check pins which function).
"""

from __future__ import annotations

import math

import torch

EPS = 1e-6
ROPE_THETA = 1_000_000.0
HEAD_DIM = 128
NUM_Q_HEADS = 16
NUM_KV_HEADS = 8
BF16 = torch.bfloat16


def bf16(x: torch.Tensor) -> torch.Tensor:
    return x.to(BF16)


def rms_norm(x32: torch.Tensor, weight: torch.Tensor, eps: float = EPS) -> torch.Tensor:
    """``bf16(bf16(x * rsqrt(mean(x^2) + eps)) * w)`` over the last dim; x is fp32."""

    scale = torch.rsqrt(x32.pow(2).mean(dim=-1, keepdim=True) + eps)
    return bf16(bf16(x32 * scale).float() * weight.float())


def add_rms_norm(hidden: torch.Tensor, residual: torch.Tensor | None, weight, eps=EPS):
    """Returns ``(normed bf16, new residual bf16)``; ``residual=None`` is layer 0."""

    s = hidden.float() if residual is None else hidden.float() + residual.float()
    return rms_norm(s, weight, eps), bf16(s)


def rope_tables(max_position: int = 2048, theta: float = ROPE_THETA, head_dim: int = HEAD_DIM):
    inv_freq = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.float32) / head_dim))
    freqs = torch.arange(max_position, dtype=torch.float32)[:, None] * inv_freq[None, :]
    return torch.cos(freqs), torch.sin(freqs)


def rope(x_bf16: torch.Tensor, cos_row: torch.Tensor, sin_row: torch.Tensor) -> torch.Tensor:
    """Rotate-half RoPE of ``[..., head_dim]`` at one position (fp32 math, bf16 out)."""

    half = x_bf16.shape[-1] // 2
    x = x_bf16.float()
    x1, x2 = x[..., :half], x[..., half:]
    return bf16(torch.cat((x1 * cos_row - x2 * sin_row, x2 * cos_row + x1 * sin_row), dim=-1))


def linear(x_bf16: torch.Tensor, w32: torch.Tensor) -> torch.Tensor:
    """``bf16(x @ W^T)`` with fp32 products/accumulation (``w32`` is the fp32 copy)."""

    return bf16(x_bf16.float() @ w32.t())


def silu_mul(gate_bf16: torch.Tensor, up_bf16: torch.Tensor) -> torch.Tensor:
    g = gate_bf16.float()
    return bf16(g / (1.0 + torch.exp(-g)) * up_bf16.float())


def attention_one(q, keys, values, scale=HEAD_DIM ** -0.5):
    """One row: q ``[Hq, D]`` bf16, keys/values ``[T, Hkv, D]`` bf16 -> ``[Hq, D]`` bf16."""

    group = q.shape[0] // keys.shape[1]
    out = []
    for hq in range(q.shape[0]):
        kv = hq // group
        s = (keys[:, kv, :].float() @ q[hq].float()) * scale
        p = torch.softmax(s, dim=0)
        out.append(p @ values[:, kv, :].float())
    return bf16(torch.stack(out))


def argmax_first(values: torch.Tensor) -> int:
    """Index of the first maximal element (``torch.argmax`` rule: a NaN ranks
    above every number, so the first NaN wins when there is one)."""

    best, idx = None, -1
    flat = values.float().tolist()
    for i, v in enumerate(flat):
        if v != v:
            return i
        if best is None or v > best:
            best, idx = v, i
    return idx


class Oracle:
    """Holds fp32 weight copies; runs decode steps against a paged KV cache.

    ``weights`` is a :class:`nanovllm.synthetic.SyntheticWeights`-like object
    (``layers``, ``embed``, ``final_norm``). The caches are bf16 tensors shaped
    ``[layers, blocks, block_size, kv_heads, head_dim]`` and are updated in
    place exactly where the decode step writes.
    """

    def __init__(self, weights, max_position: int = 2048, theta: float = ROPE_THETA):
        self.w = weights
        self.num_layers = len(weights.layers)
        f32 = lambda t: t.float()  # noqa: E731
        self.layers32 = [
            {k: f32(v) for k, v in layer.items() if v.dim() == 2} for layer in weights.layers
        ]
        self.embed32 = f32(weights.embed)
        self.cos, self.sin = rope_tables(max_position, theta)

    def _attention(self, l, q_heads, k_new, v_new, k_cache, v_cache, table, pos, active):
        bs = k_cache.shape[2]
        if active:
            blk, off = int(table[pos // bs]), pos % bs
            k_cache[l, blk, off] = k_new
            v_cache[l, blk, off] = v_new
        positions = torch.arange(pos + 1)
        blocks = torch.as_tensor([int(table[p // bs]) for p in range(pos + 1)], dtype=torch.long)
        keys = k_cache[l, blocks, positions % bs].clone()
        vals = v_cache[l, blocks, positions % bs].clone()
        # The row's own new token is always attended with its fresh K/V, also
        # when the cache write is masked off (inactive row).
        keys[pos], vals[pos] = k_new, v_new
        return attention_one(q_heads, keys, vals)

    def decode_step(self, input_ids, positions, block_tables, k_cache, v_cache,
                    row_active=None, trace: dict | None = None):
        """One greedy decode step for ``B`` rows.

        ``positions[b]`` is the pre-decode cache length (= the position this
        token is written to); ``block_tables[b]`` its page list. Returns
        ``(logits bf16 [B, V], tokens list[int])``. When ``trace`` is a dict it
        receives the last layer's intermediates (``qkv``, ``attn``, ``o``,
        ``act``, ``down``, ``resid_post``) for per-op comparisons.
        """

        hidden, residual = self.embed_rows(input_ids), None
        for l in range(self.num_layers):
            hidden, residual = self.layer(l, hidden, residual, positions, block_tables, k_cache, v_cache,
                                          row_active=row_active, trace=trace)
        return self.head(hidden, residual)

    def embed_rows(self, input_ids) -> torch.Tensor:
        """bf16 embedding rows of the step's token ids (``models/qwen3.py:177-181``)."""

        return self.w.embed[torch.as_tensor(list(input_ids), dtype=torch.long)]

    def layer(self, l, hidden, residual, positions, block_tables, k_cache, v_cache,
              row_active=None, trace: dict | None = None):
        """Decoder layer ``l`` (``models/qwen3.py:147-160``) on bf16 ``hidden`` and
        ``residual`` (``None`` at layer 0): returns ``(down output, residual after
        the post-attention add)``, the pair the next layer (or the final norm)
        adds. Writes the rows' K/V into the caches where the step writes them."""

        rows = hidden.shape[0]
        active = [True] * rows if row_active is None else [bool(a) for a in row_active]
        w, w32 = self.w.layers[l], self.layers32[l]
        h, residual = add_rms_norm(hidden, residual, w["ln_in"])
        q = linear(h, w32["q"]).view(rows, NUM_Q_HEADS, HEAD_DIM)
        k = linear(h, w32["k"]).view(rows, NUM_KV_HEADS, HEAD_DIM)
        v = linear(h, w32["v"]).view(rows, NUM_KV_HEADS, HEAD_DIM)
        if trace is not None:
            trace["qkv"] = torch.cat([q.reshape(rows, -1), k.reshape(rows, -1), v.reshape(rows, -1)], -1)
            trace["resid_in"] = residual
        q = rms_norm(q.float(), w["q_norm"])
        k = rms_norm(k.float(), w["k_norm"])
        attn = []
        for b in range(rows):
            pos = int(positions[b])
            qb = rope(q[b], self.cos[pos], self.sin[pos])
            kb = rope(k[b], self.cos[pos], self.sin[pos])
            attn.append(self._attention(l, qb, kb, v[b], k_cache, v_cache,
                                        block_tables[b], pos, active[b]))
        attn_flat = torch.stack(attn).reshape(rows, -1)
        o = linear(attn_flat, w32["o"])
        h, residual = add_rms_norm(o, residual, w["ln_post"])
        gate, up = linear(h, w32["gate"]), linear(h, w32["up"])
        act = silu_mul(gate, up)
        hidden = linear(act, w32["down"])
        if trace is not None:
            trace.update(attn=attn_flat, o=o, gate=gate, up=up, act=act, down=hidden, resid_post=residual)
        return hidden, residual

    def head(self, hidden, residual):
        """Final RMSNorm, tied LM head (bf16 logits) and greedy tokens
        (``models/qwen3.py:183-187``, ``embed_head.py:56-66``, ``sampler.py:5-16``)."""

        h, _ = add_rms_norm(hidden, residual, self.w.final_norm)
        logits = linear(h, self.embed32)
        tokens = logits.float().argmax(dim=-1).tolist()
        return logits, tokens

    def teacher_force(self, token_ids, block_table, k_cache, v_cache, start: int = 0):
        """Write K/V for ``token_ids`` at positions ``start..`` one decode step at a
        time (mathematically the causal prefill). Returns the last step's output."""

        out = None
        for i, tok in enumerate(token_ids):
            out = self.decode_step([tok], [start + i], [block_table], k_cache, v_cache)
        return out
