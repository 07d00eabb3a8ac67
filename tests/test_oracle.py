"""Pins the CPU oracle (oracle/qwen3_oracle.py) against checks that do not
retype its formulas:

* rms_norm: exact invariances (power-of-two scaling; a constant vector maps to
  the weight) and a float64 textbook RMSNorm within one bf16 rounding;
* rope: identity at position 0, norm preservation, and equality with the
  complex-multiplication form (x1 + i x2) * exp(i p theta^(-2j/d)) in float64;
* attention_one: torch's scaled_dot_product_attention (library routine) on the
  same bf16 inputs, a one-position context returning V exactly, and a
  pure-Python double loop on a tiny case;
* linear / silu_mul / argmax_first: float64 matmul, torch's silu, torch.argmax
  and an explicit tie case (first maximal index);
* the whole decode step: Hugging Face transformers' Qwen3ForCausalLM (an
  independent implementation of the same architecture) on the same weights,
  and the package's torch path; plus the committed C1 golden fixture.
"""

from __future__ import annotations

import json
import math
import os

import numpy as np
import pytest
import torch

from conftest import ROOT, synthetic_weights
from oracle import qwen3_oracle as orc


def test_rms_norm_power_of_two_scale_invariance():
    g = torch.Generator().manual_seed(1)
    x = torch.randn(3, 1024, generator=g)
    w = (1 + 0.1 * torch.randn(1024, generator=g)).to(torch.bfloat16)
    assert torch.equal(orc.rms_norm(x, w), orc.rms_norm(x * 8.0, w))


def test_rms_norm_constant_vector_gives_weight():
    w = (1 + 0.1 * torch.randn(128)).to(torch.bfloat16)
    for c in (0.37, -5.0, 1e3):
        out = orc.rms_norm(torch.full((128,), c), w, eps=0.0)
        assert torch.equal(out, (w.float() * math.copysign(1.0, c)).to(torch.bfloat16))


def test_rms_norm_matches_float64_textbook():
    g = torch.Generator().manual_seed(2)
    x = torch.randn(4, 1024, generator=g).to(torch.bfloat16)
    w = (1 + 0.02 * torch.randn(1024, generator=g)).to(torch.bfloat16)
    x64 = x.double().numpy()
    ref = x64 / np.sqrt((x64 ** 2).mean(-1, keepdims=True) + 1e-6) * w.double().numpy()
    got = orc.rms_norm(x.float(), w).double().numpy()
    assert np.abs(got - ref).max() <= 2 * 2.0 ** -7 * np.abs(ref).max()


def test_rope_identity_at_position_zero_and_norm_preserving():
    cos, sin = orc.rope_tables(64)
    x = torch.randn(2, 128).to(torch.bfloat16)
    assert torch.equal(orc.rope(x, cos[0], sin[0]), x)
    y = orc.rope(x, cos[37], sin[37]).float()
    assert torch.allclose(y.norm(dim=-1), x.float().norm(dim=-1), rtol=1e-2)


def test_rope_matches_complex_rotation():
    cos, sin = orc.rope_tables(2048)
    g = torch.Generator().manual_seed(3)
    x = torch.randn(128, generator=g).to(torch.bfloat16)
    for p in (1, 255, 1999):
        theta = 1e6 ** (-np.arange(0, 128, 2) / 128.0)
        z = (x[:64].double().numpy() + 1j * x[64:].double().numpy()) * np.exp(1j * p * theta)
        ref = np.concatenate([z.real, z.imag])
        got = orc.rope(x, cos[p], sin[p]).double().numpy()
        assert np.abs(got - ref).max() <= 2.0 ** -6 * max(1.0, np.abs(ref).max())


def test_attention_matches_sdpa_and_edge_cases():
    g = torch.Generator().manual_seed(4)
    q = torch.randn(16, 128, generator=g).to(torch.bfloat16)
    k = torch.randn(300, 8, 128, generator=g).to(torch.bfloat16)
    v = torch.randn(300, 8, 128, generator=g).to(torch.bfloat16)
    got = orc.attention_one(q, k, v).float()
    kk = k.float().repeat_interleave(2, dim=1).permute(1, 0, 2)
    vv = v.float().repeat_interleave(2, dim=1).permute(1, 0, 2)
    ref = torch.nn.functional.scaled_dot_product_attention(q.float()[:, None, :], kk, vv).squeeze(1)
    assert (got - ref).abs().max() <= 2.0 ** -7
    one = orc.attention_one(q, k[:1], v[:1])
    assert torch.equal(one, v[0].repeat_interleave(2, dim=0))


def test_attention_tiny_brute_force():
    g = torch.Generator().manual_seed(5)
    q = torch.randn(2, 4, generator=g).to(torch.bfloat16)
    k = torch.randn(3, 1, 4, generator=g).to(torch.bfloat16)
    v = torch.randn(3, 1, 4, generator=g).to(torch.bfloat16)
    got = orc.attention_one(q, k, v, scale=0.5).double()
    for h in range(2):
        s = [sum(float(q[h, d]) * float(k[t, 0, d]) for d in range(4)) * 0.5 for t in range(3)]
        m = max(s)
        e = [math.exp(x - m) for x in s]
        for d in range(4):
            ref = sum(e[t] * float(v[t, 0, d]) for t in range(3)) / sum(e)
            assert abs(got[h, d].item() - ref) <= 2.0 ** -8 * max(1.0, abs(ref))


def test_linear_silu_argmax():
    g = torch.Generator().manual_seed(6)
    x = torch.randn(2, 512, generator=g).to(torch.bfloat16)
    w = (0.02 * torch.randn(64, 512, generator=g)).to(torch.bfloat16)
    ref = x.double().numpy() @ w.double().numpy().T
    assert np.abs(orc.linear(x, w.float()).double().numpy() - ref).max() <= 2.0 ** -8 * np.abs(ref).max()
    a = torch.randn(100, generator=g).to(torch.bfloat16)
    b = torch.randn(100, generator=g).to(torch.bfloat16)
    assert torch.equal(orc.silu_mul(a, b), (torch.nn.functional.silu(a.float()) * b.float()).to(torch.bfloat16))
    vals = torch.tensor([0.5, 2.0, -1.0, 2.0, 1.0])
    assert orc.argmax_first(vals) == 1 == int(torch.argmax(vals))
    # NaN ranks above every number in torch.argmax; the first NaN wins
    nan = float("nan")
    for case in ([0.5, nan, 3.0, nan], [nan, 1.0], [1.0, 2.0, nan], [float("inf"), nan, 0.0]):
        t = torch.tensor(case)
        assert orc.argmax_first(t) == int(torch.argmax(t)), case
    # the same rule over bf16 logits with exact ties spread through the array
    g2 = torch.Generator().manual_seed(11)
    for _ in range(50):
        v = torch.randint(-3, 4, (300,), generator=g2).to(torch.bfloat16)
        assert orc.argmax_first(v) == int(torch.argmax(v.float()))


def _hf_qwen3(num_layers, weights):
    from transformers import Qwen3Config, Qwen3ForCausalLM

    from nanovllm.synthetic import hf_config_dict

    cfg = Qwen3Config(**{k: v for k, v in hf_config_dict(num_layers=num_layers).items()
                         if k not in ("architectures", "torch_dtype")})
    cfg._attn_implementation = "eager"
    model = Qwen3ForCausalLM(cfg).to(torch.bfloat16).eval()
    sd = {"model.embed_tokens.weight": weights.embed, "model.norm.weight": weights.final_norm,
          "lm_head.weight": weights.embed}
    names = {"ln_in": "input_layernorm", "q": "self_attn.q_proj", "k": "self_attn.k_proj",
             "v": "self_attn.v_proj", "q_norm": "self_attn.q_norm", "k_norm": "self_attn.k_norm",
             "o": "self_attn.o_proj", "ln_post": "post_attention_layernorm", "gate": "mlp.gate_proj",
             "up": "mlp.up_proj", "down": "mlp.down_proj"}
    for i, layer in enumerate(weights.layers):
        for key, name in names.items():
            sd[f"model.layers.{i}.{name}.weight"] = layer[key]
    model.load_state_dict(sd, strict=False)
    return model


def test_decode_step_matches_huggingface_qwen3():
    """Prefill by teacher forcing then one decode step, vs HF on the full sequence."""
    weights = synthetic_weights(2)
    oracle = orc.Oracle(weights)
    prompt = [11, 4096, 77777, 151935, 3]
    kc = torch.zeros(2, 1, 256, 8, 128, dtype=torch.bfloat16)
    vc = torch.zeros_like(kc)
    logits, _ = oracle.teacher_force(prompt, [0], kc, vc)
    model = _hf_qwen3(2, weights)
    with torch.no_grad():
        ref = model(torch.tensor([prompt])).logits[0, -1].float()
    err = (logits[0].float() - ref).abs().max().item()
    assert err <= 4e-2, err
    assert int(logits[0].float().argmax()) == int(ref.argmax())


def test_package_torch_path_matches_oracle_first_tokens(tmp_path):
    from nanovllm import LLM, SamplingParams
    from nanovllm.synthetic import write_model_dir

    path = write_model_dir(str(tmp_path / "model_2l"), num_layers=2)
    llm = LLM(path, max_model_len=2048, num_kvcache_blocks=4, decode_backend="torch")
    out = llm.generate([[1, 2, 3, 4, 5, 6, 7, 8]], SamplingParams(temperature=0.0, max_tokens=4, ignore_eos=True))
    oracle = orc.Oracle(synthetic_weights(2))
    kc = torch.zeros(2, 1, 256, 8, 128, dtype=torch.bfloat16)
    vc = torch.zeros_like(kc)
    _, toks = oracle.teacher_force([1, 2, 3, 4, 5, 6, 7, 8], [0], kc, vc)
    seq = [toks[0]]
    for i in range(3):
        _, t = oracle.decode_step([seq[-1]], [8 + i], [[0]], kc, vc)
        seq.append(t[0])
    assert out[0]["token_ids"] == seq


def test_c1_golden_first_steps():
    """The committed C1 fixture (full 28-layer model) reproduces: prompt, first
    greedy token and the first step's top logits."""
    with open(os.path.join(ROOT, "tests", "golden", "c1_greedy.json")) as f:
        gold = json.load(f)
    gen = torch.Generator().manual_seed(0)
    assert torch.randint(0, 151936, (16,), generator=gen).tolist() == gold["prompt"]
    oracle = orc.Oracle(synthetic_weights(28))
    kc = torch.zeros(28, 1, 256, 8, 128, dtype=torch.bfloat16)
    vc = torch.zeros_like(kc)
    logits, toks = oracle.teacher_force(gold["prompt"], [0], kc, vc)
    assert toks[0] == gold["tokens"][0]
    top = torch.topk(logits[0].float(), 8)
    assert top.indices.tolist() == gold["first_step_top8_ids"]
    assert torch.allclose(top.values, torch.tensor(gold["first_step_top8_logits"]))
