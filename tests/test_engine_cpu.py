"""Plugin surface on the CPU: admission (reference reason strings), the Qwen3
contract, config validation, the runner's fallback reporting, and the
engine end to end on the torch path."""

from __future__ import annotations

import os
import warnings
from types import SimpleNamespace

import pytest

from conftest import ROOT
from nanovllm.backends.megakernel import (
    MegakernelBackend, TG_MAX_BATCH, gcn_arch_supported, qwen3_contract_mismatch, taskgraph_compatibility,
)
from nanovllm.backends.megakernel.row_contract import row_active_mask


def _cfg(**kw):
    hf = SimpleNamespace(tie_word_embeddings=True, attention_bias=False, model_type="qwen3", hidden_size=1024,
                         intermediate_size=3072, num_hidden_layers=28, num_attention_heads=16,
                         num_key_value_heads=8, vocab_size=151936, head_dim=128)
    for k, v in kw.pop("hf", {}).items():
        setattr(hf, k, v)
    base = dict(hf_config=hf, max_num_seqs=8, tensor_parallel_size=1, max_model_len=2048)
    base.update(kw)
    return SimpleNamespace(**base)


def _seq(t=0.0):
    return SimpleNamespace(temperature=t, is_greedy=t <= 1e-10)


def test_admission_reasons():
    cfg = _cfg()
    assert taskgraph_compatibility(cfg, [_seq()], True).reason == \
        "Task-graph megakernel is decode-only; use the prefill backend"
    assert taskgraph_compatibility(cfg, [], False).reason == "Task-graph megakernel needs at least one sequence"
    assert "batch sizes 1..8" in taskgraph_compatibility(cfg, [_seq()] * 9, False).reason
    assert taskgraph_compatibility(_cfg(max_num_seqs=2), [_seq()] * 3, False).reason == \
        "batch 3 exceeds max_num_seqs=2"
    assert taskgraph_compatibility(_cfg(tensor_parallel_size=2), [_seq()], False).reason == \
        "Task-graph megakernel requires tensor_parallel_size=1"
    assert taskgraph_compatibility(cfg, [_seq(0.7)], False).reason == \
        "Task-graph megakernel supports greedy sampling only"
    for n in range(1, TG_MAX_BATCH + 1):
        assert taskgraph_compatibility(cfg, [_seq()] * n, False).supported


def test_qwen3_contract():
    assert qwen3_contract_mismatch(_cfg()) is None
    assert qwen3_contract_mismatch(_cfg(hf={"tie_word_embeddings": False})) == "tie_word_embeddings"
    assert qwen3_contract_mismatch(_cfg(hf={"attention_bias": True})) == "attention_bias"
    assert qwen3_contract_mismatch(_cfg(hf={"num_hidden_layers": 2})) == "num_hidden_layers"
    assert qwen3_contract_mismatch(_cfg(max_model_len=4096)) == "max_model_len"
    assert MegakernelBackend.compatibility(_cfg(hf={"vocab_size": 1000}), [_seq()], False).reason == \
        "unsupported Qwen config: vocab_size"


def test_backend_surface_without_gpu():
    be = MegakernelBackend(_cfg(), model=None)
    with pytest.raises(ValueError, match="kv_cache must have shape"):
        be.set_kv_cache(None)
    assert not be.ready
    be.disable("manual")
    with pytest.raises(RuntimeError, match="manual"):
        be.ensure_ready()
    assert gcn_arch_supported("gfx950:sramecc+:xnack-") and not gcn_arch_supported("gfx942")


def test_row_active_mask():
    assert row_active_mask(None, 3) == [1, 1, 1]
    assert row_active_mask([True, 0, 5], 3) == [1, 0, 1]
    with pytest.raises(ValueError):
        row_active_mask([1], 2)
    with pytest.raises(ValueError):
        row_active_mask([0, 0], 2)


def test_config_validation(tmp_path):
    from nanovllm.config import Config
    from nanovllm.synthetic import write_model_dir

    path = write_model_dir(str(tmp_path), num_layers=1)
    with pytest.raises(ValueError, match="decode_backend"):
        Config(path, decode_backend="cuda")
    with pytest.raises(ValueError, match="multiple of 256"):
        Config(path, kvcache_block_size=128)
    with pytest.raises(ValueError, match="megakernel_launch"):
        Config(path, megakernel_launch="eager")
    with pytest.raises(ValueError, match="does not exist"):
        Config(str(tmp_path / "missing"))
    cfg = Config(path, max_model_len=1 << 20)
    assert cfg.max_model_len == 40960 and cfg.hf_config.num_hidden_layers == 1


def test_engine_megakernel_falls_back_with_reason_on_cpu(tmp_path):
    """No GPU here: the backend is disabled at startup with an explicit reason,
    and every decode step reports the torch path plus that reason."""
    from nanovllm import LLM, SamplingParams
    from nanovllm.synthetic import write_model_dir

    path = write_model_dir(str(tmp_path / "model_2l"), num_layers=2)
    with warnings.catch_warnings(record=True) as caught:
        warnings.simplefilter("always")
        llm = LLM(path, max_model_len=2048, num_kvcache_blocks=4, decode_backend="megakernel")
    assert any("Megakernel disabled at startup" in str(w.message) for w in caught)
    res = llm.generate_with_metrics([[5, 6, 7]], SamplingParams(temperature=0.0, max_tokens=3, ignore_eos=True))
    m = res["metrics"]
    assert m["decode_backends"] == {"torch": 2}
    assert list(m["fallback_reasons"]) == ["Megakernel requires a ROCm (HIP) device"]
    assert len(res["outputs"][0]["token_ids"]) == 3


def test_engine_megakernel_warns_on_long_max_model_len(tmp_path):
    from nanovllm import LLM
    from nanovllm.synthetic import write_model_dir

    path = write_model_dir(str(tmp_path / "model_2l"), num_layers=2)
    with pytest.warns(RuntimeWarning, match="requires max_model_len <= 2048"):
        LLM(path, max_model_len=4096, num_kvcache_blocks=4, decode_backend="megakernel")


def test_scheduler_batches_and_preempts(tmp_path):
    from nanovllm import SamplingParams
    from nanovllm.config import Config
    from nanovllm.engine.scheduler import Scheduler
    from nanovllm.engine.sequence import Sequence
    from nanovllm.synthetic import write_model_dir

    Sequence.block_size = 256
    cfg = Config(write_model_dir(str(tmp_path), num_layers=1), num_kvcache_blocks=3, max_num_seqs=4)
    sched = Scheduler(cfg)
    seqs = [Sequence([1] * 200, SamplingParams(max_tokens=100)) for _ in range(3)]
    for s in seqs:
        sched.add(s)
    picked, prefill = sched.schedule()
    assert prefill and len(picked) == 3
    sched.postprocess(picked, [9, 9, 9], True)
    for _ in range(60):   # grow until the pool is exhausted: someone must be preempted
        picked, prefill = sched.schedule()
        if prefill:
            break
        sched.postprocess(picked, [9] * len(picked), False)
    assert sched.block_manager.stats()["allocated_blocks"] <= 3
    assert any(s.status.name == "WAITING" for s in seqs) or prefill


def test_safetensors_checkpoint_round_trip(tmp_path):
    """The checkpoint loader (reference ``utils/loader.py:12-28``) reads Hugging Face
    names. q/k/v and gate/up are separate tensors there, and it packs them into the
    fused projections. The synthetic model is written as such a checkpoint, with the
    fused tensors split and the tied ``lm_head.weight`` included. Loaded back, it must
    give bit-identical parameters and the same greedy tokens."""
    import shutil

    import torch
    from safetensors.torch import save_file

    from nanovllm import LLM, SamplingParams
    from nanovllm.synthetic import write_model_dir

    src = write_model_dir(str(tmp_path / "synthetic"), num_layers=2)
    ref = LLM(src, max_model_len=2048, num_kvcache_blocks=4, decode_backend="torch")
    model = ref.model_runner.model
    attn = model.model.layers[0].self_attn
    tensors = {}
    for name, p in model.named_parameters():
        t = p.detach().cpu().contiguous()
        if "qkv_proj" in name:
            q, k, v = t.split([attn.q_size, attn.kv_size, attn.kv_size])
            for short, part in (("q_proj", q), ("k_proj", k), ("v_proj", v)):
                tensors[name.replace("qkv_proj", short)] = part.contiguous()
        elif "gate_up_proj" in name:
            g, u = t.chunk(2)
            tensors[name.replace("gate_up_proj", "gate_proj")] = g.contiguous()
            tensors[name.replace("gate_up_proj", "up_proj")] = u.contiguous()
        else:
            tensors[name] = t
    tensors["lm_head.weight"] = model.model.embed_tokens.weight.detach().cpu().clone()
    assert any(k.endswith("self_attn.k_proj.weight") for k in tensors)
    ckpt = tmp_path / "checkpoint"
    ckpt.mkdir()
    shutil.copy(os.path.join(src, "config.json"), ckpt / "config.json")
    names = sorted(tensors)
    half = len(names) // 2   # two shards, as multi-file checkpoints have
    save_file({k: tensors[k] for k in names[:half]}, str(ckpt / "model-00001-of-00002.safetensors"))
    save_file({k: tensors[k] for k in names[half:]}, str(ckpt / "model-00002-of-00002.safetensors"))

    loaded = LLM(str(ckpt), max_model_len=2048, num_kvcache_blocks=4, decode_backend="torch")
    got = dict(loaded.model_runner.model.named_parameters())
    for name, p in model.named_parameters():
        assert torch.equal(p.detach().cpu(), got[name].detach().cpu()), name
    sp = SamplingParams(temperature=0.0, max_tokens=4, ignore_eos=True)
    prompts = [[11, 22, 33, 44, 55], [7] * 20]
    assert loaded.generate(prompts, sp) == ref.generate(prompts, sp)
    empty = tmp_path / "no_weights"
    empty.mkdir()
    shutil.copy(os.path.join(src, "config.json"), empty / "config.json")
    with pytest.raises(FileNotFoundError, match="no safetensors"):
        LLM(str(empty), max_model_len=2048, num_kvcache_blocks=4)


def test_page_pool_prefix_reuse_and_revival():
    """Full pages are keyed by content: a second prompt with the same prefix maps
    the first one's pages (shared, ref-counted), a released prefix stays
    reusable until its pages are handed out again, and the last page is never
    shared (reference engine/block_manager.py:26-143 behaviour)."""
    from nanovllm.engine.block_manager import BlockManager
    from nanovllm.engine.sequence import Sequence

    Sequence.block_size = 4
    pool = BlockManager(num_blocks=8, block_size=4)
    a = Sequence(list(range(10)))                       # pages [0-3] [4-7] [8,9]
    assert pool.can_allocate(a) == 0
    pool.allocate(a, 0)
    a.num_scheduled_tokens = 10
    pool.hash_blocks(a)                                 # keys the two full pages
    a.num_cached_tokens, a.num_scheduled_tokens = 10, 0
    b = Sequence(list(range(8)) + [99, 98, 97])         # same two full pages, different tail
    assert pool.can_allocate(b) == 2
    pool.allocate(b, 2)
    assert b.block_table[:2] == a.block_table[:2] and b.block_table[2] != a.block_table[2]
    assert b.num_cached_tokens == 8 and pool.stats()["allocated_blocks"] == 4
    a_pages = list(a.block_table)
    pool.deallocate(a)
    pool.deallocate(b)
    assert pool.stats()["allocated_blocks"] == 0 and not a.block_table
    c = Sequence(list(range(9)))                        # revives the freed, still-keyed prefix pages
    assert pool.can_allocate(c) == 2
    pool.allocate(c, 2)
    assert c.block_table[:2] == a_pages[:2]
    # a decode step needs a page exactly when the length becomes 1 mod the page size
    d = Sequence([5] * 4)
    pool.allocate(d, pool.can_allocate(d))
    d.append_token(6)
    assert len(d) % 4 == 1 and pool.can_append(d)
    before = len(d.block_table)
    pool.may_append(d)
    assert len(d.block_table) == before + 1
    d.append_token(7)
    pool.may_append(d)
    assert len(d.block_table) == before + 1
    s = pool.stats()
    assert s["prefix_cache_hits"] == 4 and s["freed_blocks"] == 4
