"""Paged-KV integer contract: bit-exact against the reference's own test cases
(tests/golden/kv_contract.json, transcribed from the reference's
test_paged_kv.py, test_kv_block_boundary.py and test_kv_cache_indexing.py),
the scheduler/BlockManager around the 255/256/257 block boundary, and the
oracle's restatement of the kernel offset."""

from __future__ import annotations

import json
import os

import pytest

from conftest import ROOT
from nanovllm.backends.megakernel.cache import PagedKVCacheSpec
from nanovllm.engine import kv_layout as kl
from oracle import kv_oracle

with open(os.path.join(ROOT, "tests", "golden", "kv_contract.json")) as f:
    GOLD = json.load(f)
BS = GOLD["block_size"]


def test_paged_spec_small_strides_slots_offsets():
    g = GOLD["paged_spec_small"]
    spec = PagedKVCacheSpec(*g["spec"])
    assert list(spec.shape) == g["shape"]
    assert (spec.token_stride, spec.block_stride, spec.layer_stride, spec.total_bytes) == (
        g["token_stride"], g["block_stride"], g["layer_stride"], g["total_bytes"])
    for table, p, want in g["physical_slot"]:
        assert list(spec.physical_slot(table, p)) == want
    for layer, table, p, head, d, want in g["element_offset"]:
        assert spec.element_offset(layer, table, p, head, d) == want
        assert kv_oracle.element_offset(layer, table, p, head, d, num_blocks=16, block_size=4,
                                        num_kv_heads=2, head_dim=8) == want
    with pytest.raises(ValueError, match="block table"):
        spec.physical_slot([], 0)
    with pytest.raises(IndexError, match="position"):
        spec.physical_slot([7], 4)
    with pytest.raises(ValueError, match="physical block"):
        spec.physical_slot([-1], 0)
    with pytest.raises(ValueError, match="positive"):
        PagedKVCacheSpec(0, 1, 4, 1, 8, 2)


def test_model_geometry_slot():
    g = GOLD["paged_spec_model"]
    spec = PagedKVCacheSpec(*g["spec"])
    assert list(spec.shape) == g["shape"]
    for table, p, want in g["physical_slot"]:
        assert list(spec.physical_slot(table, p)) == want


def test_offsets_agree_with_oracle_exhaustively_small():
    spec = PagedKVCacheSpec(3, 9, 4, 2, 8, 2)
    table = [8, 0, 5, 2]
    for layer in range(3):
        for p in range(16):
            for h in range(2):
                for d in (0, 7):
                    assert spec.element_offset(layer, table, p, h, d) == kv_oracle.element_offset(
                        layer, table, p, h, d, num_blocks=9, block_size=4, num_kv_heads=2, head_dim=8)


def _scheduler(tmpdir, blocks=64):
    from nanovllm.config import Config
    from nanovllm.engine.scheduler import Scheduler
    from nanovllm.engine.sequence import Sequence
    from nanovllm.synthetic import write_model_dir

    Sequence.block_size = BS
    cfg = Config(write_model_dir(str(tmpdir), num_layers=1), num_kvcache_blocks=blocks)
    return Scheduler(cfg)


@pytest.mark.parametrize("case", GOLD["prefill"])
def test_prefill_boundary(tmp_path, case):
    from nanovllm.engine.sequence import Sequence

    n, blocks, last = case
    sched = _scheduler(tmp_path)
    seq = Sequence([7] * n)
    sched.add(seq)
    seqs, is_prefill = sched.schedule()
    assert is_prefill and seqs == [seq]
    assert len(seq.block_table) == blocks and seq.last_block_num_tokens == last
    slots = kl.prefill_slot_mapping(seq.block_table, 0, n, BS)
    assert slots == [seq.block_table[p // BS] * BS + p % BS for p in range(n)]


@pytest.mark.parametrize("case", GOLD["first_decode"])
def test_first_decode_boundary(tmp_path, case):
    from nanovllm.engine.sequence import Sequence

    n, position, (blk_idx, off) = case
    sched = _scheduler(tmp_path)
    seq = Sequence([7] * n)
    sched.add(seq)
    sched.schedule()
    sched.postprocess([seq], [42], True)
    seqs, is_prefill = sched.schedule()
    assert not is_prefill and seqs == [seq]
    assert kl.decode_position(len(seq)) == position
    assert kl.decode_cache_seqlens(len(seq)) == position
    assert kl.decode_cache_len(len(seq)) == position + 1
    slot = kl.decode_slot_mapping(seq.block_table, len(seq), BS)
    assert slot == seq.block_table[blk_idx] * BS + off
    assert slot == kv_oracle.decode_slot(seq.block_table, len(seq), BS)


def test_decode_slot_matches_legacy_expression():
    for n, table in GOLD["decode_slot_legacy"]:
        legacy = table[-1] * BS + (n - (len(table) - 1) * BS) - 1
        assert kl.decode_slot_mapping(table, n, BS) == legacy == kv_oracle.decode_slot(table, n, BS)


def test_chunked_prefill_continues_prefix(tmp_path):
    from nanovllm.engine.sequence import Sequence

    c = GOLD["chunked_prefill"]
    sched = _scheduler(tmp_path)
    seq = Sequence([7] * c["prompt"])
    sched.add(seq)
    sched.schedule()
    suffix = kl.prefill_slot_mapping(seq.block_table, c["start"], c["end"], BS)
    assert len(suffix) == c["count"]
    assert suffix[0] == seq.block_table[c["first"][0]] * BS + c["first"][1]
    assert suffix[-1] == seq.block_table[c["last"][0]] * BS + c["last"][1]
    assert list(kl.prefill_positions(c["start"], c["count"])) == list(range(c["start"], c["end"]))


def test_slot_mapping_guards():
    with pytest.raises(RuntimeError, match="need 2 blocks"):
        kl.prefill_slot_mapping([3], 0, 257, BS)
    with pytest.raises(RuntimeError, match="allocated block table"):
        kl.prefill_slot_mapping([], 0, 4, BS)
    with pytest.raises(RuntimeError, match="may_append"):
        kl.decode_slot_mapping([3], 257, BS)
    with pytest.raises(RuntimeError, match="block table has 3"):
        kl.decode_slot_mapping([3, 4, 5], 257, BS)
    assert kl.prefill_slot_mapping([3], 4, 4, BS) == []
    for bad in (lambda: kl.prefill_positions(-1, 4), lambda: kl.decode_position(0),
                lambda: kl.decode_slot_mapping([1], 1, 0)):
        with pytest.raises(ValueError):
            bad()


def test_padding_is_block_zero_and_keeps_reads_in_bounds():
    g = GOLD["padded_tables"]
    assert kl.pad_block_table([], 1) == [GOLD["pad_value"]]
    width = max(len(g["short"]), len(g["long"]))
    spec = PagedKVCacheSpec(1, g["num_blocks"], g["block_size"], 8, 128, 2)
    for table in (g["short"], g["long"]):
        padded = kl.pad_block_table(table, width)
        assert padded == kv_oracle.pad_table(table, width)
        for p in range(width * g["block_size"]):
            off = spec.element_offset(0, padded, p, 7, 127)
            assert 0 <= off < spec.total_elements
    with pytest.raises(ValueError):
        kl.pad_block_table([1, 2, 3], 2)


def test_decode_at_boundary_appends_block_and_second_decode_stays(tmp_path):
    from nanovllm.engine.sequence import Sequence

    sched = _scheduler(tmp_path)
    seq = Sequence([7] * 256)
    sched.add(seq)
    sched.schedule()
    sched.postprocess([seq], [42], True)
    assert len(seq.block_table) == 1
    sched.schedule()
    assert len(seq.block_table) == 2
    assert kl.decode_slot_mapping(seq.block_table, len(seq), BS) == seq.block_table[1] * BS
    sched.postprocess([seq], [43], False)
    sched.schedule()
    assert kl.decode_slot_mapping(seq.block_table, len(seq), BS) == seq.block_table[1] * BS + 1
