"""Task-graph generator + verifier (CPU): every supported geometry verifies
(deadlock-free by maximal execution, exact arrivals, single ownership), and
the verifier rejects mutated schedules."""

from __future__ import annotations

import copy
import dataclasses

import pytest

from nanovllm.backends.megakernel import native
from nanovllm.backends.megakernel.schedule import (
    Task, auto_attn_splits, batch_bucket, build_schedule, build_segments, split_layers,
)
from nanovllm.backends.megakernel.verifier import arrivals, ownership, simulate, verify


@pytest.mark.parametrize("batch", [1, 2, 4, 8])
@pytest.mark.parametrize("grid", [1, 7, 64, 256])
@pytest.mark.parametrize("splits", [1, 4, 16])
def test_geometries_verify(batch, grid, splits):
    layers = 2 if grid < 64 else 28
    sched = build_schedule(batch, splits, grid, layers)
    assert verify(sched) == []


def test_segments_cover_the_step_and_verify_jointly():
    whole = build_schedule(2, 2, 256, 28)
    segs = build_segments(2, 2, 256, 28, groups=4)
    assert sum(s.num_tasks for s in segs) == whole.num_tasks
    assert split_layers(28, 4) == [(0, 7), (7, 14), (14, 21), (21, 28)]
    # running the segments back to back is the whole schedule run in order
    merged = dataclasses.replace(whole, rows=[sum((s.rows[g] for s in segs), []) for g in range(256)])
    assert simulate(merged) == []


def test_task_counts_at_256_cus():
    s = build_schedule(1, 1, 256, 28)
    by_op = {}
    for st in s.stages:
        by_op.setdefault(st.op, []).append(len(st.tasks))
    assert by_op[native.OP_QKV][0] == 256 and by_op[native.OP_OPROJ][0] == 256
    assert by_op[native.OP_GATEUP][0] == 256 and by_op[native.OP_DOWN][0] == 256
    assert by_op[native.OP_ATTN][0] == 8 and by_op[native.OP_LMHEAD] == [256]
    assert s.lm_slots == 256


def _mutate(sched, fn):
    m = copy.deepcopy(sched)
    fn(m)
    return m


def test_verifier_rejects_mutants():
    base = build_schedule(1, 2, 16, 2)
    assert verify(base) == []

    def wrong_count(m):
        t = m.stages[2].tasks[0]
        m.stages[2].tasks[0] = dataclasses.replace(t, wait_count=t.wait_count + 1)
        m.rows = [[m.stages[2].tasks[0] if x is t else x for x in r] for r in m.rows]

    def reversed_row(m):
        m.rows[0] = list(reversed(m.rows[0]))

    def duplicate_row(m):
        t = m.stages[0].tasks[1]
        m.stages[0].tasks[1] = dataclasses.replace(t, a0=m.stages[0].tasks[0].a0)

    def missing_signal(m):
        t = m.stages[4].tasks[0]
        new = dataclasses.replace(t, signal=-1)
        m.stages[4].tasks[0] = new
        m.rows = [[new if x is t else x for x in r] for r in m.rows]

    assert arrivals(_mutate(base, wrong_count))
    assert simulate(_mutate(base, reversed_row))
    assert ownership(_mutate(base, duplicate_row))
    assert arrivals(_mutate(base, missing_signal)) or simulate(_mutate(base, missing_signal))


def test_instruction_words_and_padding():
    s = build_schedule(1, 1, 4, 1)
    flat, counts = s.persistent_words()
    assert len(flat) == 4 * s.max_inst * native.INST_WORDS
    assert sum(counts) == s.num_tasks
    words, table = s.stage_words()
    assert sum(c for _, _, _, c in table) == s.num_tasks
    assert Task(1, 0, 2, 3, 4, 5, 6, 7).words() == [1, 0, 2, 3, 4, 5, 6, 7]


def test_buckets_and_auto_splits():
    assert [batch_bucket(r) for r in range(1, 9)] == [1, 2, 4, 4, 8, 8, 8, 8]
    with pytest.raises(ValueError):
        batch_bucket(9)
    assert auto_attn_splits(1) == 1 and auto_attn_splits(256) == 1 and auto_attn_splits(257) == 2
    assert auto_attn_splits(2048) == 8 and auto_attn_splits(10 ** 6) == 16
    assert auto_attn_splits(100, minimum=4) == 4
    # batch cap: batch x splits <= 16, the minimum still wins
    assert [auto_attn_splits(2048, batch=b) for b in (1, 2, 4, 8)] == [8, 8, 4, 2]
    assert auto_attn_splits(10 ** 6, batch=2) == 8 and auto_attn_splits(300, batch=8) == 2
    assert auto_attn_splits(200, batch=8) == 1 and auto_attn_splits(2048, minimum=8, batch=8) == 8


@pytest.mark.parametrize("batch", [1, 2, 4, 8])
@pytest.mark.parametrize("splits", [1, 2, 4, 8, 16])
def test_tagged_exchange_preconditions_at_256_cus(batch, splits):
    """Even GEMV row blocks of <= 32 rows and an LM task on every workgroup, with
    attention tasks of one query head (flagged) or of both heads of a KV head."""
    from nanovllm.backends.megakernel.taskgraph import _check_tagged_preconditions
    for pair in (False, True):
        for groups in (1, 4):
            segs = build_segments(batch, splits, 256, 28, groups, q_head_tasks=True, pair_heads=pair)
            _check_tagged_preconditions(segs)
            attn = [t for seg in segs for st in seg.stages if st.op == native.OP_ATTN for t in st.tasks]
            # every (row, KV head, split, query head) exactly once per layer
            assert len(attn) == 28 * batch * 8 * splits * (1 if pair else 2)
            heads = {(t.a0 & native.ATTN_QHEAD) // native.ATTN_QHEAD for t in attn}
            assert all(bool(t.a0 & native.ATTN_ONE_HEAD) != pair for t in attn)
            assert heads == ({0} if pair else {0, 1})


def test_tagged_exchange_needs_one_norm_task_per_workgroup_per_layer():
    """Each workgroup keeps the residual stream in registers through every RMSNorm
    prologue. A row missing a QKV task, or holding two gate/up tasks, in a layer is
    rejected on the host before any launch."""
    from nanovllm.backends.megakernel.taskgraph import _check_tagged_preconditions
    for op in (native.OP_QKV, native.OP_GATEUP):
        segs = build_segments(1, 1, 256, 28, 1, q_head_tasks=True)
        row = segs[0].rows[5]
        i = next(k for k, t in enumerate(row) if t.op == op and t.layer == 3)
        del row[i]
        with pytest.raises(RuntimeError, match="exactly one QKV and one gate/up"):
            _check_tagged_preconditions(segs)
    segs = build_segments(1, 1, 256, 28, 1, q_head_tasks=True)
    row = segs[0].rows[7]
    row.append(next(t for t in row if t.op == native.OP_GATEUP))
    with pytest.raises(RuntimeError, match="exactly one QKV and one gate/up"):
        _check_tagged_preconditions(segs)


def test_gate_up_publishes_residual_only_at_segment_ends():
    """Tagged schedule: the gate/up tasks of the last layer of each segment but
    the step's last carry the publish flag; no other task does."""
    for groups in (1, 4, 28):
        segs = build_segments(2, 1, 256, 28, groups, q_head_tasks=True)
        ends = {seg.stages[-2].layer if seg.stages[-1].op == native.OP_LMHEAD else seg.stages[-1].layer for seg in segs}
        for seg in segs:
            for row in seg.rows:
                for t in row:
                    flagged = t.op == native.OP_GATEUP and bool(t.a2 & native.GATEUP_PUBLISH_RES)
                    assert flagged == (t.op == native.OP_GATEUP and t.layer in ends and t.layer < 27)
    # the counter-protocol schedule is unchanged
    for seg in build_segments(2, 1, 256, 28, 4):
        assert all(t.a2 == 0 for row in seg.rows for t in row if t.op == native.OP_GATEUP)


def test_query_head_attention_tasks():
    """The tagged schedule has two ATTN tasks per (row, KV head, split): query
    heads 2h and 2h + 1, flagged in a0 and placed on the KV head's die."""
    from nanovllm.backends.megakernel.schedule import task_kv_head
    for batch, splits in ((1, 1), (8, 4)):
        seg = build_segments(batch, splits, 256, 28, 1, q_head_tasks=True)[0]
        per_layer = {}
        for w, row in enumerate(seg.rows):
            for t in row:
                if t.op == native.OP_ATTN:
                    assert t.a0 & native.ATTN_ONE_HEAD
                    assert task_kv_head(t) % 8 == w % 8
                    key = (t.layer, t.a0 & (native.ATTN_QHEAD - 1), t.a1)
                    per_layer.setdefault(key, []).append(bool(t.a0 & native.ATTN_QHEAD))
        assert len(per_layer) == 28 * batch * 8 * splits
        assert all(sorted(v) == [False, True] for v in per_layer.values())


def test_xcd_aware_placement_keeps_heads_on_their_die():
    """QKV and attention tasks of KV head h sit on workgroups w with w % 8 == h % 8;
    every workgroup still gets one LM task and the schedule still verifies."""
    from nanovllm.backends.megakernel.schedule import task_kv_head
    for batch, splits in ((1, 1), (8, 4)):
        s = build_schedule(batch, splits, 256, 28)
        assert verify(s) == []
        for w, row in enumerate(s.rows):
            for t in row:
                if t.op in (native.OP_QKV, native.OP_ATTN):
                    assert task_kv_head(t) % 8 == w % 8
            assert sum(t.op == native.OP_LMHEAD for t in row) == 1


def test_stage_schedules_one_task_per_workgroup_with_published_residuals():
    """The per-op comparator on the tagged kernel: one launch per stage, one task
    per workgroup, every QKV and gate/up task publishing its residual, stages in
    the persistent schedule's order, and no stage larger than the grid."""
    from nanovllm.backends.megakernel import native
    from nanovllm.backends.megakernel.schedule import build_stage_schedules, build_stages

    for batch, splits in ((1, 1), (1, 16), (8, 2), (4, 4)):
        scheds = build_stage_schedules(batch, splits, num_layers=3, max_grid=256)
        ref = build_stages(batch, splits, 256, 3, q_head_tasks=True)
        assert [(s.stages[0].op, s.stages[0].layer) for s in scheds] == [(s.op, s.layer) for s in ref]
        for s, r in zip(scheds, ref):
            assert s.grid == len(r.tasks) <= 256 and all(len(row) == 1 for row in s.rows)
            for t, u in zip((row[0] for row in s.rows), r.tasks):
                if t.op == native.OP_QKV:
                    assert t.a2 & native.QKV_PUBLISH_RES
                elif t.op == native.OP_GATEUP:
                    assert t.a2 & native.GATEUP_PUBLISH_RES
                else:
                    assert t == u
        assert scheds[-1].stages[0].op == native.OP_LMHEAD and scheds[-1].grid == 256
    import pytest

    with pytest.raises(ValueError, match="co-resident"):
        build_stage_schedules(8, 4, num_layers=1, max_grid=256)   # 8 x 16 x 4 = 512 attention tasks


def test_tagged_split_rule():
    """The tagged kernel's measured split rule: at batch 1 one split up to ctx 192,
    eight up to 1700, then 16; 64 positions per split at batch 2, 256 at batch 4-8,
    capped at 16 // batch."""
    from nanovllm.backends.megakernel.schedule import tagged_attn_splits as t

    assert [t(c) for c in (1, 129, 192, 193, 480, 1000, 1700, 1701, 2048)] == [1, 1, 1, 8, 8, 8, 8, 16, 16]
    assert [t(c, batch=2) for c in (64, 65, 480, 1000, 2048)] == [1, 2, 8, 8, 8]
    # one-head tasks at batch 4-8: 192 positions per split, capped at 16 // batch
    assert [t(c, batch=8) for c in (192, 193, 2048)] == [1, 2, 2] and t(2048, batch=4) == 4
    assert [t(c, batch=4) for c in (192, 193, 400)] == [1, 2, 4]
    assert t(100, minimum=4) == 4 and t(2048, minimum=16, batch=8) == 16


def test_pair_head_rule_and_its_split_rule():
    """Tasks of both query heads from batch 4 at contexts of two pages or more
    (batch 8: from ctx 193); they take 32 // batch splits (at most 16)."""
    from nanovllm.backends.megakernel.schedule import tagged_attn_splits as t, tagged_pair_heads as p

    assert [p(b, 2000) for b in (1, 2, 4, 8)] == [False, False, True, True]
    assert [p(8, c) for c in (1, 192, 193, 2048)] == [False, False, True, True]
    assert [p(4, c) for c in (1, 256, 257, 2048)] == [False, False, True, True]
    assert [t(c, batch=8, pair_heads=True) for c in (300, 700, 1100, 2048)] == [4, 4, 4, 4]
    assert [t(c, batch=4, pair_heads=True) for c in (300, 1100, 2048)] == [8, 8, 8]
    assert t(2048, batch=1, pair_heads=True) == 16 and t(300, batch=2, pair_heads=True) == 16
    assert t(100, minimum=8, batch=8, pair_heads=True) == 8
    # a stage of pair tasks at the cap fills the 256 workgroups exactly once
    for b in (4, 8):
        splits = t(10 ** 5, batch=b, pair_heads=True)
        assert b * 8 * splits == 256
