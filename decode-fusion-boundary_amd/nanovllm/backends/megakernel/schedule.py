"""Task-graph generator for one Qwen3 decode step (host side, pure Python).

Counterpart of the reference ``backends/megakernel/schedule.py``
(``build_schedule`` :1102-1165, wave builders :718-1001, ``place_round_robin``
:1040-1055, ``serialize_inst_buf`` :1063-1082), redesigned for the MI355X
kernels in ``csrc/mkd_tasks.h``:

* one task = one workgroup-sized unit; GEMV stages are split into row blocks
  so that a stage has about one task per compute unit (16 QKV rows, 4 O rows,
  12 gate/up channel pairs, 4 down rows, ~594 LM-head rows at 256 CUs);
* QKV row blocks never straddle a KV head's rows (q: 256 rows, k/v: 128 each
  per KV head), so attention of head ``h`` waits only on head ``h``'s blocks;
* dependencies are fan-in counters: a task waits until a counter reaches the
  number of producer tasks and arrives on one counter when done; the split-KV
  partials of one (row, head) are merged by their last arriving split, which
  alone arrives on the layer's attention counter;
* placement is round-robin with a cursor carried across stages; each
  workgroup's row is in global stage order, which makes the graph
  deadlock-free by construction (checked by :mod:`.verifier`).

Instruction words: ``[op, layer, a0, a1, a2, wait, wait_count, signal]``
(``include/mkd_abi.h``). Fan-in counter ids: ``layer * 12 + k`` with
k = 0..7 the QKV blocks of KV head k, 8 attention, 9 O-proj, 10 gate/up,
11 down.
"""

from __future__ import annotations

import dataclasses
from dataclasses import dataclass, field

from .native import (
    ATTN_ONE_HEAD, ATTN_QHEAD, GATEUP_PUBLISH_RES, QKV_PUBLISH_RES, INST_WORDS, MAX_BATCH, MAX_LM_SLOTS, MAX_SPLITS, OP_ATTN, OP_DOWN, OP_GATEUP,
    OP_LMHEAD, OP_OPROJ, OP_QKV,
)

HIDDEN = 1024
INTERMEDIATE = 3072
NUM_Q_HEADS = 16
NUM_KV_HEADS = 8
HEAD_DIM = 128
Q_SIZE = NUM_Q_HEADS * HEAD_DIM
KV_SIZE = NUM_KV_HEADS * HEAD_DIM
QKV_ROWS = Q_SIZE + 2 * KV_SIZE
VOCAB = 151936
NUM_LAYERS = 28
FANIN_PER_LAYER = NUM_KV_HEADS + 4
BATCH_BUCKETS = (1, 2, 4, 8)


def fanin_qkv(layer: int, kv_head: int) -> int:
    return layer * FANIN_PER_LAYER + kv_head


def fanin_attn(layer: int) -> int:
    return layer * FANIN_PER_LAYER + NUM_KV_HEADS


def fanin_oproj(layer: int) -> int:
    return layer * FANIN_PER_LAYER + NUM_KV_HEADS + 1


def fanin_gateup(layer: int) -> int:
    return layer * FANIN_PER_LAYER + NUM_KV_HEADS + 2


def fanin_down(layer: int) -> int:
    return layer * FANIN_PER_LAYER + NUM_KV_HEADS + 3


def batch_bucket(rows: int) -> int:
    for b in BATCH_BUCKETS:
        if rows <= b:
            return b
    raise ValueError(f"batch {rows} exceeds the compiled maximum {MAX_BATCH}")


PAIR_HEADS_MIN_BATCH = 4         # smallest batch bucket whose tagged kernel runs tasks of both query heads
PAIR_HEADS_MIN_CONTEXT = 257     # and the shortest step context at which they are used
PAIR_HEADS_MIN_CONTEXT_B8 = 193  # (batch 8: ctx 240 840 us with both heads, 4 splits; 861 one head, 2)
ONE_HEAD_POSITIONS_PER_SPLIT = 192  # batch 4-8, one-head tasks (ctx 240 at batch 4: 701 us with 2, 730 with 1)


def tagged_pair_heads(batch: int, max_context: int) -> bool:
    """Whether the tagged kernel's attention tasks cover both query heads of
    their KV head (each cached K/V chunk read once) rather than one (the chunk
    read by two tasks, each with half the dependent work).

    Measured on MI355X (device us per step, tagged kernel): batch 8, C5 contexts
    (~1100-1900): 1426 one-head (2 splits) -> 1224 both heads (4 splits); C4
    (ctx ~520): 1073 -> 1046; batch 4, C5: 932 -> 912; but at short contexts
    (ctx < 100) one-head tasks are faster (batch 8: 894 vs 911, batch 4: 694 vs
    706), and at batch 2, C5: 710 one-head vs 765 both heads."""

    b = int(batch)
    return b >= PAIR_HEADS_MIN_BATCH and int(max_context) >= (PAIR_HEADS_MIN_CONTEXT_B8 if b >= 8
                                                               else PAIR_HEADS_MIN_CONTEXT)


B1_ONE_SPLIT_MAX = 192       # batch 1: one split up to this context,
B1_EIGHT_SPLITS_MAX = 1700   # eight up to this one (one merge round of 7 partials), then 16


def tagged_attn_splits(max_context: int, minimum: int = 1, batch: int = 1, pair_heads: bool = False) -> int:
    """Split-KV factor of the tagged persistent kernel: a power of two, at most
    16 // batch, never below ``minimum``.

    Tasks of both query heads (batch 4-8, two pages and more) take 32 // batch
    splits: measured (1 / 2 / 4 / 8 splits) batch 4 at ctx 300: 772 / 764 / 727
    / 720, ctx 1000: 1078 / 903 / 789 / 737; batch 8 (1 / 2 / 4 / 8) at ctx 300:
    928 / 925 / 879 / 1035, ctx 450: 1019 / 965 / 894 / 1047, ctx 1000: 1236 /
    1056 / 963 / 1122.

    One-head tasks at batch 4-8 aim at 192 positions per split (rounded up to
    a power of two, capped at 16 // batch).

    Batch 1: one split up to ctx 192, eight up to 1700 (the last split folds
    the other seven's partials in one poll round of eight), then 16. Batch 2
    aims at 64 positions per split (rounded up), batch 4 and 8 at 256 (rounded
    up, as :func:`auto_attn_splits`). Measured on MI355X (device us per step,
    tagged kernel, splits forced; 1 / 2 / 4 / 8 / 16): batch 1 at ctx 150: 537 /
    555 / 544 / 545 / 574; ctx 300: 599 / 587 / 551 / 549 / 582; ctx 600: 744 /
    650 / 583 / 562 / 595; ctx 1500: 1129 / 841 / 680 / 578 / 603; ctx 1900:
    1288 / 924 / 736 / 630 / 611. Batch 2 at ctx 300-1500: 8 best (587 / 611 /
    632 / 666 at ctx 300 / 600 / 1000 / 1500)."""

    b = max(1, int(batch))
    cap = max(1, MAX_SPLITS // b)
    ctx = max(1, int(max_context))
    if pair_heads:
        # half the tasks per split: 32 // batch splits (at most 16), the fastest
        # at every context the both-head tasks run at (two pages and more)
        cap = max(1, min(MAX_SPLITS, 2 * MAX_SPLITS // b))
        return max(min(int(minimum), MAX_SPLITS), cap)
    if b == 1:
        splits = 1 if ctx <= B1_ONE_SPLIT_MAX else (8 if ctx <= B1_EIGHT_SPLITS_MAX else 16)
    elif b == 2:
        want = -(-ctx // 64)
        splits = 1
        while splits < want:
            splits *= 2
    else:
        want = -(-ctx // ONE_HEAD_POSITIONS_PER_SPLIT)
        splits = 1
        while splits < want:
            splits *= 2
    return max(min(int(minimum), MAX_SPLITS), min(splits, cap))


def auto_attn_splits(max_context: int, minimum: int = 1, batch: int = 1) -> int:
    """Split-KV factor: one split per 256 cached positions, a power of two, at most
    16 // batch (so batch x splits <= 16) and never below ``minimum``.

    The batch cap is measured (MI355X, tagged persistent kernel, C5 contexts): at
    batch 8 and ctx ~1600 a step takes 1401 us with 2 splits and 1619 us with 8; at
    batch 4 and ctx ~1300, 911 us with 4 and 972 us with 8. At batch 1-2 the
    per-256-positions rule is already the fastest. With 16 query-head tasks per row,
    more splits than that add merge work and poll rounds, not parallelism."""

    want = max(1, -(-int(max_context) // 256))
    cap = max(1, MAX_SPLITS // max(1, int(batch)))
    splits = 1
    while splits < want and splits < cap:
        splits *= 2
    return max(min(int(minimum), MAX_SPLITS), splits)


@dataclass(frozen=True)
class Task:
    op: int
    layer: int
    a0: int
    a1: int = 0
    a2: int = 0
    wait: int = -1
    wait_count: int = 0
    signal: int = -1

    def words(self) -> list[int]:
        return [self.op, self.layer, self.a0, self.a1, self.a2, self.wait,
                self.wait_count, self.signal]


@dataclass
class Stage:
    op: int
    layer: int
    tasks: list[Task] = field(default_factory=list)


@dataclass
class Schedule:
    batch: int
    attn_splits: int
    num_layers: int
    grid: int
    stages: list[Stage]
    rows: list[list[Task]]          # per workgroup, in execution order

    @property
    def num_tasks(self) -> int:
        return sum(len(s.tasks) for s in self.stages)

    @property
    def max_inst(self) -> int:
        return max(1, max(len(r) for r in self.rows))

    @property
    def lm_slots(self) -> int:
        return sum(len(s.tasks) for s in self.stages if s.op == OP_LMHEAD)

    def persistent_words(self) -> tuple[list[int], list[int]]:
        """``[grid][max_inst][8]`` flattened (NOP-padded) and ``num_inst[grid]``."""

        flat: list[int] = []
        pad = [0] * INST_WORDS
        for row in self.rows:
            for t in row:
                flat.extend(t.words())
            for _ in range(self.max_inst - len(row)):
                flat.extend(pad)
        return flat, [len(r) for r in self.rows]

    def stage_words(self) -> tuple[list[int], list[tuple[int, int, int, int]]]:
        """Instruction list in stage order and ``(op, layer, first, count)`` per stage."""

        flat: list[int] = []
        table = []
        first = 0
        for st in self.stages:
            for t in st.tasks:
                flat.extend(t.words())
            table.append((st.op, st.layer, first, len(st.tasks)))
            first += len(st.tasks)
        return flat, table


def split_range(start: int, length: int, pieces: int) -> list[tuple[int, int]]:
    """Split ``[start, start+length)`` into ``pieces`` near-equal (first, count) blocks."""

    pieces = max(1, min(pieces, length))
    base, extra = divmod(length, pieces)
    out = []
    cur = start
    for i in range(pieces):
        n = base + (1 if i < extra else 0)
        out.append((cur, n))
        cur += n
    return out


def split_pairs(start: int, length: int, pieces: int) -> list[tuple[int, int]]:
    """Like :func:`split_range` but every block starts on an even row and holds an
    even number of rows (``length`` and ``start`` even): the persistent kernel
    exchanges activations as words of two bf16 values, each word from one task."""

    return [(start + 2 * f, 2 * n) for f, n in split_range(0, length // 2, pieces)]


def _qkv_segments():
    """(first row, rows, kv head) of every per-head row segment of [Wq; Wk; Wv]."""

    segs = []
    for h in range(NUM_KV_HEADS):
        segs.append((2 * h * HEAD_DIM, 2 * HEAD_DIM, h))         # q heads 2h, 2h+1
    for h in range(NUM_KV_HEADS):
        segs.append((Q_SIZE + h * HEAD_DIM, HEAD_DIM, h))        # k head h
    for h in range(NUM_KV_HEADS):
        segs.append((Q_SIZE + KV_SIZE + h * HEAD_DIM, HEAD_DIM, h))  # v head h
    return segs


def build_stages(batch: int, attn_splits: int, num_wgs: int,
                 num_layers: int = NUM_LAYERS, q_head_tasks: bool = False,
                 pair_heads: bool = False) -> list[Stage]:
    """The step's stages in dependency order. ``q_head_tasks`` (the tagged
    kernel's schedule) makes one ATTN task per query head instead of per KV
    head: task word a0 = b * 8 + h + ATTN_ONE_HEAD (+ ATTN_QHEAD for head 2h + 1),
    unless ``pair_heads`` keeps one task per KV head (a0 = b * 8 + h)."""

    if batch not in BATCH_BUCKETS:
        raise ValueError(f"batch bucket must be one of {BATCH_BUCKETS}; got {batch}")
    if not 1 <= attn_splits <= MAX_SPLITS:
        raise ValueError(f"attn_splits must be 1..{MAX_SPLITS}; got {attn_splits}")
    if not 1 <= num_layers <= NUM_LAYERS:
        raise ValueError(f"num_layers must be 1..{NUM_LAYERS}; got {num_layers}")
    if num_wgs < 1:
        raise ValueError("num_wgs must be >= 1")
    stages: list[Stage] = []
    qkv_target = -(-QKV_ROWS // num_wgs)
    prev_down: tuple[int, int] | None = None   # (fanin id, producer count)
    for layer in range(num_layers):
        # QKV: per-head segments cut into blocks of ~qkv_target rows
        qkv = Stage(OP_QKV, layer)
        per_head = [0] * NUM_KV_HEADS
        for first, rows, h in _qkv_segments():
            for r0, n in split_pairs(first, rows, -(-rows // qkv_target)):
                wait, cnt = prev_down if prev_down else (-1, 0)
                qkv.tasks.append(Task(OP_QKV, layer, r0, n, 0, wait, cnt, fanin_qkv(layer, h)))
                per_head[h] += 1
        stages.append(qkv)
        attn = Stage(OP_ATTN, layer)
        heads = ([ATTN_ONE_HEAD, ATTN_ONE_HEAD | ATTN_QHEAD] if q_head_tasks and not pair_heads else [0])
        for b in range(batch):
            for h in range(NUM_KV_HEADS):
                for s in range(attn_splits):
                    for flags in heads:
                        attn.tasks.append(Task(OP_ATTN, layer, b * NUM_KV_HEADS + h + flags, s, attn_splits,
                                               fanin_qkv(layer, h), per_head[h], fanin_attn(layer)))
        stages.append(attn)
        oproj = Stage(OP_OPROJ, layer)
        for r0, n in split_pairs(0, HIDDEN, num_wgs):
            oproj.tasks.append(Task(OP_OPROJ, layer, r0, n, 0, fanin_attn(layer),
                                    batch * NUM_KV_HEADS * len(heads), fanin_oproj(layer)))
        stages.append(oproj)
        gu = Stage(OP_GATEUP, layer)
        for c0, n in split_pairs(0, INTERMEDIATE, num_wgs):
            gu.tasks.append(Task(OP_GATEUP, layer, c0, n, 0, fanin_oproj(layer),
                                 len(oproj.tasks), fanin_gateup(layer)))
        stages.append(gu)
        down = Stage(OP_DOWN, layer)
        for r0, n in split_pairs(0, HIDDEN, num_wgs):
            down.tasks.append(Task(OP_DOWN, layer, r0, n, 0, fanin_gateup(layer),
                                   len(gu.tasks), fanin_down(layer)))
        stages.append(down)
        prev_down = (fanin_down(layer), len(down.tasks))
    lm = Stage(OP_LMHEAD, num_layers)
    blocks = split_range(0, VOCAB, min(num_wgs, MAX_LM_SLOTS))
    for slot, (r0, n) in enumerate(blocks):
        lm.tasks.append(Task(OP_LMHEAD, num_layers, r0, n, slot, prev_down[0], prev_down[1], -1))
    stages.append(lm)
    return stages


def place_round_robin(stages: list[Stage], num_wgs: int) -> list[list[Task]]:
    rows: list[list[Task]] = [[] for _ in range(num_wgs)]
    cursor = 0
    for st in stages:
        for t in st.tasks:
            rows[cursor].append(t)
            cursor = (cursor + 1) % num_wgs
    return rows


XCDS = 8  # accelerator dies of an MI355X; workgroup w of a launch runs on die w % 8


def task_kv_head(t: Task) -> int:
    """KV head whose rows a QKV task computes, or whose attention an ATTN task runs."""

    if t.op == OP_ATTN:
        return t.a0 % NUM_KV_HEADS
    r = t.a0
    if r < Q_SIZE:
        return r // (2 * HEAD_DIM)
    if r < Q_SIZE + KV_SIZE:
        return (r - Q_SIZE) // HEAD_DIM
    return (r - Q_SIZE - KV_SIZE) // HEAD_DIM


def place_xcd_aware(stages: list[Stage], num_wgs: int) -> list[list[Task]]:
    """Round-robin placement, except that the QKV and attention tasks of KV head
    ``h`` go to the workgroups of die ``h % 8`` (w % 8 == h % 8): their exchange
    (and the split-KV merge) then stays in that die's L2. Rows stay in stage order.
    Falls back to plain round-robin when the grid is not a multiple of 8."""

    if num_wgs % XCDS:
        return place_round_robin(stages, num_wgs)
    rows: list[list[Task]] = [[] for _ in range(num_wgs)]
    per_die = num_wgs // XCDS
    cursor = 0
    head_cursor = [0] * NUM_KV_HEADS
    for st in stages:
        if st.op in (OP_QKV, OP_ATTN):
            for t in st.tasks:
                h = task_kv_head(t)
                rows[h % XCDS + XCDS * (head_cursor[h] % per_die)].append(t)
                head_cursor[h] += 1
        else:
            for t in st.tasks:
                rows[cursor].append(t)
                cursor = (cursor + 1) % num_wgs
    return rows


def build_schedule(batch: int, attn_splits: int, num_wgs: int,
                   num_layers: int = NUM_LAYERS) -> Schedule:
    stages = build_stages(batch, attn_splits, num_wgs, num_layers)
    rows = place_xcd_aware(stages, num_wgs)
    return Schedule(batch=batch, attn_splits=attn_splits, num_layers=num_layers,
                    grid=num_wgs, stages=stages, rows=rows)


def split_layers(num_layers: int, groups: int) -> list[tuple[int, int]]:
    """Contiguous layer segments ``[start, end)`` for ``groups`` launches
    (reference ``schedule.split_layers`` :1168-1195)."""

    if not 1 <= groups <= num_layers:
        raise ValueError(f"fusion_groups must be in [1, {num_layers}]; got {groups}")
    return [(r0, r0 + n) for r0, n in split_range(0, num_layers, groups)]


def build_segments(batch: int, attn_splits: int, num_wgs: int, num_layers: int = NUM_LAYERS,
                   groups: int = 1, q_head_tasks: bool = False, pair_heads: bool = False) -> list[Schedule]:
    """One persistent launch per layer segment. Segment ``k`` holds the stages of
    its layers (the last one also the LM head); its first QKV stage waits on the
    previous segment's down counter, which the earlier launch already completed,
    and the final LM-head task clears every fan-in counter of the step."""

    stages = build_stages(batch, attn_splits, num_wgs, num_layers, q_head_tasks, pair_heads)
    out = []
    for start, end in split_layers(num_layers, groups):
        seg = [s for s in stages if start <= s.layer < end or (end == num_layers and s.op == OP_LMHEAD)]
        if q_head_tasks and end < num_layers:
            # the tagged kernel keeps the residual stream in registers within a
            # launch; the segment's last gate/up tasks publish it for the next one
            seg = [Stage(s.op, s.layer, [dataclasses.replace(t, a2=t.a2 | GATEUP_PUBLISH_RES) for t in s.tasks])
                   if s.op == OP_GATEUP and s.layer == end - 1 else s for s in seg]
        out.append(Schedule(batch=batch, attn_splits=attn_splits, num_layers=num_layers,
                            grid=num_wgs, stages=seg, rows=place_xcd_aware(seg, num_wgs)))
    return out


def build_stage_schedules(batch: int, attn_splits: int, num_layers: int = NUM_LAYERS,
                          max_grid: int = 256, pair_heads: bool = False) -> list[Schedule]:
    """The per-op comparator on the tagged persistent kernel's own task bodies:
    one persistent launch per stage, one task per workgroup (``grid`` = the
    stage's task count). Every QKV task publishes the residual after the input
    add and every gate/up task the residual after the post-attention add, since
    each consumer runs in a later launch and cannot keep them in registers. A
    stage's workgroups must all be resident (the last split-KV task and the last
    LM slot wait on their stage siblings), so a stage holds at most ``max_grid``
    tasks."""

    out = []
    for st in build_stages(batch, attn_splits, max_grid, num_layers, q_head_tasks=True, pair_heads=pair_heads):
        flag = QKV_PUBLISH_RES if st.op == OP_QKV else (GATEUP_PUBLISH_RES if st.op == OP_GATEUP else 0)
        tasks = [dataclasses.replace(t, a2=t.a2 | flag) for t in st.tasks] if flag else list(st.tasks)
        if len(tasks) > max_grid:
            raise ValueError(f"stage {st.op} of layer {st.layer} has {len(tasks)} tasks; one launch holds "
                             f"at most {max_grid} co-resident workgroups (reduce the split-KV factor)")
        out.append(Schedule(batch=batch, attn_splits=attn_splits, num_layers=num_layers, grid=len(tasks),
                            stages=[Stage(st.op, st.layer, tasks)], rows=[[t] for t in tasks]))
    return out
