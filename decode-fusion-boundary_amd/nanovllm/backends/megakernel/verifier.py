"""CPU verifier of a task-graph schedule: deadlock freedom, exact arrivals,
single ownership. Counterpart of the reference ``verifier.py`` (maximal
execution simulator :273-313, arrivals audit :445-470) and ``audit.py``
(ownership :46-203), restated for this build's instruction format.

Checks (each returns a list of human-readable violations):

* ``simulate``: every workgroup walks its row in order; a task may run only
  when its wait counter has reached ``wait_count``; attention tasks of one
  (row, head) arrive on their ticket and only the last one signals. The
  schedule passes when every task runs (no deadlock) and no wait target
  exceeds the arrivals its counter can ever get.
* ``arrivals``: for every fan-in counter, the arrivals the producers make
  equal the count every consumer waits for.
* ``ownership``: every output row/channel/vocab entry of every stage is
  written by exactly one task, every (row, head, split) attention task exists
  once, and LM-head argmax slots are 0..n-1 without repeats.
"""

from __future__ import annotations

from collections import defaultdict

from .native import OP_ATTN, OP_DOWN, OP_GATEUP, OP_LMHEAD, OP_OPROJ, OP_QKV
from .schedule import HIDDEN, INTERMEDIATE, NUM_KV_HEADS, QKV_ROWS, VOCAB, Schedule


def arrivals(sched: Schedule) -> list[str]:
    produced: dict[int, int] = defaultdict(int)
    attn_groups: dict[tuple[int, int], set] = defaultdict(set)
    for st in sched.stages:
        for t in st.tasks:
            if t.op == OP_ATTN:
                attn_groups[(t.layer, t.a0)].add(t.signal)
            elif t.signal >= 0:
                produced[t.signal] += 1
    for (_, _), sigs in attn_groups.items():
        for s in sigs:
            produced[s] += 1  # one arrival per (row, head): the last split
    errors = []
    waits: dict[int, set] = defaultdict(set)
    for st in sched.stages:
        for t in st.tasks:
            if t.wait >= 0:
                waits[t.wait].add(t.wait_count)
    for counter, counts in waits.items():
        if len(counts) != 1:
            errors.append(f"counter {counter} waited on with different counts {sorted(counts)}")
        for c in counts:
            if produced.get(counter, 0) != c:
                errors.append(f"counter {counter}: waits for {c}, producers arrive {produced.get(counter, 0)}")
    return errors


def simulate(sched: Schedule) -> list[str]:
    counters: dict[int, int] = defaultdict(int)
    tickets: dict[tuple[int, int], int] = defaultdict(int)
    pc = [0] * len(sched.rows)
    done = 0
    total = sum(len(r) for r in sched.rows)
    progress = True
    while progress:
        progress = False
        for wg, row in enumerate(sched.rows):
            while pc[wg] < len(row):
                t = row[pc[wg]]
                if t.wait >= 0 and counters[t.wait] < t.wait_count:
                    break
                if t.op == OP_ATTN:
                    key = (t.layer, t.a0)
                    tickets[key] += 1
                    if tickets[key] == t.a2 and t.signal >= 0:
                        counters[t.signal] += 1
                elif t.signal >= 0:
                    counters[t.signal] += 1
                pc[wg] += 1
                done += 1
                progress = True
    if done == total:
        return []
    stuck = [(wg, row[pc[wg]]) for wg, row in enumerate(sched.rows) if pc[wg] < len(row)]
    wg, t = stuck[0]
    return [f"deadlock: {total - done} tasks never run; e.g. workgroup {wg} waits on counter "
            f"{t.wait} for {t.wait_count} (has {counters[t.wait]})"]


def ownership(sched: Schedule) -> list[str]:
    errors = []
    by_layer: dict[tuple[int, int], list] = defaultdict(list)
    for st in sched.stages:
        by_layer[(st.op, st.layer)].extend(st.tasks)
    expect = {OP_QKV: QKV_ROWS, OP_OPROJ: HIDDEN, OP_GATEUP: INTERMEDIATE, OP_DOWN: HIDDEN,
              OP_LMHEAD: VOCAB}
    for (op, layer), tasks in by_layer.items():
        if op in expect:
            cover = [0] * expect[op]
            for t in tasks:
                if t.a1 < 1 or t.a0 < 0 or t.a0 + t.a1 > expect[op]:
                    errors.append(f"op {op} layer {layer}: range [{t.a0}, {t.a0 + t.a1}) out of bounds")
                    continue
                for r in range(t.a0, t.a0 + t.a1):
                    cover[r] += 1
            bad = [r for r, c in enumerate(cover) if c != 1]
            if bad:
                errors.append(f"op {op} layer {layer}: {len(bad)} outputs not written exactly once "
                              f"(first {bad[0]})")
        if op == OP_ATTN:
            seen = defaultdict(int)
            for t in tasks:
                seen[(t.a0, t.a1)] += 1
                if t.a2 != sched.attn_splits or not 0 <= t.a1 < t.a2:
                    errors.append(f"attn layer {layer}: bad split {t.a1}/{t.a2}")
            want = {(b * NUM_KV_HEADS + h, s) for b in range(sched.batch)
                    for h in range(NUM_KV_HEADS) for s in range(sched.attn_splits)}
            if set(seen) != want or any(v != 1 for v in seen.values()):
                errors.append(f"attn layer {layer}: (row, head, split) tasks are not exactly once")
        if op == OP_LMHEAD:
            slots = sorted(t.a2 for t in tasks)
            if slots != list(range(len(tasks))):
                errors.append("lm-head argmax slots are not 0..n-1")
    if sched.stages[-1].op != OP_LMHEAD:
        errors.append("the LM-head stage must be last")
    return errors


def verify(sched: Schedule) -> list[str]:
    return ownership(sched) + arrivals(sched) + simulate(sched)
