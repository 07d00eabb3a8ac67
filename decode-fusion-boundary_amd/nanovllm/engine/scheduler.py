"""Continuous-batching scheduler (reference ``src/nanovllm/engine/scheduler.py``).

Decode is preferred while prefill requests wait, for at most
``prefill_decode_ratio`` consecutive decode steps; prefill is budgeted by
``max_num_batched_tokens`` and ``max_prefill_tokens_per_step`` (chunked when a
single prompt is larger); KV pressure preempts the most recently scheduled
running sequence back to the waiting queue.
"""

from collections import deque

from nanovllm.config import Config
from nanovllm.engine.block_manager import BlockManager
from nanovllm.engine.sequence import Sequence, SequenceStatus


class Scheduler:
    def __init__(self, config: Config):
        self.max_num_seqs = config.max_num_seqs
        self.max_num_batched_tokens = config.max_num_batched_tokens
        self.max_prefill_tokens_per_step = (
            config.max_prefill_tokens_per_step or config.max_num_batched_tokens
        )
        self.prefill_decode_ratio = config.prefill_decode_ratio
        self._decode_steps_since_prefill = 0
        self.eos = config.eos
        self.block_size = config.kvcache_block_size
        self.block_manager = BlockManager(config.num_kvcache_blocks, config.kvcache_block_size)
        self.waiting: deque[Sequence] = deque()
        self.running: deque[Sequence] = deque()
        self._peak_waiting = 0
        self._peak_running = 0

    def _note_peaks(self) -> None:
        self._peak_waiting = max(self._peak_waiting, len(self.waiting))
        self._peak_running = max(self._peak_running, len(self.running))

    def is_finished(self) -> bool:
        return not self.waiting and not self.running

    def add(self, seq: Sequence) -> None:
        self.waiting.append(seq)
        self._note_peaks()

    def _decode_first(self) -> bool:
        return bool(self.running) and (
            not self.waiting
            or self._decode_steps_since_prefill < self.prefill_decode_ratio
        )

    def schedule(self) -> tuple[list[Sequence], bool]:
        self._note_peaks()
        if self._decode_first():
            seqs = self._schedule_decode()
            if seqs:
                self._decode_steps_since_prefill += 1
                self._note_peaks()
                return seqs, False
        seqs = self._schedule_prefill()
        if seqs:
            self._decode_steps_since_prefill = 0
            self._note_peaks()
            return seqs, True
        seqs = self._schedule_decode()
        if seqs:
            self._decode_steps_since_prefill += 1
            self._note_peaks()
            return seqs, False
        raise RuntimeError("scheduler made no progress")

    def _schedule_prefill(self) -> list[Sequence]:
        picked: list[Sequence] = []
        used = 0
        budget = self.max_prefill_tokens_per_step
        while self.waiting and len(picked) < self.max_num_seqs:
            seq = self.waiting[0]
            room = min(self.max_num_batched_tokens - used, budget - used)
            if room == 0:
                break
            if not seq.block_table:
                cached_blocks = self.block_manager.can_allocate(seq)
                if cached_blocks == -1:
                    break
                todo = seq.num_tokens - cached_blocks * self.block_size
            else:
                todo = seq.num_tokens - seq.num_cached_tokens
            if room < todo and picked:
                break
            if not seq.block_table:
                self.block_manager.allocate(seq, cached_blocks)
            seq.num_scheduled_tokens = min(todo, room)
            used += seq.num_scheduled_tokens
            if seq.num_cached_tokens + seq.num_scheduled_tokens == seq.num_tokens:
                seq.status = SequenceStatus.RUNNING
                self.waiting.popleft()
                self.running.append(seq)
            picked.append(seq)
        return picked

    def _schedule_decode(self) -> list[Sequence]:
        picked: list[Sequence] = []
        while self.running and len(picked) < self.max_num_seqs:
            seq = self.running.popleft()
            while not self.block_manager.can_append(seq):
                if self.running:
                    self.preempt(self.running.pop())
                else:
                    self.preempt(seq)
                    break
            else:
                seq.num_scheduled_tokens = 1
                seq.is_prefill = False
                self.block_manager.may_append(seq)
                picked.append(seq)
        self.running.extendleft(reversed(picked))
        return picked

    def preempt(self, seq: Sequence) -> None:
        seq.status = SequenceStatus.WAITING
        seq.is_prefill = True
        self.block_manager.deallocate(seq)
        self.waiting.appendleft(seq)

    def postprocess(self, seqs: list[Sequence], token_ids: list[int], is_prefill: bool) -> None:
        for seq, token_id in zip(seqs, token_ids):
            self.block_manager.hash_blocks(seq)
            seq.num_cached_tokens += seq.num_scheduled_tokens
            seq.num_scheduled_tokens = 0
            if is_prefill and seq.num_cached_tokens < seq.num_tokens:
                continue
            seq.append_token(token_id)
            hit_eos = not seq.ignore_eos and token_id == self.eos
            if hit_eos or seq.num_completion_tokens == seq.max_tokens:
                seq.status = SequenceStatus.FINISHED
                self.block_manager.deallocate(seq)
                self.running.remove(seq)

    def stats(self) -> dict[str, int]:
        return {
            "waiting_sequences": len(self.waiting),
            "running_sequences": len(self.running),
            "peak_waiting_sequences": self._peak_waiting,
            "peak_running_sequences": self._peak_running,
            "decode_steps_since_prefill": self._decode_steps_since_prefill,
            "prefill_decode_ratio": self.prefill_decode_ratio,
            **self.block_manager.stats(),
        }
