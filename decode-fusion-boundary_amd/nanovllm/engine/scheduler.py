"""Continuous-batching scheduler: which sequences run in the next model step.

Policy (the nano-vLLM engine's, reference ``engine/scheduler.py``):

* a step is either a prefill step or a decode step, never both;
* while sequences are decoding, decode steps are preferred, but after
  ``prefill_decode_ratio`` decode steps in a row a waiting prompt gets a
  prefill step (with nothing waiting, decode always runs);
* a prefill step takes waiting prompts in arrival order under a token budget
  of ``min(max_num_batched_tokens, max_prefill_tokens_per_step)``; the first
  prompt of a step may be chunked to fit, later ones must fit whole; pages come
  from the pool with prefix reuse, and a prompt whose pages do not fit waits;
* a decode step takes up to ``max_num_seqs`` running sequences in order; when
  the pool cannot give one its next page, the most recently admitted running
  sequence is preempted (pages freed, back to the head of the waiting queue),
  the sequence itself if it is the only one left.
"""

from __future__ import annotations

from collections import deque

from nanovllm.config import Config
from nanovllm.engine.block_manager import BlockManager
from nanovllm.engine.sequence import Sequence, SequenceStatus


class Scheduler:
    def __init__(self, config: Config):
        self.max_num_seqs = config.max_num_seqs
        self.max_num_batched_tokens = config.max_num_batched_tokens
        self.max_prefill_tokens_per_step = config.max_prefill_tokens_per_step or config.max_num_batched_tokens
        self.prefill_decode_ratio = config.prefill_decode_ratio
        self.eos = config.eos
        self.block_size = config.kvcache_block_size
        self.block_manager = BlockManager(config.num_kvcache_blocks, config.kvcache_block_size)
        self.waiting: deque[Sequence] = deque()
        self.running: deque[Sequence] = deque()
        self._decode_streak = 0          # decode steps since the last prefill step
        self._peaks = {"waiting": 0, "running": 0}

    # -- queue state ---------------------------------------------------------------
    def _track(self) -> None:
        self._peaks["waiting"] = max(self._peaks["waiting"], len(self.waiting))
        self._peaks["running"] = max(self._peaks["running"], len(self.running))

    def is_finished(self) -> bool:
        return not (self.waiting or self.running)

    def add(self, seq: Sequence) -> None:
        self.waiting.append(seq)
        self._track()

    # -- one step ------------------------------------------------------------------
    def schedule(self) -> tuple[list[Sequence], bool]:
        """Returns ``(sequences, is_prefill)`` of the next step."""

        self._track()
        prefer_decode = bool(self.running) and (not self.waiting
                                                or self._decode_streak < self.prefill_decode_ratio)
        order = ((False, self._decode_batch), (True, self._prefill_batch))
        for is_prefill, make in (order if prefer_decode else order[::-1]):
            batch = make()
            if batch:
                self._decode_streak = 0 if is_prefill else self._decode_streak + 1
                self._track()
                return batch, is_prefill
        raise RuntimeError("scheduler made no progress")

    def _prefill_batch(self) -> list[Sequence]:
        pool = self.block_manager
        budget = min(self.max_num_batched_tokens, self.max_prefill_tokens_per_step)
        batch: list[Sequence] = []
        used = 0
        while self.waiting and len(batch) < self.max_num_seqs and used < budget:
            seq = self.waiting[0]
            has_pages = bool(seq.block_table)
            reuse = 0
            if not has_pages:
                reuse = pool.can_allocate(seq)
                if reuse < 0:
                    break                                    # the pool cannot hold this prompt yet
            todo = seq.num_tokens - (seq.num_cached_tokens if has_pages else reuse * self.block_size)
            room = budget - used
            if batch and room < todo:
                break                                        # only a step's first prompt is chunked
            if not has_pages:
                pool.allocate(seq, reuse)
            seq.num_scheduled_tokens = min(todo, room)
            used += seq.num_scheduled_tokens
            batch.append(seq)
            if seq.num_cached_tokens + seq.num_scheduled_tokens == seq.num_tokens:
                self.waiting.popleft()                       # prompt complete after this step
                seq.status = SequenceStatus.RUNNING
                self.running.append(seq)
        return batch

    def _decode_batch(self) -> list[Sequence]:
        pool = self.block_manager
        batch: list[Sequence] = []
        while self.running and len(batch) < self.max_num_seqs:
            seq = self.running.popleft()
            while not pool.can_append(seq) and self.running:
                self.preempt(self.running.pop())             # newest admission gives its pages back
            if not pool.can_append(seq):
                self.preempt(seq)
                continue
            pool.may_append(seq)
            seq.num_scheduled_tokens = 1
            seq.is_prefill = False
            batch.append(seq)
        self.running.extendleft(reversed(batch))             # keep the running order
        return batch

    def preempt(self, seq: Sequence) -> None:
        self.block_manager.deallocate(seq)
        seq.status = SequenceStatus.WAITING
        seq.is_prefill = True
        self.waiting.appendleft(seq)

    # -- after the step --------------------------------------------------------------
    def postprocess(self, seqs: list[Sequence], token_ids: list[int], is_prefill: bool) -> None:
        pool = self.block_manager
        for seq, token in zip(seqs, token_ids):
            pool.hash_blocks(seq)
            seq.num_cached_tokens += seq.num_scheduled_tokens
            seq.num_scheduled_tokens = 0
            if is_prefill and seq.num_cached_tokens < seq.num_tokens:
                continue                                     # a chunk of a longer prompt: no token yet
            seq.append_token(token)
            if (token == self.eos and not seq.ignore_eos) or seq.num_completion_tokens == seq.max_tokens:
                seq.status = SequenceStatus.FINISHED
                pool.deallocate(seq)
                self.running.remove(seq)

    def stats(self) -> dict[str, int]:
        return {"waiting_sequences": len(self.waiting), "running_sequences": len(self.running),
                "peak_waiting_sequences": self._peaks["waiting"], "peak_running_sequences": self._peaks["running"],
                "decode_steps_since_prefill": self._decode_streak, "prefill_decode_ratio": self.prefill_decode_ratio,
                **self.block_manager.stats()}
