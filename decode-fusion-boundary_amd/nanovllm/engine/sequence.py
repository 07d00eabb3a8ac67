"""A request as the engine tracks it: its tokens, where they sit in the paged
KV cache, and how far prefill has got.

Attribute and method names are the nano-vLLM engine's (the scheduler, the
model runner, the megakernel backend and the KV helpers read them; reference
``engine/sequence.py``). The counters are derived from the token list rather
than kept beside it, so they cannot drift apart.
"""

from __future__ import annotations

import itertools
from enum import Enum

from nanovllm.sampling_params import GREEDY_TEMPERATURE, SamplingParams

_ids = itertools.count()


class SequenceStatus(Enum):
    WAITING = "waiting"      # queued for (more) prefill, or preempted
    RUNNING = "running"      # prompt fully cached, decoding
    FINISHED = "finished"    # hit max_tokens or EOS; pages released


class Sequence:
    """Token state of one request. ``block_size`` is the engine's page size
    (set once by the engine from its config)."""

    block_size = 256

    def __init__(self, token_ids: list[int], sampling_params: SamplingParams | None = None):
        if len(token_ids) == 0:
            raise ValueError("a sequence needs at least one token")
        params = sampling_params if sampling_params is not None else SamplingParams()
        self.seq_id = next(_ids)
        self.status = SequenceStatus.WAITING
        self.token_ids: list[int] = list(token_ids)
        self.num_prompt_tokens = len(self.token_ids)
        # tokens whose K/V are in the cache, and tokens the current step computes
        self.num_cached_tokens = 0
        self.num_scheduled_tokens = 0
        self.is_prefill = True
        self.block_table: list[int] = []
        self.temperature = params.temperature
        self.max_tokens = params.max_tokens
        self.ignore_eos = params.ignore_eos

    # -- tokens ---------------------------------------------------------------
    def __len__(self) -> int:
        return len(self.token_ids)

    def __getitem__(self, key):
        return self.token_ids[key]

    @property
    def num_tokens(self) -> int:
        return len(self.token_ids)

    @property
    def last_token(self) -> int:
        return self.token_ids[-1]

    @property
    def prompt_token_ids(self) -> list[int]:
        return self.token_ids[:self.num_prompt_tokens]

    @property
    def completion_token_ids(self) -> list[int]:
        return self.token_ids[self.num_prompt_tokens:]

    @property
    def num_completion_tokens(self) -> int:
        return len(self.token_ids) - self.num_prompt_tokens

    def append_token(self, token_id: int) -> None:
        self.token_ids.append(int(token_id))

    # -- sampling / status --------------------------------------------------------
    @property
    def is_greedy(self) -> bool:
        return self.temperature <= GREEDY_TEMPERATURE

    @property
    def is_finished(self) -> bool:
        return self.status is SequenceStatus.FINISHED

    # -- pages ------------------------------------------------------------------
    @property
    def num_blocks(self) -> int:
        """Pages the current tokens occupy."""
        return -(-len(self.token_ids) // self.block_size)

    @property
    def last_block_num_tokens(self) -> int:
        """Tokens in the last occupied page (1 .. block_size)."""
        return len(self.token_ids) - (self.num_blocks - 1) * self.block_size

    def block(self, i: int) -> list[int]:
        """Token ids of page ``i``."""
        if i < 0 or i >= self.num_blocks:
            raise IndexError(f"block {i} outside [0, {self.num_blocks})")
        start = i * self.block_size
        return self.token_ids[start:start + self.block_size]
