"""Paged-KV block allocator with xxhash prefix caching.

Behaviour follows the reference ``src/nanovllm/engine/block_manager.py:26-143``:
full blocks are content-hashed (chained xxh64 over the previous block's hash
and the block's token ids); a new prompt reuses cached full blocks whose
tokens match; a decode appends a block exactly when the sequence length
becomes ``1 (mod block_size)``.
"""

from collections import deque

import numpy as np
import xxhash

from nanovllm.engine.sequence import Sequence


class Block:
    __slots__ = ("block_id", "ref_count", "hash", "token_ids")

    def __init__(self, block_id: int):
        self.block_id = block_id
        self.ref_count = 0
        self.hash = -1
        self.token_ids: list[int] = []

    def update(self, h: int, token_ids: list[int]) -> None:
        self.hash = h
        self.token_ids = token_ids

    def reset(self) -> None:
        self.ref_count = 1
        self.hash = -1
        self.token_ids = []


class BlockManager:
    def __init__(self, num_blocks: int, block_size: int):
        if num_blocks < 1:
            raise ValueError(f"num_blocks must be >= 1; got {num_blocks}")
        self.block_size = block_size
        self.blocks = [Block(i) for i in range(num_blocks)]
        self.hash_to_block_id: dict[int, int] = {}
        self.free_block_ids: deque[int] = deque(range(num_blocks))
        self.used_block_ids: set[int] = set()
        self.prefix_cache_hits = 0
        self.prefix_cache_misses = 0
        self.freed_blocks = 0
        self.peak_used_blocks = 0

    @staticmethod
    def compute_hash(token_ids: list[int], prefix: int = -1) -> int:
        h = xxhash.xxh64()
        if prefix != -1:
            h.update(prefix.to_bytes(8, "little"))
        h.update(np.asarray(token_ids, dtype=np.int64).tobytes())
        return h.intdigest()

    def _take_block(self) -> int:
        block_id = self.free_block_ids.popleft()
        block = self.blocks[block_id]
        if block.ref_count != 0:
            raise RuntimeError(f"free block {block_id} still has references")
        if block.hash != -1 and self.hash_to_block_id.get(block.hash) == block_id:
            del self.hash_to_block_id[block.hash]
        block.reset()
        self.used_block_ids.add(block_id)
        self.peak_used_blocks = max(self.peak_used_blocks, len(self.used_block_ids))
        return block_id

    def _release_block(self, block_id: int) -> None:
        self.used_block_ids.remove(block_id)
        self.free_block_ids.append(block_id)
        self.freed_blocks += 1

    def _cached_prefix(self, seq: Sequence) -> tuple[int, int]:
        """(number of reusable full blocks, blocks that must come off the free list)."""

        h = -1
        cached = 0
        new_blocks = seq.num_blocks
        for i in range(seq.num_blocks - 1):
            tokens = seq.block(i)
            h = self.compute_hash(tokens, h)
            block_id = self.hash_to_block_id.get(h, -1)
            if block_id == -1 or self.blocks[block_id].token_ids != tokens:
                break
            cached += 1
            if block_id in self.used_block_ids:
                new_blocks -= 1
        return cached, new_blocks

    def can_allocate(self, seq: Sequence) -> int:
        """Number of prefix-cached blocks, or -1 when the pool is too small."""

        cached, new_blocks = self._cached_prefix(seq)
        return cached if len(self.free_block_ids) >= new_blocks else -1

    def allocate(self, seq: Sequence, num_cached_blocks: int) -> None:
        if seq.block_table:
            raise RuntimeError("sequence already owns blocks")
        self.prefix_cache_hits += num_cached_blocks
        self.prefix_cache_misses += max(0, seq.num_blocks - num_cached_blocks)
        h = -1
        for i in range(num_cached_blocks):
            h = self.compute_hash(seq.block(i), h)
            block_id = self.hash_to_block_id[h]
            block = self.blocks[block_id]
            if block_id in self.used_block_ids:
                block.ref_count += 1
            else:
                block.ref_count = 1
                self.free_block_ids.remove(block_id)
                self.used_block_ids.add(block_id)
            seq.block_table.append(block_id)
        for _ in range(num_cached_blocks, seq.num_blocks):
            seq.block_table.append(self._take_block())
        seq.num_cached_tokens = num_cached_blocks * self.block_size

    def deallocate(self, seq: Sequence) -> None:
        for block_id in reversed(seq.block_table):
            block = self.blocks[block_id]
            block.ref_count -= 1
            if block.ref_count == 0:
                self._release_block(block_id)
        seq.num_cached_tokens = 0
        seq.block_table.clear()

    def can_append(self, seq: Sequence) -> bool:
        needs_block = len(seq) % self.block_size == 1
        return len(self.free_block_ids) >= int(needs_block)

    def may_append(self, seq: Sequence) -> None:
        if len(seq) % self.block_size == 1:
            seq.block_table.append(self._take_block())

    def hash_blocks(self, seq: Sequence) -> None:
        first = seq.num_cached_tokens // self.block_size
        last = (seq.num_cached_tokens + seq.num_scheduled_tokens) // self.block_size
        if first == last:
            return
        h = self.blocks[seq.block_table[first - 1]].hash if first > 0 else -1
        for i in range(first, last):
            block = self.blocks[seq.block_table[i]]
            tokens = seq.block(i)
            h = self.compute_hash(tokens, h)
            block.update(h, tokens)
            self.hash_to_block_id[h] = block.block_id

    def stats(self) -> dict[str, int]:
        return {
            "block_size": self.block_size,
            "allocated_blocks": len(self.used_block_ids),
            "free_blocks": len(self.free_block_ids),
            "freed_blocks": self.freed_blocks,
            "peak_used_blocks": self.peak_used_blocks,
            "prefix_cache_hits": self.prefix_cache_hits,
            "prefix_cache_misses": self.prefix_cache_misses,
        }
