"""Page pool of the paged KV cache, with prefix reuse of full pages.

Pages are reference-counted. A page whose tokens are complete gets a content
key (an xxh3 digest chained over the parent page's key and the page's token
ids), so a later prompt with the same prefix maps those pages instead of
recomputing them; a page freed by its last owner keeps its key until the pool
hands it out again, so a finished request's prefix stays reusable for a while.
Free pages are handed out oldest-freed first.

Behaviour the rest of the engine relies on (reference
``engine/block_manager.py:26-143``): a prompt occupies ``ceil(len / page)``
pages; a decode step needs a new page exactly when the sequence length becomes
``1 (mod page)``; releasing a sequence frees the pages no other sequence holds.
The public name ``BlockManager`` and its ``stats()`` keys are kept for callers.
"""

from __future__ import annotations

from collections import deque

import numpy as np
import xxhash

from nanovllm.engine.sequence import Sequence

NO_KEY = -1


def page_key(token_ids: list[int], parent: int = NO_KEY) -> int:
    """Content key of a full page: xxh3-64 of the parent key and the token ids."""

    h = xxhash.xxh3_64()
    h.update((parent & 0xFFFFFFFFFFFFFFFF).to_bytes(8, "little"))
    h.update(np.asarray(token_ids, dtype=np.int32).tobytes())
    return h.intdigest()


class BlockManager:
    def __init__(self, num_blocks: int, block_size: int):
        if num_blocks < 1:
            raise ValueError(f"num_blocks must be >= 1; got {num_blocks}")
        self.block_size = block_size
        self.num_blocks = num_blocks
        self._refs = [0] * num_blocks                 # owners per page
        self._key = [NO_KEY] * num_blocks             # content key per page (NO_KEY: none)
        self._tokens: list[list[int] | None] = [None] * num_blocks
        self._by_key: dict[int, int] = {}             # content key -> page
        self._free: deque[int] = deque(range(num_blocks))
        self._counts = {"prefix_cache_hits": 0, "prefix_cache_misses": 0, "freed_blocks": 0,
                        "peak_used_blocks": 0}

    # -- pool primitives ---------------------------------------------------------
    @property
    def num_used(self) -> int:
        return self.num_blocks - len(self._free)

    def _hand_out(self) -> int:
        page = self._free.popleft()
        if self._refs[page]:
            raise RuntimeError(f"page {page} on the free list still has owners")
        self._forget(page)
        self._refs[page] = 1
        self._counts["peak_used_blocks"] = max(self._counts["peak_used_blocks"], self.num_used)
        return page

    def _forget(self, page: int) -> None:
        key = self._key[page]
        if key != NO_KEY and self._by_key.get(key) == page:
            del self._by_key[key]
        self._key[page] = NO_KEY
        self._tokens[page] = None

    def _drop(self, page: int) -> None:
        self._refs[page] -= 1
        if self._refs[page] == 0:
            self._free.append(page)
            self._counts["freed_blocks"] += 1

    def _lookup(self, key: int, tokens: list[int]) -> int:
        page = self._by_key.get(key, -1)
        return page if page >= 0 and self._tokens[page] == tokens else -1

    def _reusable_prefix(self, seq: Sequence) -> list[int]:
        """Pages holding the sequence's leading full pages, as far as they match.
        The last page is never reused (its token is recomputed to get logits)."""

        pages, key = [], NO_KEY
        for i in range(seq.num_blocks - 1):
            tokens = seq.block(i)
            key = page_key(tokens, key)
            page = self._lookup(key, tokens)
            if page < 0:
                break
            pages.append(page)
        return pages

    # -- what the scheduler calls --------------------------------------------------
    def can_allocate(self, seq: Sequence) -> int:
        """Leading pages reusable for ``seq``, or -1 when the free list cannot
        supply the rest."""

        reuse = self._reusable_prefix(seq)
        fresh = seq.num_blocks - sum(1 for p in reuse if self._refs[p] > 0)
        return len(reuse) if len(self._free) >= fresh else -1

    def allocate(self, seq: Sequence, num_cached_blocks: int) -> None:
        """Give ``seq`` its pages: the first ``num_cached_blocks`` from the prefix
        index (as :meth:`can_allocate` found them), the rest from the free list."""

        if seq.block_table:
            raise RuntimeError("sequence already owns blocks")
        reuse = self._reusable_prefix(seq)[:num_cached_blocks]
        if len(reuse) != num_cached_blocks:
            raise RuntimeError("prefix pages changed between can_allocate and allocate")
        for page in reuse:
            if self._refs[page] == 0:
                self._free.remove(page)       # revived from the free list
            self._refs[page] += 1
        self._counts["peak_used_blocks"] = max(self._counts["peak_used_blocks"], self.num_used)
        seq.block_table.extend(reuse)
        seq.block_table.extend(self._hand_out() for _ in range(seq.num_blocks - len(reuse)))
        seq.num_cached_tokens = len(reuse) * self.block_size
        self._counts["prefix_cache_hits"] += len(reuse)
        self._counts["prefix_cache_misses"] += seq.num_blocks - len(reuse)

    def deallocate(self, seq: Sequence) -> None:
        for page in reversed(seq.block_table):
            self._drop(page)
        seq.block_table.clear()
        seq.num_cached_tokens = 0

    def can_append(self, seq: Sequence) -> bool:
        """Whether the pool can cover the page the next decode step may need."""
        return not self._needs_page(seq) or bool(self._free)

    def may_append(self, seq: Sequence) -> None:
        if self._needs_page(seq):
            seq.block_table.append(self._hand_out())

    def _needs_page(self, seq: Sequence) -> bool:
        return len(seq) % self.block_size == 1

    def hash_blocks(self, seq: Sequence) -> None:
        """Key the pages this step completes (after its tokens are cached)."""

        done_before = seq.num_cached_tokens // self.block_size
        done_after = (seq.num_cached_tokens + seq.num_scheduled_tokens) // self.block_size
        key = self._key[seq.block_table[done_before - 1]] if done_before else NO_KEY
        for i in range(done_before, done_after):
            page, tokens = seq.block_table[i], seq.block(i)
            key = page_key(tokens, key)
            self._key[page], self._tokens[page] = key, tokens
            self._by_key[key] = page

    def stats(self) -> dict[str, int]:
        return {"block_size": self.block_size, "allocated_blocks": self.num_used,
                "free_blocks": len(self._free), **self._counts}
