"""Position, cache-length and slot contract shared by every decode consumer.

Same identities as the reference ``src/nanovllm/engine/kv_layout.py:1-197``:

* prefill of ``[cached, cached + scheduled)``: positions are that range, the
  visible KV length is its end;
* decode with ``num_tokens`` tokens (the sampled token already appended):
  ``position = num_tokens - 1``; the step writes K/V at ``position`` and then
  attends over ``position + 1`` entries (``decode_cache_len``); the HIP step
  descriptor carries the *pre-decode* length ``position``
  (``decode_cache_seqlens``), the torch path carries ``num_tokens``;
* a slot is ``block_table[p // block_size] * block_size + p % block_size``;
* block tables are right-padded with physical block 0, never -1, because the
  HIP kernels index ``block_table[p // block_size]`` directly.

Torch-free so the CPU suite can pin it.
"""

from __future__ import annotations

from typing import Iterable, Sequence


def _check_nonneg(name: str, value: int) -> None:
    if value < 0:
        raise ValueError(f"{name} must be non-negative")


def prefill_positions(num_cached_tokens: int, num_scheduled_tokens: int) -> range:
    _check_nonneg("num_cached_tokens", num_cached_tokens)
    _check_nonneg("num_scheduled_tokens", num_scheduled_tokens)
    return range(num_cached_tokens, num_cached_tokens + num_scheduled_tokens)


def prefill_cache_len(num_cached_tokens: int, num_scheduled_tokens: int) -> int:
    _check_nonneg("num_cached_tokens", num_cached_tokens)
    _check_nonneg("num_scheduled_tokens", num_scheduled_tokens)
    return num_cached_tokens + num_scheduled_tokens


def slot_of(block_table: Sequence[int], position: int, block_size: int) -> int:
    """Flat slot of one logical position (``block * block_size + offset``)."""

    block, offset = divmod(position, block_size)
    return int(block_table[block]) * block_size + offset


def prefill_slot_mapping(
    block_table: Sequence[int], start: int, end: int, block_size: int
) -> list[int]:
    if block_size <= 0:
        raise ValueError("block_size must be positive")
    if start < 0 or end < start:
        raise ValueError(f"invalid prefill range [{start}, {end})")
    if start == end:
        return []
    if not block_table:
        raise RuntimeError(
            "prefill slot mapping requires an allocated block table; the "
            "scheduler must call BlockManager.allocate() before the model runs"
        )
    blocks_needed = -(-end // block_size)
    if len(block_table) < blocks_needed:
        raise RuntimeError(
            f"prefill tokens [{start}, {end}) need {blocks_needed} blocks but the "
            f"sequence only owns {len(block_table)}"
        )
    return [slot_of(block_table, p, block_size) for p in range(start, end)]


def decode_position(num_tokens: int) -> int:
    if num_tokens < 1:
        raise ValueError(f"num_tokens must be at least 1; got {num_tokens}")
    return num_tokens - 1


def decode_cache_seqlens(num_tokens: int) -> int:
    """Pre-decode KV length, the value the HIP step descriptor carries."""

    return decode_position(num_tokens)


def decode_cache_len(num_tokens: int) -> int:
    if num_tokens < 1:
        raise ValueError(f"num_tokens must be at least 1; got {num_tokens}")
    return num_tokens


def decode_slot_mapping(block_table: Sequence[int], num_tokens: int, block_size: int) -> int:
    if block_size <= 0:
        raise ValueError("block_size must be positive")
    position = decode_position(num_tokens)
    blocks_needed = -(-num_tokens // block_size)
    if len(block_table) != blocks_needed:
        raise RuntimeError(
            f"decode of {num_tokens} tokens needs {blocks_needed} blocks but the "
            f"block table has {len(block_table)}; BlockManager.may_append() "
            "must run before the model call"
        )
    return slot_of(block_table, position, block_size)


def pad_block_table(block_table: Iterable[int], max_pages: int) -> list[int]:
    table = list(block_table)
    if len(table) > max_pages:
        raise ValueError(f"block table has {len(table)} pages but the stride is {max_pages}")
    return table + [0] * (max_pages - len(table))
