"""Paged KV-cache shape/stride contract (reference ``backends/megakernel/cache.py:16-119``).

K and V are separate views ``[layers, blocks, block_size, kv_heads, head_dim]``
of the engine-owned ``[2, layers, ...]`` cache; offsets are in elements. The
HIP kernels compute the same offset (``csrc/mkd_tasks.h``, ``task_attn``):
``layer * layer_stride + (block_table[p // bs] * bs + p % bs) * token_stride
+ head * head_dim + d``.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Sequence


@dataclass(frozen=True)
class PagedKVCacheSpec:
    num_layers: int
    num_blocks: int
    block_size: int
    num_kv_heads: int
    head_dim: int
    dtype_itemsize: int

    def __post_init__(self) -> None:
        for name in ("num_layers", "num_blocks", "num_kv_heads", "head_dim", "dtype_itemsize"):
            if getattr(self, name) <= 0:
                raise ValueError(f"{name} must be positive")
        if self.block_size <= 0:
            raise ValueError("block_size must be positive")

    @property
    def shape(self) -> tuple[int, ...]:
        return (2, self.num_layers, self.num_blocks, self.block_size, self.num_kv_heads, self.head_dim)

    @property
    def head_stride(self) -> int:
        return self.head_dim

    @property
    def token_stride(self) -> int:
        return self.num_kv_heads * self.head_dim

    @property
    def block_stride(self) -> int:
        return self.block_size * self.token_stride

    @property
    def layer_stride(self) -> int:
        return self.num_blocks * self.block_stride

    @property
    def total_elements(self) -> int:
        return self.num_layers * self.layer_stride

    @property
    def total_bytes(self) -> int:
        return 2 * self.total_elements * self.dtype_itemsize

    def physical_slot(self, block_table: Sequence[int], logical_position: int) -> tuple[int, int]:
        if logical_position < 0:
            raise IndexError("position must be non-negative")
        if not block_table:
            raise ValueError("block table must not be empty")
        logical_block, offset = divmod(logical_position, self.block_size)
        if logical_block >= len(block_table):
            raise IndexError("position is outside the block table")
        block = int(block_table[logical_block])
        if not 0 <= block < self.num_blocks:
            raise ValueError("block table contains an invalid physical block")
        return block, offset

    def element_offset(self, layer: int, block_table: Sequence[int], logical_position: int,
                       kv_head: int, head_dim_index: int) -> int:
        if not 0 <= layer < self.num_layers:
            raise IndexError("layer is outside the cache")
        if not 0 <= kv_head < self.num_kv_heads:
            raise IndexError("kv_head is outside the cache")
        if not 0 <= head_dim_index < self.head_dim:
            raise IndexError("head dimension is outside the cache")
        block, offset = self.physical_slot(block_table, logical_position)
        return (layer * self.layer_stride + block * self.block_stride
                + offset * self.token_stride + kv_head * self.head_stride + head_dim_index)
