"""Paged KV-cache geometry: shape, strides and the element offset of a
(layer, position, kv head, dim) coordinate through a block table.

The engine owns one ``[2, layers, blocks, block_size, kv_heads, head_dim]``
tensor; K and V are its two halves. The offset identity is the one the
reference states in ``backends/megakernel/cache.py:94-119`` and its kernel in
``tg_kv_offset`` (``taskgraph_kernel.cu:484-493``); the HIP kernels here use the
same arithmetic (``csrc/mkd_pk4.h`` ``dma_issue_attn``, ``csrc/mkd_tasks.h``
``task_attn``):

    offset = layer * L + page * P + slot * T + head * D + d,
    page, slot = block_table[position // block_size], position % block_size,

with T = kv_heads * head_dim, P = block_size * T, L = blocks * P. The class
name, properties and error types are the reference's public contract.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Sequence

_DIMS = ("num_layers", "num_blocks", "block_size", "num_kv_heads", "head_dim", "dtype_itemsize")


@dataclass(frozen=True)
class PagedKVCacheSpec:
    num_layers: int
    num_blocks: int
    block_size: int
    num_kv_heads: int
    head_dim: int
    dtype_itemsize: int
    # element strides of (layer, page, slot, head), derived once
    _strides: tuple[int, int, int, int] = field(init=False, repr=False, compare=False)

    def __post_init__(self) -> None:
        bad = [name for name in _DIMS if int(getattr(self, name)) <= 0]
        if bad:
            raise ValueError(f"{', '.join(bad)} must be positive")
        head = self.head_dim
        slot = self.num_kv_heads * head
        page = self.block_size * slot
        object.__setattr__(self, "_strides", (self.num_blocks * page, page, slot, head))

    # -- geometry ---------------------------------------------------------------
    @property
    def shape(self) -> tuple[int, ...]:
        return (2, self.num_layers, self.num_blocks, self.block_size, self.num_kv_heads, self.head_dim)

    @property
    def layer_stride(self) -> int:
        return self._strides[0]

    @property
    def block_stride(self) -> int:
        return self._strides[1]

    @property
    def token_stride(self) -> int:
        return self._strides[2]

    @property
    def head_stride(self) -> int:
        return self._strides[3]

    @property
    def total_elements(self) -> int:
        """Elements of one of the two halves (K or V)."""
        return self.num_layers * self.layer_stride

    @property
    def total_bytes(self) -> int:
        return 2 * self.total_elements * self.dtype_itemsize

    # -- addressing ---------------------------------------------------------------
    def physical_slot(self, block_table: Sequence[int], logical_position: int) -> tuple[int, int]:
        """``(physical block, slot in block)`` of a position of a sequence."""

        if logical_position < 0:
            raise IndexError(f"position {logical_position} must be non-negative")
        if len(block_table) == 0:
            raise ValueError("block table must not be empty")
        page_index, slot = divmod(logical_position, self.block_size)
        if page_index >= len(block_table):
            raise IndexError(f"position {logical_position} is outside the block table "
                             f"({len(block_table)} blocks of {self.block_size})")
        page = int(block_table[page_index])
        if page < 0 or page >= self.num_blocks:
            raise ValueError(f"block table holds {page}, not a physical block of [0, {self.num_blocks})")
        return page, slot

    def element_offset(self, layer: int, block_table: Sequence[int], logical_position: int,
                       kv_head: int, head_dim_index: int) -> int:
        """Element offset into the K (or V) half."""

        for name, value, limit in (("layer", layer, self.num_layers), ("kv_head", kv_head, self.num_kv_heads),
                                   ("head dimension", head_dim_index, self.head_dim)):
            if not 0 <= value < limit:
                raise IndexError(f"{name} {value} is outside the cache (0..{limit - 1})")
        page, slot = self.physical_slot(block_table, logical_position)
        coords = (layer, page, slot, kv_head)
        return sum(c * s for c, s in zip(coords, self._strides)) + head_dim_index
