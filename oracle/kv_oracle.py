"""Integer KV-cache contract restated on the CPU -- TEST INFRASTRUCTURE ONLY.

Restates, as the checker for the HIP kernels' paged addressing:

* ``backends/megakernel/cache.py:94-119`` (``element_offset``) and
  ``taskgraph_kernel.cu:484-493`` (``tg_kv_offset``): the flat element offset
  ``layer*Ls + block_table[p//bs]*bs*T + (p%bs)*T + head*D + d`` with
  ``T = kv_heads*D`` and ``Ls = blocks*bs*T``;
* ``engine/kv_layout.py:154-197``: decode slot and right-padding with block 0.

Pinned by the numeric cases of the reference tests
(``tests/test_paged_kv.py:17-81``, ``tests/test_kv_block_boundary.py:78-300``,
``tests/test_kv_cache_indexing.py:84-190``), reproduced as vectors in
``tests/golden/kv_contract.json``.
"""

from __future__ import annotations


def element_offset(layer, block_table, position, kv_head, dim, *, num_blocks,
                   block_size, num_kv_heads, head_dim):
    token_stride = num_kv_heads * head_dim
    block_stride = block_size * token_stride
    layer_stride = num_blocks * block_stride
    block = block_table[position // block_size]
    return (layer * layer_stride + block * block_stride
            + (position % block_size) * token_stride + kv_head * head_dim + dim)


def decode_slot(block_table, num_tokens, block_size):
    position = num_tokens - 1
    return block_table[position // block_size] * block_size + position % block_size


def pad_table(table, width):
    return list(table) + [0] * (width - len(table))
