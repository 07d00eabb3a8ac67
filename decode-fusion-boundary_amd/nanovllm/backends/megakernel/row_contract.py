"""Per-row activation mask of a decode launch (reference ``row_contract.py:32-52``).

An inactive row skips only its paged-KV write: under continuous batching a
finished sequence's pages may already belong to a new sequence, so a stale row
must not write them. Everything else an inactive row computes is private
scratch the host ignores, and it still arrives on every counter, so the
schedule does not depend on the mask.
"""

from __future__ import annotations

from typing import Iterable


def row_active_mask(active_rows: Iterable[object] | None, batch_size: int) -> list[int]:
    if batch_size < 1:
        raise ValueError(f"batch_size must be >= 1; got {batch_size}")
    if active_rows is None:
        return [1] * batch_size
    mask = [1 if v else 0 for v in active_rows]
    if len(mask) != batch_size:
        raise ValueError(f"active_rows has {len(mask)} entries for a {batch_size}-row launch")
    if not any(mask):
        raise ValueError("active_rows activates no row; there is nothing to launch")
    return mask
