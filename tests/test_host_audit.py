"""Host audit of a step's rows (``taskgraph.audit_rows``): what it accepts and
the first bad row it names. Runs on the CPU (no decoder, no device)."""

from __future__ import annotations

import pytest

from nanovllm.backends.megakernel.native import MegakernelError
from nanovllm.backends.megakernel.taskgraph import audit_rows

GEO = dict(block_size=256, num_blocks=10, max_model_len=2048, max_pages=8)


def test_accepts_valid_rows_and_ignores_padding():
    # pages past position // block_size are padding and are not checked
    audit_rows([1, 151935], [0, 511], [[3, 99], [4, 9, -1]], **GEO)
    audit_rows([7], [2047], [[0, 1, 2, 3, 4, 5, 6, 7]], **GEO)


@pytest.mark.parametrize("ids,pos,tables,msg", [
    ([151936], [0], [[1]], "token id 151936"),
    ([-1], [0], [[1]], "token id -1"),
    ([5], [2048], [[1] * 8], "position 2048"),
    ([5], [-1], [[1]], "position -1"),
    ([5], [256], [[1]], "needs page 1"),
    ([5], [300], [[1, 10]], "block id 10 (page 1)"),
    ([5, 6], [0, 40], [[1], [-3]], "row 1: block id -3"),
    ([1] * 9, [0] * 9, [[1]] * 9, "9 rows"),
])
def test_rejects_the_first_bad_row(ids, pos, tables, msg):
    with pytest.raises(MegakernelError, match=msg.replace("(", r"\(").replace(")", r"\)")):
        audit_rows(ids, pos, tables, **GEO)


def test_max_model_len_bounds_positions():
    with pytest.raises(MegakernelError, match="position 600"):
        audit_rows([1], [600], [[1, 2, 3]], block_size=256, num_blocks=10, max_model_len=512, max_pages=2)
