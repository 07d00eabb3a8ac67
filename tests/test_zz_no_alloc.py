"""The allocation-free entry point ``mkd_launch_persistent_noalloc`` against
``mkd_launch_persistent`` (include/mkd_abi.h): same schedule, same inputs, the
library's per-device scratch instead of the caller's workspace. Tokens, logits
and the KV cache writes must be bit-identical, on two calls in a row (8 rows,
then 2 rows), and the status word must read 0."""

from __future__ import annotations

import ctypes

import pytest
import torch

from conftest import gpu_available
from gpu_support import VOCAB, Harness

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not gpu_available(), reason="needs a ROCm GPU")]


def _run_noalloc(h: Harness, ids, pos, tables):
    """One step through the allocation-free entry point with the decoder's own
    schedule and row buffers; returns (tokens, logits, status)."""
    from nanovllm.backends.megakernel import native

    dec = h.dec
    rows = len(ids)
    width = max(len(t) for t in tables)
    dec.stage_rows(torch.tensor(ids, dtype=torch.int64, device="cuda"),
                   torch.tensor(pos, dtype=torch.int64, device="cuda"),
                   torch.tensor([list(t) + [0] * (width - len(t)) for t in tables], dtype=torch.int32,
                                device="cuda"))
    geo = dec.geometry_for(width * dec.block_size, rows)
    logits = torch.zeros(rows, VOCAB, dtype=torch.bfloat16, device="cuda")
    out = torch.full((rows,), -1, dtype=torch.int32, device="cuda")
    status = torch.full((1,), -7, dtype=torch.int32, device="cuda")
    desc = dec._desc_for(rows, geo, logits=logits)
    desc.out_tokens = out.data_ptr()
    desc.workspace = None
    desc.workspace_bytes = 0
    assert len(geo.persistent) == 1
    _, _, sched = geo.persistent[0]
    native.check(dec._lib.mkd_launch_persistent_noalloc(ctypes.byref(desc), ctypes.byref(sched),
                                                        status.data_ptr(), dec._stream_ptr()))
    torch.cuda.synchronize()
    return out.cpu().tolist(), logits.float().cpu(), int(status.item())


def test_noalloc_matches_workspace_entry_two_calls():
    print("case: no-alloc entry vs workspace entry, 2 layers, 8 rows then 2 rows", flush=True)
    h = Harness(num_layers=2, num_blocks=24, kv_fill_seed=4, variant="tagged")
    kv0 = h.kv.clone()
    cases = [
        ([11, 22, 33, 44, 55, 66, 77, 88], [700, 3, 256, 1023, 90, 0, 511, 1500],
         [[1, 2, 3], [4], [5, 6], [7, 8, 9, 10], [11], [12], [13, 14], [15, 16, 17, 18, 19, 20]]),
        ([99, 151935], [300, 40], [[21, 22], [23]]),
    ]
    for ids, pos, tables in cases:
        h.kv.copy_(kv0)
        ref_toks, ref_logits = h.step(ids, pos, tables)
        kv_ref = h.kv.clone()
        h.kv.copy_(kv0)
        toks, logits, status = _run_noalloc(h, ids, pos, tables)
        print(f"  rows {len(ids)}: tokens {toks} vs {ref_toks}, status {status}", flush=True)
        assert status == 0
        assert toks == ref_toks
        assert torch.equal(logits, ref_logits)
        assert torch.equal(h.kv, kv_ref)
    h.close()
