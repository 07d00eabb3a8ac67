"""GPU checks of the step's integer contract and error paths, through the C ABI.

* Greedy argmax (reference ``layers/sampler.py:5-16``: ``logits.float().argmax``,
  the first maximal index, a NaN ranking above every number): exact bf16 ties
  built by duplicating embedding rows of the tied LM head (in the same 8-row
  chunk, in another LM slot, and at a higher index), at batch 1 and 8, on the
  tagged persistent kernel and the per-op hipGraph path.
* A cached position whose block id lies outside the cache: the step reports
  ``MegakernelError`` (device error word), every kernel exits normally, and the
  next step on the same decoder is correct again.
* C1 end to end through ``LLM(..., decode_backend="megakernel")`` with one
  prompt (so every decode step takes the batch-1 ``decode_row`` path), against
  the committed oracle golden ``tests/golden/c1_greedy.json``, classified as the
  reference's correctness smoke does (``tools/correctness_smoke.py:318-362``).
"""

from __future__ import annotations

import json
import os

import pytest
import torch

from agreement import classify
from conftest import ROOT, gpu_available
from gpu_support import Harness

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not gpu_available(), reason="needs a ROCm GPU")]

V = 151936


def _tie_rows(j: int, taken: set[int]) -> list[int]:
    """Vocabulary rows to duplicate row j into: its neighbour in the same
    8-row chunk, one ~700 rows lower (another LM slot) and one higher."""
    same_chunk = j - 1 if j % 8 else j + 1
    far = j - 700 if j >= 700 else j + 700
    higher = min(j + 3, V - 1)
    return [r for r in (same_chunk, far, higher) if r not in taken and r != j]


@pytest.mark.parametrize("launch", ["persistent", "graph"])
@pytest.mark.parametrize("batch", [1, 8])
def test_argmax_exact_ties_take_the_first_index(batch, launch):
    print(f"case: argmax ties, batch {batch}, launch {launch}", flush=True)
    variant = "tagged" if launch == "persistent" else "lds_dma"
    h = Harness(num_layers=2, num_blocks=batch + 1, launch=launch, variant=variant)
    ids = [(7919 * (b + 3)) % V for b in range(batch)]
    pos = [5 + b for b in range(batch)]
    tables = [[b] for b in range(batch)]
    toks0, logits0 = h.step(ids, pos, tables)
    emb = h.w["embed"]
    taken = set(ids)
    tied = {}
    for b in range(batch):
        j = int(torch.argmax(logits0[b]))
        rows = _tie_rows(j, taken | set(tied))
        for r in rows:
            emb[r].copy_(emb[j])
        taken |= set(rows) | {j}
        tied[j] = rows
    torch.cuda.synchronize()
    toks, logits = h.step(ids, pos, tables)
    n_tied_rows = 0
    for b in range(batch):
        row = logits[b]
        best = row.max()
        first = int(torch.argmax(row))
        n_max = int((row == best).sum())
        n_tied_rows += n_max >= 2
        print(f"  row {b}: token {toks[b]}, first maximal index {first}, {n_max} maximal entries", flush=True)
        assert toks[b] == first
    # every row whose own top was duplicated must see an exact tie
    assert n_tied_rows >= 1 and (batch == 1 or n_tied_rows >= batch // 2), n_tied_rows
    h.close()


@pytest.mark.parametrize("launch", ["persistent", "graph"])
def test_argmax_nan_logit_wins_like_torch(launch):
    print(f"case: argmax NaN logits, launch {launch}", flush=True)
    variant = "tagged" if launch == "persistent" else "lds_dma"
    h = Harness(num_layers=1, num_blocks=3, launch=launch, variant=variant)
    emb = h.w["embed"]
    emb[90001].fill_(float("nan"))
    emb[120000].fill_(float("nan"))
    torch.cuda.synchronize()
    toks, logits = h.step([5, 6], [0, 7], [[1], [2]])
    for b in range(2):
        assert int(torch.argmax(logits[b])) == 90001
    assert toks == [90001, 90001], toks
    h.close()


@pytest.mark.parametrize("mode,variant", [("persistent", "tagged"), ("persistent", "lds_dma"),
                                          ("graph", "lds_dma")])
def test_bad_cached_block_id_is_an_error_not_a_fault(mode, variant):
    from nanovllm.backends.megakernel.native import MegakernelError

    print(f"case: bad cached block id, mode {mode} variant {variant}", flush=True)
    h = Harness(num_layers=2, num_blocks=6, kv_fill_seed=2, launch=mode, variant=variant)
    # row 0 at position 300 reads page 0 (block 1, cached) and writes page 1 (block 2);
    # the cached page's id is out of range, the written one is valid
    ids, pos = [17, 23], [300, 40]
    with pytest.raises(MegakernelError, match="out of range"):
        h.step(ids, pos, [[99, 2], [3]])
    torch.cuda.synchronize()
    # the decoder is usable again (the error path reset its counters)
    h.kv.copy_(h.kv_cpu.to("cuda"))
    toks, logits = h.step(ids, pos, [[1, 2], [3]])
    ref_toks, ref_logits = h.oracle_step(ids, pos, [[1, 2], [3]])
    assert (logits - ref_logits).abs().max().item() <= 2e-2
    assert toks == ref_toks
    h.close()


def test_c1_engine_batch1_path_against_golden(tmp_path):
    """C1: one prompt of 16 ids, 32 greedy tokens, 28 layers, block 256, through
    the engine (torch prefill, megakernel decode on the batch-1 path)."""
    from nanovllm import LLM, SamplingParams
    from nanovllm.synthetic import write_model_dir

    golden = json.load(open(os.path.join(ROOT, "tests", "golden", "c1_greedy.json")))
    path = write_model_dir(str(tmp_path / "c1"), num_layers=28)
    llm = LLM(path, max_model_len=2048, num_kvcache_blocks=4, max_num_seqs=1, decode_backend="megakernel")
    sp = SamplingParams(temperature=0.0, max_tokens=32, ignore_eos=True)
    try:
        out = llm.generate_with_metrics([golden["prompt"]], sp)
    finally:
        llm.exit()
    toks = out["outputs"][0]["token_ids"]
    m = out["metrics"]
    assert set(m["decode_backends"]) == {"megakernel"} and not m["fallback_reasons"], m
    status, details = classify([golden["tokens"]], [toks])
    print(f"  C1 megakernel {toks}\n  golden        {golden['tokens']}\n  status {status} {details}", flush=True)
    report = {"config": "C1: 28 layers, 16-token prompt, 32 greedy tokens, engine with torch prefill and "
                        "megakernel batch-1 decode, vs the CPU oracle golden",
              "status": status, "details": details, "tokens": toks, "golden": golden["tokens"],
              "agree": sum(a == b for a, b in zip(toks, golden["tokens"]))}
    os.makedirs(os.path.join(ROOT, "gpurun_out"), exist_ok=True)
    with open(os.path.join(ROOT, "gpurun_out", "agreement_c1.json"), "w") as f:
        json.dump(report, f, indent=1)
    assert status != "FAIL", details


@pytest.mark.parametrize("batch", [1, 8])
def test_torch_operator_step_matches_ctypes_step(batch):
    """The step driven through ``torch.ops.nanovllm_megakernel_C.mkd_decode_step``
    (the C++ shim on the device dispatch key) gives bit-identical tokens, logits
    and KV writes to the ctypes call of the C ABI, and raises on a bad call."""
    from nanovllm.backends.megakernel import torch_ops
    from nanovllm.backends.megakernel.taskgraph import TaskGraphDecoder

    print(f"case: torch operator vs ctypes, batch {batch}", flush=True)
    h = Harness(num_layers=2, num_blocks=2 * batch + 2, kv_fill_seed=6, variant="tagged")
    ids = [(311 * (b + 1)) % V for b in range(batch)]
    pos = [300 + 5 * b for b in range(batch)]
    tables = [[2 * b + 2, 2 * b + 3] for b in range(batch)]
    kv0 = h.kv.clone()
    ref_toks, ref_logits = h.step(ids, pos, tables)
    kv_ref = h.kv.clone()
    h.kv.copy_(kv0)
    op_dec = TaskGraphDecoder(h.w, k_cache=h.kv[0], v_cache=h.kv[1], block_size=256,
                              num_cache_blocks=2 * batch + 2, max_model_len=2048, binding="torch_ops")
    h.dec.close()
    h.dec = op_dec
    toks, logits = h.step(ids, pos, tables)
    print(f"  tokens {toks} vs {ref_toks}", flush=True)
    assert toks == ref_toks
    assert torch.equal(logits, ref_logits)
    assert torch.equal(h.kv, kv_ref)
    # a non-zero return code of the library becomes a RuntimeError with its message
    ops = torch_ops.load()
    with pytest.raises(RuntimeError, match="batch must be 1, 2, 4 or 8"):
        geo = op_dec._geometry(1, 1)
        inst, num, sched = geo.persistent[0]
        ops.mkd_decode_step(op_dec._layer_ptrs, h.w["embed"], h.w["final_norm"], h.w["cos"], h.w["sin"],
                            op_dec._k_cache, op_dec._v_cache, op_dec._table, op_dec._seqlens, op_dec._row_active,
                            op_dec._ids, op_dec._op_tokens, None, op_dec._workspace, inst, num, sched.grid,
                            sched.max_inst, 1, 3, 2, 1, 16, 2 * batch + 2, 256)
    h.close()
