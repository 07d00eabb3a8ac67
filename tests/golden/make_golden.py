"""Writes the golden fixtures under tests/golden/.

* kv_contract.json -- the numeric cases of the reference's own KV tests
  (tests/test_paged_kv.py:17-81, tests/test_kv_block_boundary.py:78-300,
  tests/test_kv_cache_indexing.py:84-190), written down as input/output data.
* c1_greedy.json -- BASELINE config C1 on the CPU oracle: seed-0 random-init
  Qwen3-0.6B geometry, one prompt of 16 ids ~ U[0, 151936) (torch.Generator
  seed 0), 32 greedy tokens, block size 256 (first-token logit slice and the
  token sequence).

Run from the repository root: ``python tests/golden/make_golden.py``.
"""

from __future__ import annotations

import json
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "decode-fusion-boundary_amd"))
sys.path.insert(0, ROOT)


def kv_contract() -> dict:
    bs = 256
    return {
        "paged_spec_small": {  # PagedKVCacheSpec(2, 16, 4, 2, 8, 2)
            "spec": [2, 16, 4, 2, 8, 2], "shape": [2, 2, 16, 4, 2, 8],
            "token_stride": 16, "block_stride": 64, "layer_stride": 1024, "total_bytes": 8192,
            "physical_slot": [[[7, 3, 12], 0, [7, 0]], [[7, 3, 12], 5, [3, 1]], [[7, 3, 12], 11, [12, 3]]],
            "element_offset": [[1, [7, 3, 12], 5, 1, 2, 1 * 1024 + 3 * 64 + 1 * 16 + 1 * 8 + 2]],
        },
        "paged_spec_model": {"spec": [28, 32, 256, 8, 128, 2], "shape": [2, 28, 32, 256, 8, 128],
                             "physical_slot": [[[11, 4], 257, [4, 1]]]},
        "block_size": bs,
        # prompt length -> blocks after prefill, last-block tokens, first decode position, slot of that position
        "prefill": [[255, 1, 255], [256, 1, 256], [257, 2, 1]],
        "first_decode": [[255, 255, [0, 255]], [256, 256, [1, 0]], [257, 257, [1, 1]]],
        "decode_slot_legacy": [[n, list(range(100, 100 + (n + bs - 1) // bs))] for n in (1, 255, 256, 257, 512, 513)],
        "chunked_prefill": {"prompt": 300, "start": 256, "end": 300, "count": 44, "first": [1, 0], "last": [1, 43]},
        "pad_value": 0,
        "padded_tables": {"short": [0, 1], "long": [2, 3, 4, 5, 6], "block_size": 16, "num_blocks": 64},
    }


def c1_greedy() -> dict:
    import torch

    from nanovllm.synthetic import make_weights
    from oracle.qwen3_oracle import Oracle

    gen = torch.Generator().manual_seed(0)
    prompt = torch.randint(0, 151936, (16,), generator=gen).tolist()
    oracle = Oracle(make_weights(seed=0))
    kc = torch.zeros(28, 1, 256, 8, 128, dtype=torch.bfloat16)
    vc = torch.zeros_like(kc)
    logits, toks = oracle.teacher_force(prompt, [0], kc, vc)
    first_logits = logits[0].float()
    out = [toks[0]]
    for i in range(31):
        _, t = oracle.decode_step([out[-1]], [len(prompt) + i], [[0]], kc, vc)
        out.append(t[0])
    top = torch.topk(first_logits, 8)
    return {"prompt": prompt, "tokens": out, "first_step_top8_ids": top.indices.tolist(),
            "first_step_top8_logits": top.values.tolist(),
            "first_step_logit_sum": float(first_logits.double().sum()),
            "note": "CPU oracle, seed-0 synthetic weights (N(0,0.02) matrices, N(1,0.02) norms)"}


if __name__ == "__main__":
    with open(os.path.join(HERE, "kv_contract.json"), "w") as f:
        json.dump(kv_contract(), f, indent=1)
    with open(os.path.join(HERE, "c1_greedy.json"), "w") as f:
        json.dump(c1_greedy(), f, indent=1)
    print("wrote kv_contract.json and c1_greedy.json")
