"""GPU parity: the HIP decode step vs the CPU oracle on identical weights/inputs.

Bar (north star): logits max |diff| <= 2e-2 (fp32 accumulation, bf16 logits),
greedy token equal to the oracle's, KV cache writes equal within bf16
rounding, block-table/slot addressing exact (a wrong slot shows up as a KV
mismatch far above the tolerance).
"""

from __future__ import annotations

import pytest
import torch

from conftest import gpu_available
from gpu_support import Harness, max_abs

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not gpu_available(), reason="needs a ROCm GPU")]

LOGIT_TOL = 2e-2


@pytest.mark.parametrize("mode", ["persistent", "stages", "graph"])
def test_first_step_two_layers(mode):
    print(f"case: first step, 2 layers, mode={mode}", flush=True)
    h = Harness(num_layers=2, num_blocks=4)
    toks, logits = h.step([42], [0], [[1]], mode=mode)
    ref_toks, ref_logits = h.oracle_step([42], [0], [[1]])
    err = max_abs(logits, ref_logits)
    print(f"  tokens {toks} oracle {ref_toks} max|dlogit| {err:.3e}", flush=True)
    assert err <= LOGIT_TOL
    assert toks == ref_toks
    assert max_abs(h.kv.float().cpu(), h.kv_cpu.float()) <= 2e-2
    h.close()


@pytest.mark.parametrize("batch", [1, 4, 8])
def test_random_kv_context_256(batch):
    """C2-style: random KV of context 256 in shuffled physical blocks, full 28 layers."""
    print(f"case: random KV ctx 256, batch={batch}", flush=True)
    h = Harness(num_layers=28, num_blocks=2 * batch + 2, kv_fill_seed=1)
    ids = [(977 * (b + 1)) % 151936 for b in range(batch)]
    positions = [256 - (b % 3) for b in range(batch)]
    tables = [[2 * b + 3, 2 * b + 2] for b in range(batch)]
    toks, logits = h.step(ids, positions, tables)
    ref_toks, ref_logits = h.oracle_step(ids, positions, tables)
    err = max_abs(logits, ref_logits)
    print(f"  max|dlogit| {err:.3e} tokens {toks} oracle {ref_toks}", flush=True)
    assert err <= LOGIT_TOL
    assert toks == ref_toks
    kv_err = max_abs(h.kv.float().cpu(), h.kv_cpu.float())
    assert kv_err <= 2e-2, kv_err
    h.close()
