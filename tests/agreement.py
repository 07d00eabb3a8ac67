"""Greedy-token agreement classes, by the rule of the reference's correctness
smoke (``tools/correctness_smoke.py:318-362``):

* PASS -- every sequence token-for-token identical;
* CASCADE -- every divergence starts at a decode token (index >= 1; index 0
  is the prefill's token and must match) and no length differs: the bf16
  reduction-order cascade, tolerated;
* FAIL -- a divergence at token 0, or a length or sequence-count mismatch.
"""

from __future__ import annotations


def classify(reference: list[list[int]], actual: list[list[int]]) -> tuple[str, list[dict]]:
    details: list[dict] = []
    failed = len(reference) != len(actual)
    if failed:
        details.append({"kind": "count", "reference": len(reference), "actual": len(actual)})
    for i, (ref, act) in enumerate(zip(reference, actual)):
        if ref == act:
            continue
        if len(ref) != len(act):
            failed = True
            details.append({"seq": i, "kind": "length", "reference": len(ref), "actual": len(act)})
            continue
        first = next(j for j, (a, b) in enumerate(zip(ref, act)) if a != b)
        failed |= first == 0
        details.append({"seq": i, "kind": "token", "first": first, "expected": ref[first], "actual": act[first]})
    if failed:
        return "FAIL", details
    return ("CASCADE" if details else "PASS"), details
