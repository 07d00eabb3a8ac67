"""The PASS / CASCADE / FAIL rule of tests/agreement.py on hand-made cases
(reference ``tools/correctness_smoke.py:318-362``)."""

from agreement import classify


def test_pass_cascade_fail():
    assert classify([[1, 2, 3]], [[1, 2, 3]]) == ("PASS", [])
    status, det = classify([[1, 2, 3], [4, 5]], [[1, 9, 3], [4, 5]])
    assert status == "CASCADE" and det == [{"seq": 0, "kind": "token", "first": 1, "expected": 2, "actual": 9}]
    assert classify([[1, 2]], [[7, 2]])[0] == "FAIL"            # token 0 is the prefill's
    assert classify([[1, 2]], [[1, 2, 3]])[0] == "FAIL"         # length mismatch
    assert classify([[1], [2]], [[1]])[0] == "FAIL"             # sequence count
