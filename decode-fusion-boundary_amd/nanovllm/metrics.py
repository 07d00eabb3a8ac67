"""Per-request and per-step metrics (subset of reference ``metrics.py:233-372``):
TTFT / TPOT, decode step wall times, which backend ran each decode step and
the fallback reasons seen."""

from __future__ import annotations

import statistics
from collections import Counter


class MetricsCollector:
    def __init__(self, decode_backend: str):
        self.decode_backend = decode_backend
        self.requests: dict[int, dict] = {}
        self.decode_steps: list[float] = []
        self.prefill_steps: list[float] = []
        self.backends = Counter()
        self.fallback_reasons = Counter()

    def add_request(self, seq_id: int, prompt_tokens: int, t: float) -> None:
        self.requests[seq_id] = {"prompt_tokens": prompt_tokens, "arrival": t, "tokens": []}

    def record_step(self, seqs, is_prefill: bool, duration: float, backend: str, reason) -> None:
        (self.prefill_steps if is_prefill else self.decode_steps).append(duration)
        if not is_prefill:
            self.backends[backend] += 1
            if reason:
                self.fallback_reasons[reason] += 1

    def record_token(self, seq_id: int, t: float) -> None:
        self.requests[seq_id]["tokens"].append(t)

    def report(self, wall_time: float, scheduler_stats: dict | None = None) -> dict:
        ttft = [r["tokens"][0] - r["arrival"] for r in self.requests.values() if r["tokens"]]
        tpot = []
        for r in self.requests.values():
            ts = r["tokens"]
            if len(ts) > 1:
                tpot.append((ts[-1] - ts[0]) / (len(ts) - 1))
        generated = sum(len(r["tokens"]) for r in self.requests.values())
        med = lambda xs: statistics.median(xs) if xs else None  # noqa: E731
        return {
            "decode_backend": self.decode_backend,
            "wall_time_s": wall_time,
            "generated_tokens": generated,
            "tokens_per_s": generated / wall_time if wall_time > 0 else None,
            "ttft_median_s": med(ttft),
            "tpot_median_s": med(tpot),
            "decode_step_median_s": med(self.decode_steps),
            "decode_steps": len(self.decode_steps),
            "decode_backends": dict(self.backends),
            "fallback_reasons": dict(self.fallback_reasons),
            "scheduler": scheduler_stats or {},
        }
