"""Per-request sampling knobs (reference ``src/nanovllm/sampling_params.py:5-21``).

Greedy decoding is ``temperature <= 1e-10``; that is the only mode the
megakernel backend admits.
"""

from dataclasses import dataclass

GREEDY_TEMPERATURE = 1e-10


@dataclass(slots=True)
class SamplingParams:
    temperature: float = 1.0
    max_tokens: int = 64
    ignore_eos: bool = False

    def __post_init__(self):
        if self.temperature < 0.0:
            raise ValueError("temperature must be non-negative")
        if self.max_tokens < 1:
            raise ValueError("max_tokens must be at least 1")

    @property
    def is_greedy(self) -> bool:
        return self.temperature <= GREEDY_TEMPERATURE
