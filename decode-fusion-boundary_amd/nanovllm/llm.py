"""``LLM`` entry point (reference ``src/nanovllm/llm.py:1-5``)."""

from nanovllm.engine.llm_engine import LLMEngine


class LLM(LLMEngine):
    pass
