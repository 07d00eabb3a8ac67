"""nano-vLLM-compatible host surface for the MI355X decode-step engine.

Mirrors the public API of the reference package (``LLM``, ``SamplingParams``;
reference ``src/nanovllm/__init__.py:1-15``). Both names are resolved lazily so
that importing the package never imports torch or builds the HIP library.
"""

__all__ = ["LLM", "SamplingParams"]


def __getattr__(name):
    if name == "LLM":
        from nanovllm.llm import LLM

        return LLM
    if name == "SamplingParams":
        from nanovllm.sampling_params import SamplingParams

        return SamplingParams
    raise AttributeError(f"module {__name__!r} has no attribute {name!r}")
