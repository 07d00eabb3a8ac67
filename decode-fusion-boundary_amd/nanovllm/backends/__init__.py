"""Optional decode backends (reference ``src/nanovllm/backends/__init__.py``)."""

from nanovllm.backends.megakernel import MegakernelBackend

__all__ = ["MegakernelBackend"]
