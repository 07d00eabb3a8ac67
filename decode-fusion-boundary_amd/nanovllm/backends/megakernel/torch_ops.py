"""The decode step as torch operators: ``torch.ops.nanovllm_megakernel_C``.

``libmkd_torch_ops.so`` (built from ``csrc/mkd_torch_ops.cpp`` by
:func:`build.build`) registers ``mkd_decode_step`` and ``mkd_reset_counters`` on
the device dispatch key, as the reference's extension registers ``tg_decode_step``
and ``tg_zero_regions`` (``csrc/torch_bindings.cpp:227-264``). The operators
check their tensors, call the C ABI on the current stream and raise
``RuntimeError`` on a non-zero return code. :func:`load` fails loudly when the
shim is not built.
"""

from __future__ import annotations

import threading

import torch

from . import build, native

NAMESPACE = "nanovllm_megakernel_C"
_loaded = False
_lock = threading.Lock()


def load():
    """Register the operators (once) and return ``torch.ops.nanovllm_megakernel_C``."""

    global _loaded
    with _lock:
        if not _loaded:
            native.load()  # the C-ABI library the shim links against, ABI-checked
            path = build.TORCH_OPS_PATH
            if not path.exists():
                raise native.MegakernelError(
                    f"{path} is not built; run __graft_entry__.build() or "
                    "nanovllm.backends.megakernel.build.build()")
            torch.ops.load_library(str(path))
            _loaded = True
    return getattr(torch.ops, NAMESPACE)
