"""The C ABI (include/mkd_abi.h) and its ctypes mirror, on the CPU: the
library loads, exports every declared entry point, the POD layouts agree, and
host-side validation rejects bad descriptors without touching a device."""

from __future__ import annotations

import ctypes
import os
import re

import pytest

from conftest import ROOT
from nanovllm.backends.megakernel import build, native

HEADER = os.path.join(ROOT, "include", "mkd_abi.h")


def _lib():
    if not build.LIB_PATH.exists():
        pytest.skip("libmkd_decode.so not built (run __graft_entry__.build())")
    return native.load()


def declared_functions():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:int|uint64_t|const char\*)\s+(mkd_\w+)\s*\(", text, re.M)))


def test_every_declared_symbol_is_exported():
    lib = _lib()
    names = declared_functions()
    assert set(names) == set(native.EXPORTED_SYMBOLS)
    for name in names:
        assert hasattr(lib, name), name


def test_struct_layouts_match_header():
    text = open(HEADER).read()
    body = text[text.index("typedef struct MkdStepDesc"):text.index("} MkdStepDesc;")]
    fields = re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(\w+);", body, re.M)
    assert fields == [f for f, _ in native.MkdStepDesc._fields_]
    assert ctypes.sizeof(native.MkdStepDesc) == 176
    assert ctypes.sizeof(native.MkdSchedule) == 24 and ctypes.sizeof(native.MkdStage) == 16
    assert native.MkdStepDesc.kv_layer_stride.offset == 56


def test_constants_match_header_and_spec():
    from nanovllm.model_spec import QWEN3_06B

    text = open(HEADER).read()
    val = lambda n: int(re.search(rf"#define {n} (\d+)", text).group(1))  # noqa: E731
    assert val("MKD_ABI_VERSION") == native.MKD_ABI_VERSION
    assert val("MKD_HIDDEN") == QWEN3_06B.hidden_size and val("MKD_VOCAB") == QWEN3_06B.vocab_size
    assert val("MKD_NUM_LAYERS") == QWEN3_06B.num_layers and val("MKD_HEAD_DIM") == QWEN3_06B.head_dim
    assert val("MKD_MAX_BATCH") == native.MAX_BATCH and val("MKD_MAX_SPLITS") == native.MAX_SPLITS
    assert QWEN3_06B.weight_bytes() == 1_192_099_840


def test_workspace_layout_and_validation():
    lib = _lib()
    assert lib.mkd_abi_version() == native.MKD_ABI_VERSION
    layout = native.workspace_layout()
    assert layout["counters"][0] == lib.mkd_status_offset()
    assert lib.mkd_workspace_bytes() > lib.mkd_status_offset()
    desc = native.MkdStepDesc(batch=3, rows=1)
    rc = lib.mkd_launch_stages(ctypes.byref(desc), None, None, 0, None)
    assert rc == -1 and b"batch must be 1, 2, 4 or 8" in lib.mkd_last_error()
    desc = native.MkdStepDesc(batch=1, rows=1, num_layers=28, lm_slots=1)
    rc = lib.mkd_launch_persistent(ctypes.byref(desc), None, None)
    assert rc == -1 and b"workspace" in lib.mkd_last_error()


def test_tagged_region_layout_matches_library():
    """The Python view of the tagged exchange region ends exactly at the
    library's workspace size (same constants on both sides)."""
    lib = _lib()
    layout = native.workspace_layout()
    assert layout["end"][0] == lib.mkd_workspace_bytes()
    assert layout["tw_res1"][0] % 256 == 0


def test_torch_operator_shim_registers_the_ops():
    """libmkd_torch_ops.so loads on the CPU and registers the operators with the
    schema the decoder calls (reference torch_bindings.cpp:227-264 namespace)."""
    import torch

    if not build.TORCH_OPS_PATH.exists():
        pytest.skip("libmkd_torch_ops.so not built (run __graft_entry__.build())")
    from nanovllm.backends.megakernel import torch_ops

    ops = torch_ops.load()
    schema = str(ops.mkd_decode_step.default._schema)
    assert schema.startswith("nanovllm_megakernel_C::mkd_decode_step(Tensor layer_ptrs")
    for arg in ("Tensor(a!) k_cache", "Tensor(e!) workspace", "int block_size"):
        assert arg in schema, arg
    assert "Tensor(a!) workspace" in str(ops.mkd_reset_counters.default._schema)
    # a CPU tensor has no kernel on the CPU key: dispatch fails loudly, no silent fallback
    with pytest.raises((RuntimeError, NotImplementedError)):
        ops.mkd_reset_counters(torch.zeros(16, dtype=torch.uint8))
