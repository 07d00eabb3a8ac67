"""ctypes binding of ``libmkd_decode.so`` (declared in ``include/mkd_abi.h``).

The Python side reaches the HIP kernels only through these C entry points;
PyTorch-ROCm supplies device memory (tensor ``data_ptr()``s) and the current
stream handle. Every call checks the return code and raises
:class:`MegakernelError` with the library's message.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

MKD_ABI_VERSION = 1
MAX_BATCH = 8
MAX_SPLITS = 16
MAX_POSITION = 2048   # rows of the RoPE tables (MKD_MAX_POSITION)
INST_WORDS = 8
MAX_LM_SLOTS = 1024
LAYER_PTRS = 11
TW_REPLICAS = 8          # replicas of the tagged buffers every workgroup reads (one per XCD)
KV_CHUNK = 32            # positions per KV chunk the tagged kernel stages (block_size must be a multiple)
# ATTN task word a0 = b * 8 + h; the tagged kernel runs one query head per task:
# ATTN_ONE_HEAD set, and ATTN_QHEAD set for the second head (2h + 1) of KV head h
ATTN_QHEAD = 64
ATTN_ONE_HEAD = 128
# GATEUP task word a2 (tagged kernel): publish the residual for the next launch
GATEUP_PUBLISH_RES = 1
# QKV task word a2 (tagged kernel, one launch per stage): publish the residual after the input add
QKV_PUBLISH_RES = 1

FLAG_ADVANCE = 1
FLAG_ZERO_FANIN = 2
FLAG_PK_V1 = 4
FLAG_PK_V3 = 8
FLAG_PK_TAGGED = 16
PERSISTENT_VARIANTS = {"lds_dma": 0, "v1": FLAG_PK_V1, "tagged": FLAG_PK_TAGGED}

OP_NOP, OP_QKV, OP_ATTN, OP_OPROJ, OP_GATEUP, OP_DOWN, OP_LMHEAD = range(7)
OP_NAMES = {OP_NOP: "NOP", OP_QKV: "QKV", OP_ATTN: "ATTN", OP_OPROJ: "OPROJ",
            OP_GATEUP: "GATEUP", OP_DOWN: "DOWN", OP_LMHEAD: "LMHEAD"}

EXPORTED_SYMBOLS = (
    "mkd_abi_version", "mkd_last_error", "mkd_device_info", "mkd_workspace_bytes",
    "mkd_status_offset",
    "mkd_reset_counters", "mkd_launch_persistent", "mkd_launch_stages",
    "mkd_check_error", "mkd_graph_create", "mkd_graph_launch", "mkd_graph_destroy",
    "mkd_launch_persistent_noalloc",
)


class MegakernelError(RuntimeError):
    """A library call returned an error code."""


class MkdStepDesc(ctypes.Structure):
    _fields_ = [
        ("layer_ptrs", ctypes.c_void_p),
        ("embed", ctypes.c_void_p),
        ("final_norm", ctypes.c_void_p),
        ("rope_cos", ctypes.c_void_p),
        ("rope_sin", ctypes.c_void_p),
        ("k_cache", ctypes.c_void_p),
        ("v_cache", ctypes.c_void_p),
        ("kv_layer_stride", ctypes.c_int64),
        ("num_blocks", ctypes.c_int32),
        ("block_size", ctypes.c_int32),
        ("page_table", ctypes.c_void_p),
        ("page_stride", ctypes.c_int32),
        ("_pad0", ctypes.c_int32),
        ("cache_seqlens", ctypes.c_void_p),
        ("row_active", ctypes.c_void_p),
        ("input_ids", ctypes.c_void_p),
        ("out_tokens", ctypes.c_void_p),
        ("out_logits", ctypes.c_void_p),
        ("workspace", ctypes.c_void_p),
        ("workspace_bytes", ctypes.c_uint64),
        ("rows", ctypes.c_int32),
        ("batch", ctypes.c_int32),
        ("num_layers", ctypes.c_int32),
        ("lm_slots", ctypes.c_int32),
        ("flags", ctypes.c_uint32),
        ("_pad1", ctypes.c_int32),
        ("trace", ctypes.c_void_p),
    ]


class MkdSchedule(ctypes.Structure):
    _fields_ = [
        ("inst", ctypes.c_void_p),
        ("num_inst", ctypes.c_void_p),
        ("grid", ctypes.c_int32),
        ("max_inst", ctypes.c_int32),
    ]


class MkdStage(ctypes.Structure):
    _fields_ = [
        ("op", ctypes.c_int32),
        ("layer", ctypes.c_int32),
        ("first", ctypes.c_int32),
        ("count", ctypes.c_int32),
    ]


_lib = None
_lock = threading.Lock()


def _declare(lib) -> None:
    P = ctypes.POINTER
    lib.mkd_abi_version.restype = ctypes.c_int
    lib.mkd_abi_version.argtypes = []
    lib.mkd_last_error.restype = ctypes.c_char_p
    lib.mkd_last_error.argtypes = []
    lib.mkd_device_info.restype = ctypes.c_int
    lib.mkd_device_info.argtypes = [ctypes.c_int, P(ctypes.c_int32), P(ctypes.c_int32)]
    lib.mkd_workspace_bytes.restype = ctypes.c_uint64
    lib.mkd_workspace_bytes.argtypes = []
    lib.mkd_status_offset.restype = ctypes.c_uint64
    lib.mkd_status_offset.argtypes = []
    lib.mkd_reset_counters.restype = ctypes.c_int
    lib.mkd_reset_counters.argtypes = [P(MkdStepDesc), ctypes.c_void_p]
    lib.mkd_launch_persistent.restype = ctypes.c_int
    lib.mkd_launch_persistent.argtypes = [P(MkdStepDesc), P(MkdSchedule), ctypes.c_void_p]
    lib.mkd_launch_persistent_noalloc.restype = ctypes.c_int
    lib.mkd_launch_persistent_noalloc.argtypes = [P(MkdStepDesc), P(MkdSchedule), ctypes.c_void_p,
                                                  ctypes.c_void_p]
    lib.mkd_launch_stages.restype = ctypes.c_int
    lib.mkd_launch_stages.argtypes = [P(MkdStepDesc), ctypes.c_void_p, P(MkdStage),
                                      ctypes.c_int32, ctypes.c_void_p]
    lib.mkd_check_error.restype = ctypes.c_int
    lib.mkd_check_error.argtypes = [P(MkdStepDesc), ctypes.c_void_p, P(ctypes.c_int32)]
    lib.mkd_graph_create.restype = ctypes.c_int
    lib.mkd_graph_create.argtypes = [P(MkdStepDesc), ctypes.c_int32, P(MkdSchedule),
                                     ctypes.c_void_p, P(MkdStage), ctypes.c_int32,
                                     ctypes.c_int32, ctypes.c_void_p, P(ctypes.c_void_p)]
    lib.mkd_graph_launch.restype = ctypes.c_int
    lib.mkd_graph_launch.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
    lib.mkd_graph_destroy.restype = ctypes.c_int
    lib.mkd_graph_destroy.argtypes = [ctypes.c_void_p]


def load(path: str | Path | None = None):
    """Load (once) and return the library handle."""

    global _lib
    with _lock:
        if _lib is not None and path is None:
            return _lib
        from .build import library_path

        target = Path(path) if path is not None else library_path()
        if not target.exists():
            raise MegakernelError(
                f"{target} is not built; run __graft_entry__.build() or "
                "nanovllm.backends.megakernel.build.build()"
            )
        lib = ctypes.CDLL(str(target))
        _declare(lib)
        version = lib.mkd_abi_version()
        if version != MKD_ABI_VERSION:
            raise MegakernelError(f"ABI version {version} != expected {MKD_ABI_VERSION}")
        if path is None:
            _lib = lib
        return lib


def check(rc: int, lib=None) -> None:
    if rc != 0:
        lib = lib or load()
        msg = lib.mkd_last_error().decode(errors="replace")
        raise MegakernelError(f"libmkd_decode error {rc}: {msg}")


def workspace_bytes() -> int:
    return int(load().mkd_workspace_bytes())


def workspace_layout() -> dict[str, tuple[int, int]]:
    """``name -> (byte offset, bytes)`` of the workspace regions (``csrc/mkd_common.h``).
    Used by tests to read the kernels' intermediate activations. Regions named
    ``tw_*`` are the tagged exchange of the persistent "tagged" variant: 64-bit
    words, low half two bf16 values (fp32 for ``tw_apart``/``tw_lm``), high half
    the tag ``(epoch + 1) * 32 + layer``."""

    maxb, h, i, qkv, qs, kv_heads, layers = MAX_BATCH, 1024, 3072, 4096, 2048, 8, 28
    part_stride = 2 * 128 + 2 * 2
    regions = [
        ("resid", 2 * maxb * h * 2), ("hid_a", maxb * h * 2), ("hid_f", maxb * h * 2),
        ("qkv", maxb * qkv * 2), ("attn", maxb * qs * 2), ("act", maxb * i * 2),
        ("apart", 4 * maxb * kv_heads * MAX_SPLITS * part_stride), ("lmpart", 8 * MAX_LM_SLOTS * maxb),
    ]
    out, off = {}, 0
    for name, size in regions:
        out[name] = (off, size)
        off += size
    ctr_lines = 3 + layers * maxb * kv_heads + layers * (kv_heads + 4) * 8
    out["counters"] = (off, 128 * ctr_lines)
    off = (off + 128 * ctr_lines + 255) & ~255
    group = [("tw_res1", maxb * h // 2), ("tw_res2", maxb * h // 2), ("tw_attn", maxb * qs // 2),
             ("tw_o", maxb * h // 2), ("tw_act", maxb * i // 2), ("tw_down", maxb * h // 2)]
    group_words = sum(n for _, n in group)
    for name, n in group:      # replica 0 of the replicated buffers
        out[name] = (off, 8 * n)
        off += 8 * n
    out["tw_replica_stride"] = (8 * group_words, 0)
    off += 8 * group_words * (TW_REPLICAS - 1)
    for name, n in [("tw_qkv", maxb * qkv // 2), ("tw_apart", maxb * kv_heads * MAX_SPLITS * part_stride),
                    ("tw_lm", MAX_LM_SLOTS * maxb * 2)]:
        out[name] = (off, 8 * n)
        off += 8 * n
    out["end"] = (off, 0)
    return out


def decode_tagged_bf16(raw_u8, rows: int, width: int):
    """Values of a tagged bf16 region (uint8 tensor of its bytes) as float [rows, width],
    plus the tags [rows, width // 2]."""

    import torch

    words = raw_u8.view(torch.int64)[: rows * width // 2].view(rows, width // 2)
    lo = (words & 0xFFFFFFFF)
    vals = torch.stack([(lo & 0xFFFF), (lo >> 16) & 0xFFFF], dim=-1).reshape(rows, width)
    as_bf16 = vals.to(torch.int16).view(torch.bfloat16).float()
    tags = (words >> 32) & 0xFFFFFFFF
    return as_bf16, tags
