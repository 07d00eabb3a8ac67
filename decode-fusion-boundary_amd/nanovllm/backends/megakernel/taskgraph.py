"""Task-graph decoder: owns the schedules, workspace and per-step staging.

Counterpart of the reference ``backends/megakernel/taskgraph.py``
(``TaskGraphDecoder`` :147-529, ``taskgraph_compatibility`` :92-131,
``resolve_num_sms`` :68-83, ``max_pages_per_seq`` :60-65, ``TG_MAX_BATCH`` :35).
Differences that matter:

* one schedule per (batch bucket 1/2/4/8, split-KV factor); a live batch of 3,
  5, 6 or 7 runs the next bucket with the extra rows inactive;
* the split-KV factor follows the context and the batch (one split per 256
  positions, never below ``megakernel_attn_splits``; for the tagged persistent
  kernel at most 16 // batch bucket);
* nothing is zeroed per step: the last LM-head task clears the fan-in
  counters and every ticket counter resets itself (the reference cleared about
  11.7 MB of scratch per step, ``taskgraph.py:289-295``);
* ``launch="graph"`` runs the same tasks one kernel per stage from a captured
  hipGraph (the comparator arm); ``"persistent"`` is one launch per segment.

The step returns after one 128-byte device-to-host read that carries both the
device error word and the sampled tokens.
"""

from __future__ import annotations

import dataclasses
import os
from dataclasses import dataclass
from typing import Any

import torch

from nanovllm.model_spec import QWEN3_06B

from . import native
from .row_contract import row_active_mask
from .schedule import (
    NUM_LAYERS, PAIR_HEADS_MIN_BATCH, Schedule, auto_attn_splits, batch_bucket, build_schedule, build_segments,
    build_stage_schedules, tagged_attn_splits, tagged_pair_heads,
)
from .verifier import verify
from .weights import pack_layer_pointers

TG_MAX_BATCH = native.MAX_BATCH
MAX_ATTN_SPLITS = native.MAX_SPLITS


def max_pages_per_seq(max_model_len: int, block_size: int) -> int:
    if block_size <= 0:
        raise ValueError("block_size must be positive")
    return max(1, -(-max_model_len // block_size))


def resolve_num_sms(device_cu_count: int) -> int:
    """Persistent grid: one workgroup per compute unit (``TG_NUM_SMS`` overrides)."""

    override = os.getenv("TG_NUM_SMS")
    if override:
        value = int(override)
        if value <= 0:
            raise ValueError(f"TG_NUM_SMS must be positive; got {value}")
        return min(value, int(device_cu_count))
    return max(1, int(device_cu_count))


@dataclass(frozen=True)
class TaskGraphCompatibility:
    supported: bool
    reason: str = ""


def taskgraph_compatibility(config: Any, seqs: list[Any], is_prefill: bool) -> TaskGraphCompatibility:
    """Torch-free admission policy; same rules and reason strings as the reference."""

    if is_prefill:
        return TaskGraphCompatibility(False, "Task-graph megakernel is decode-only; use the prefill backend")
    if not seqs:
        return TaskGraphCompatibility(False, "Task-graph megakernel needs at least one sequence")
    if len(seqs) > TG_MAX_BATCH:
        return TaskGraphCompatibility(
            False,
            f"Task-graph megakernel supports batch sizes 1..{TG_MAX_BATCH} "
            "(TG_MAX_BATCH, the compile-time scratch/bar ceiling)",
        )
    max_num_seqs = getattr(config, "max_num_seqs", None)
    if isinstance(max_num_seqs, int) and max_num_seqs < len(seqs):
        return TaskGraphCompatibility(False, f"batch {len(seqs)} exceeds max_num_seqs={max_num_seqs}")
    if getattr(config, "tensor_parallel_size", 1) != 1:
        return TaskGraphCompatibility(False, "Task-graph megakernel requires tensor_parallel_size=1")
    for seq in seqs:
        if bool(getattr(seq, "is_greedy", False)):
            continue
        temperature = getattr(seq, "temperature", None)
        if temperature is None or temperature > 1e-10:
            return TaskGraphCompatibility(False, "Task-graph megakernel supports greedy sampling only")
    return TaskGraphCompatibility(True)


def audit_rows(input_ids, positions, block_tables, *, block_size: int, num_blocks: int, max_model_len: int,
               max_pages: int) -> None:
    """Host audit of one step's rows (lists): at most 8 rows, token ids in the
    vocabulary, each position inside ``max_model_len`` and covered by its block
    table, and every block id the step reads or writes (pages ``0 .. position //
    block_size``) inside the cache. Raises :class:`MegakernelError` naming the
    first bad row."""

    rows = len(input_ids)
    if rows > TG_MAX_BATCH:
        raise native.MegakernelError(f"{rows} rows exceed the batch ceiling {TG_MAX_BATCH}")
    vocab = QWEN3_06B.vocab_size
    limit = min(max_model_len, native.MAX_POSITION)
    for r in range(rows):
        tok, pos, table = int(input_ids[r]), int(positions[r]), block_tables[r]
        if not 0 <= tok < vocab:
            raise native.MegakernelError(f"row {r}: token id {tok} outside [0, {vocab})")
        if not 0 <= pos < limit:
            raise native.MegakernelError(f"row {r}: position {pos} outside [0, {limit})")
        last = pos // block_size
        if last >= len(table) or last >= max_pages:
            raise native.MegakernelError(
                f"row {r}: position {pos} needs page {last} but the block table has {len(table)} pages")
        for i in range(last + 1):
            blk = int(table[i])
            if not 0 <= blk < num_blocks:
                raise native.MegakernelError(
                    f"row {r}: block id {blk} (page {i}) outside the cache's {num_blocks} blocks")


@dataclass
class _Geometry:
    batch: int
    attn_splits: int
    segments: list[Schedule]
    persistent: list[tuple[torch.Tensor, torch.Tensor, native.MkdSchedule]]
    stage_inst: torch.Tensor
    stages: Any            # ctypes array of MkdStage
    num_stages: int
    graph: Any = None      # captured per-op hipGraph (launch="graph")
    # tagged variant: the per-op comparator on the persistent kernel's task bodies,
    # one persistent launch per stage ((inst, num, MkdSchedule) each, and the array)
    stage_persistent: list = dataclasses.field(default_factory=list)
    stage_array: Any = None


def _check_tagged_preconditions(segs) -> None:
    """What the tagged-exchange kernel relies on: GEMV row blocks of even size at
    even offsets (a word carries two values of one task), at most 32 rows per
    block (its result tile), and an LM-head
    task on every workgroup of the last launch (the last LM slot advances the step counter once every workgroup has
    read it). Every workgroup also runs exactly one QKV and one gate/up task per
    layer of a launch: each keeps the residual stream in registers, updates it in
    every RMSNorm prologue, and flips a buffer parity per such task. A schedule with
    fewer QKV tasks than workgroups (32-row QKV blocks on 256 workgroups, measured)
    stalls the kernel until its dependency wait times out."""

    norm_ops = (native.OP_QKV, native.OP_GATEUP)
    for seg in segs:
        layers = {t.layer for row in seg.rows for t in row if t.op in norm_ops}
        want = {(op, layer): 1 for op in norm_ops for layer in layers}
        for w, row in enumerate(seg.rows):
            seen: dict[tuple[int, int], int] = {}
            for t in row:
                if t.op in norm_ops:
                    seen[(t.op, t.layer)] = seen.get((t.op, t.layer), 0) + 1
            if seen != want:
                (op, layer), n = next(((k, seen.get(k, 0)) for k in sorted(set(want) | set(seen))
                                       if seen.get(k, 0) != 1))
                raise RuntimeError(
                    f"workgroup {w} runs {n} tasks of op {op} in layer {layer}; the tagged exchange "
                    "needs exactly one QKV and one gate/up task per workgroup per layer")
            for t in row:
                if t.op in (native.OP_QKV, native.OP_OPROJ, native.OP_GATEUP, native.OP_DOWN):
                    # result-tile entries: GATEUP has 2 rows per channel, DOWN 2 partials per row
                    rows = 2 * t.a1 if t.op in (native.OP_GATEUP, native.OP_DOWN) else t.a1
                    if t.a0 % 2 or t.a1 % 2 or rows > 32:
                        raise RuntimeError(f"task {t} does not fit the tagged exchange (even blocks of <= 32 rows)")
    last = segs[-1]
    if any(not any(t.op == native.OP_LMHEAD for t in row) for row in last.rows):
        raise RuntimeError("the tagged exchange needs an LM-head task on every workgroup")


class TaskGraphDecoder:
    """One greedy decode step of up to 8 rows on the HIP task graph."""

    def __init__(self, weights: dict, *, k_cache, v_cache, block_size: int, num_cache_blocks: int,
                 max_model_len: int, attn_splits: int = 1, fusion_groups: int = 1,
                 launch: str = "persistent", verbose: bool = False, debug_bounds: bool = False,
                 persistent_variant: str = "tagged", binding: str = "ctypes",
                 attn_pair_heads: bool | None = None):
        self._lib = native.load()
        if binding not in ("ctypes", "torch_ops"):
            raise ValueError(f"binding must be 'ctypes' or 'torch_ops'; got {binding!r}")
        # how a persistent step reaches the library: ctypes calls of the C ABI, or
        # the registered torch operator (torch.ops.nanovllm_megakernel_C.mkd_decode_step)
        self.binding = binding
        self._ops = None
        if binding == "torch_ops":
            from . import torch_ops

            self._ops = torch_ops.load()
        if persistent_variant not in native.PERSISTENT_VARIANTS:
            raise ValueError(f"persistent_variant must be one of {sorted(native.PERSISTENT_VARIANTS)}; "
                             f"got {persistent_variant!r}")
        if persistent_variant == "tagged" and int(block_size) % native.KV_CHUNK != 0:
            # the tagged kernel stages KV chunks of 32 positions that must lie in one
            # cache block; other block sizes run the LDS-DMA kernel
            persistent_variant = "lds_dma"
        self.persistent_variant = persistent_variant
        self._variant_flags = native.PERSISTENT_VARIANTS[persistent_variant]
        if launch not in ("persistent", "graph"):
            raise ValueError(f"launch must be 'persistent' or 'graph'; got {launch!r}")
        self.launch = launch
        self.device = k_cache.device
        layers = weights["layers"]
        self.num_layers = len(layers)
        if self.num_layers > NUM_LAYERS:
            raise ValueError(f"at most {NUM_LAYERS} layers are compiled; got {self.num_layers}")
        self._weights = weights
        self._layer_ptrs = pack_layer_pointers(layers, device=self.device)
        self._k_cache, self._v_cache = k_cache, v_cache
        if k_cache.dim() != 5 or k_cache.shape != v_cache.shape or k_cache.dtype != torch.bfloat16:
            raise ValueError("k_cache/v_cache must be bf16 [layers, blocks, block_size, kv_heads, head_dim]")
        if not (k_cache.is_contiguous() and v_cache.is_contiguous()):
            raise ValueError("k_cache/v_cache views must be contiguous")
        self.block_size = int(block_size)
        self.num_cache_blocks = int(num_cache_blocks)
        self.max_pages = max_pages_per_seq(int(max_model_len), self.block_size)
        self.max_model_len = int(max_model_len)
        if not 1 <= attn_splits <= MAX_ATTN_SPLITS:
            raise ValueError(f"attn_splits must be 1..{MAX_ATTN_SPLITS}; got {attn_splits}")
        self.min_attn_splits = int(attn_splits)
        # tagged kernel: attention tasks of both query heads of a KV head (one read
        # of each K/V chunk) or of one query head; None: tagged_pair_heads(batch)
        self.attn_pair_heads = attn_pair_heads
        self.fusion_groups = int(fusion_groups)
        if not 1 <= self.fusion_groups <= self.num_layers:
            raise ValueError(f"fusion_groups must be in [1, {self.num_layers}]; got {fusion_groups}")
        self.verbose = verbose
        self.debug_bounds = debug_bounds

        cus = native.ctypes.c_int32()
        lds = native.ctypes.c_int32()
        dev_index = self.device.index if self.device.index is not None else torch.cuda.current_device()
        native.check(self._lib.mkd_device_info(dev_index, native.ctypes.byref(cus), native.ctypes.byref(lds)))
        self.grid = resolve_num_sms(cus.value)

        i32 = dict(dtype=torch.int32, device=self.device)
        self._workspace = torch.zeros(int(self._lib.mkd_workspace_bytes()), dtype=torch.uint8, device=self.device)
        self._status_off = int(self._lib.mkd_status_offset())
        # the status line's token slots (+64 bytes) as an int32 tensor: the tokens'
        # destination when the step goes through the torch operator
        self._op_tokens = self._workspace[self._status_off + 64:self._status_off + 128].view(torch.int32)
        self._op_logits = None
        # Per-step row inputs in one int32 buffer: token ids (int64, 16 words), positions
        # (8 words), block tables (8 x max_pages words). A pinned host mirror of the same
        # layout lets a host-side step stage all of them with one copy.
        self._rows_words = 2 * TG_MAX_BATCH + TG_MAX_BATCH + TG_MAX_BATCH * self.max_pages
        self._rows_dev = torch.zeros(self._rows_words, **i32)
        self._ids, self._seqlens, self._table = self._row_views(self._rows_dev)
        self._row_active = torch.ones(TG_MAX_BATCH, **i32)
        self._mask_dirty = False
        self._logits = None
        # pinned staging for host-side steps (decode_row / decode_rows_host) and the
        # status read; each step ends with a synchronous status read, so a step's
        # copies have completed before the next step rewrites these buffers
        self._rows_host = torch.zeros(self._rows_words, dtype=torch.int32, pin_memory=True)
        self._host_ids, self._host_pos, self._host_tables = self._row_views(self._rows_host)
        self._host_status = torch.zeros(32, dtype=torch.int32, pin_memory=True)

        kv_stride = k_cache.stride(0)
        w = weights
        self._desc = native.MkdStepDesc(
            layer_ptrs=self._layer_ptrs.data_ptr(), embed=w["embed"].data_ptr(),
            final_norm=w["final_norm"].data_ptr(), rope_cos=w["cos"].data_ptr(), rope_sin=w["sin"].data_ptr(),
            k_cache=k_cache.data_ptr(), v_cache=v_cache.data_ptr(), kv_layer_stride=kv_stride,
            num_blocks=self.num_cache_blocks, block_size=self.block_size,
            page_table=self._table.data_ptr(), page_stride=self.max_pages,
            cache_seqlens=self._seqlens.data_ptr(), row_active=self._row_active.data_ptr(),
            input_ids=self._ids.data_ptr(),
            out_tokens=self._workspace.data_ptr() + self._status_off + 64, out_logits=None,
            workspace=self._workspace.data_ptr(), workspace_bytes=self._workspace.numel(),
            rows=1, batch=1, num_layers=self.num_layers, lm_slots=1, flags=0,
        )
        self._stream_ptr()
        native.check(self._lib.mkd_reset_counters(native.ctypes.byref(self._desc), self._stream_ptr()))
        self._geometries: dict[tuple[int, int, bool], _Geometry] = {}
        for b in (1, 2, 4, 8):
            self._geometry(b, self.min_attn_splits)
        if verbose:
            g = self._geometries[(1, self.min_attn_splits, False)]
            print(f"taskgraph decoder: grid={self.grid} launch={self.launch} layers={self.num_layers} "
                  f"fusion_groups={self.fusion_groups} max_pages={self.max_pages} "
                  f"tasks(B=1)={sum(s.num_tasks for s in g.segments)}")

    # -- helpers -------------------------------------------------------------
    def _stream_ptr(self) -> int:
        return torch.cuda.current_stream(self.device).cuda_stream

    def _geometry(self, batch: int, splits: int, pair: bool = False) -> _Geometry:
        """Schedules of one (batch bucket, split-KV factor, attention task form)."""

        key = (batch, splits, bool(pair))
        geo = self._geometries.get(key)
        if geo is not None:
            return geo
        tagged = bool(self._variant_flags & native.FLAG_PK_TAGGED)
        pair = tagged and bool(pair)
        segs = build_segments(batch, splits, self.grid, self.num_layers, self.fusion_groups, q_head_tasks=tagged,
                              pair_heads=pair)
        whole = build_schedule(batch, splits, self.grid, self.num_layers)
        errors = verify(whole)
        if errors:
            raise RuntimeError("task-graph schedule failed verification: " + "; ".join(errors[:3]))
        if tagged:
            _check_tagged_preconditions(segs)
        persistent = []
        for seg in segs:
            flat, counts = seg.persistent_words()
            inst = torch.tensor(flat, dtype=torch.int32).to(self.device)
            num = torch.tensor(counts, dtype=torch.int32).to(self.device)
            sched = native.MkdSchedule(inst=inst.data_ptr(), num_inst=num.data_ptr(), grid=seg.grid,
                                       max_inst=seg.max_inst)
            persistent.append((inst, num, sched))
        flat, table = whole.stage_words()
        stage_inst = torch.tensor(flat, dtype=torch.int32).to(self.device)
        stages = (native.MkdStage * len(table))(*[native.MkdStage(*row) for row in table])
        geo = _Geometry(batch=batch, attn_splits=splits, segments=segs, persistent=persistent,
                        stage_inst=stage_inst, stages=stages, num_stages=len(table))
        try:
            stage_scheds = (build_stage_schedules(batch, splits, self.num_layers, max_grid=self.grid, pair_heads=pair)
                            if tagged else [])
        except ValueError:
            stage_scheds = []   # a stage too large to be co-resident: the generic per-op kernels serve it
        if stage_scheds:
            for sch in stage_scheds:
                flat, counts = sch.persistent_words()
                inst = torch.tensor(flat, dtype=torch.int32).to(self.device)
                num = torch.tensor(counts, dtype=torch.int32).to(self.device)
                geo.stage_persistent.append((inst, num, native.MkdSchedule(
                    inst=inst.data_ptr(), num_inst=num.data_ptr(), grid=sch.grid, max_inst=sch.max_inst)))
            arr = (native.MkdSchedule * len(geo.stage_persistent))(*[x[2] for x in geo.stage_persistent])
            geo.stage_array = arr
        self._geometries[key] = geo
        return geo

    def _row_views(self, buf):
        """(ids int64 [8], positions int32 [8], tables int32 [8, max_pages]) views of a row buffer."""

        n = TG_MAX_BATCH
        return buf[:2 * n].view(torch.int64), buf[2 * n:3 * n], buf[3 * n:].view(n, self.max_pages)

    def check_rows(self, input_ids, positions, block_tables) -> None:
        """Host audit of one step's rows (:func:`audit_rows`). Runs on every
        host-staged step; for device tensors only when ``debug_bounds`` is set
        (reference ``taskgraph.py:419-420``)."""

        audit_rows(input_ids, positions, block_tables, block_size=self.block_size,
                   num_blocks=self.num_cache_blocks, max_model_len=self.max_model_len, max_pages=self.max_pages)

    def _audit_device_rows(self, input_ids, positions, block_tables, geo: "_Geometry") -> None:
        """``debug_bounds``: copy the rows to the host and audit them, and re-check
        the launch's schedules (verifier and tagged-kernel preconditions)."""

        self.check_rows(input_ids.tolist(), positions.tolist(), block_tables.tolist())
        errors = verify(build_schedule(geo.batch, geo.attn_splits, self.grid, self.num_layers))
        if errors:
            raise native.MegakernelError("task-graph schedule failed verification: " + "; ".join(errors[:3]))
        if self._variant_flags & native.FLAG_PK_TAGGED:
            _check_tagged_preconditions(geo.segments)

    def _stage_host_rows(self, rows: int) -> None:
        """Copy the first ``rows`` rows of the pinned mirror to the device in one copy."""

        n = 3 * TG_MAX_BATCH + rows * self.max_pages
        self._rows_dev[:n].copy_(self._rows_host[:n], non_blocking=True)

    def _desc_for(self, rows: int, geo: _Geometry, flags: int = 0, logits=None) -> native.MkdStepDesc:
        d = native.MkdStepDesc.from_buffer_copy(self._desc)
        d.rows = rows
        d.batch = geo.batch
        d.lm_slots = geo.segments[-1].lm_slots
        d.flags = flags | self._variant_flags
        d.out_logits = None if logits is None else logits.data_ptr()
        return d

    def _launch(self, desc: native.MkdStepDesc, geo: _Geometry, mode: str | None = None,
                on_segment=None) -> None:
        stream = self._stream_ptr()
        mode = mode or self.launch
        if mode == "persistent":
            for i, (inst, num, sched) in enumerate(geo.persistent):
                if self._ops is not None:
                    self._launch_op(desc, inst, num, sched)
                else:
                    native.check(self._lib.mkd_launch_persistent(native.ctypes.byref(desc),
                                                                 native.ctypes.byref(sched), stream))
                if on_segment is not None:
                    torch.cuda.current_stream(self.device).synchronize()
                    on_segment(i, geo.segments[i])
        elif mode == "stages":
            if geo.stage_array is not None:   # tagged: one persistent launch per stage
                for _, _, sched in geo.stage_persistent:
                    native.check(self._lib.mkd_launch_persistent(native.ctypes.byref(desc),
                                                                 native.ctypes.byref(sched), stream))
            else:
                native.check(self._lib.mkd_launch_stages(native.ctypes.byref(desc), geo.stage_inst.data_ptr(),
                                                         geo.stages, geo.num_stages, stream))
        else:  # graph
            if geo.graph is None or geo.graph[0] != (desc.rows, desc.flags, desc.out_logits):
                if geo.graph is not None:
                    self._lib.mkd_graph_destroy(geo.graph[1])
                geo.graph = ((desc.rows, desc.flags, desc.out_logits), self._capture(desc, geo, stream))
            native.check(self._lib.mkd_graph_launch(geo.graph[1], stream))

    def _capture(self, desc: native.MkdStepDesc, geo: _Geometry, stream: int):
        """hipGraph of one step's per-op launches: for the tagged variant the
        persistent kernel once per stage (mode 2), otherwise the generic stage
        kernels (mode 0)."""

        handle = native.ctypes.c_void_p()
        if geo.stage_array is not None:
            native.check(self._lib.mkd_graph_create(
                native.ctypes.byref(desc), 2, geo.stage_array, None, None, len(geo.stage_persistent), 1, stream,
                native.ctypes.byref(handle)))
        else:
            native.check(self._lib.mkd_graph_create(
                native.ctypes.byref(desc), 0, None, geo.stage_inst.data_ptr(), geo.stages, geo.num_stages, 1,
                stream, native.ctypes.byref(handle)))
        return handle

    def _launch_op(self, desc: native.MkdStepDesc, inst, num, sched: native.MkdSchedule) -> None:
        """One persistent launch through the registered torch operator (same
        descriptor fields as the ctypes call, passed as tensors)."""

        w = self._weights
        logits = self._op_logits if desc.out_logits else None
        self._ops.mkd_decode_step(
            self._layer_ptrs, w["embed"], w["final_norm"], w["cos"], w["sin"], self._k_cache, self._v_cache,
            self._table, self._seqlens, self._row_active, self._ids, self._op_tokens, logits,
            self._workspace, inst, num, sched.grid, sched.max_inst, desc.rows, desc.batch, desc.num_layers,
            desc.lm_slots, desc.flags, self.num_cache_blocks, self.block_size)

    def _read_status(self, rows: int) -> list[int]:
        self._host_status.copy_(self._workspace[self._status_off:self._status_off + 128].view(torch.int32),
                                non_blocking=True)
        torch.cuda.current_stream(self.device).synchronize()
        status = self._host_status
        err = int(status[0])
        if err != 0:
            native.check(self._lib.mkd_reset_counters(native.ctypes.byref(self._desc), self._stream_ptr()))
            torch.cuda.synchronize(self.device)
            kind = {1: "a dependency wait timed out", 2: "a stage kernel met a foreign instruction",
                    3: "a position, block id or token id was out of range"}.get(err, "unknown")
            raise native.MegakernelError(f"decode step failed on the device (error {err}: {kind})")
        return status[16:16 + rows].tolist()

    def pair_heads_for(self, max_context: int, batch: int = 1) -> bool:
        """Whether the tagged kernel's attention tasks of a step cover both query
        heads of a KV head: :func:`tagged_pair_heads` of the batch bucket and the
        step's longest context, or, when forced (``attn_pair_heads``), at every
        bucket whose kernel runs them."""

        if self.persistent_variant != "tagged":
            return False
        bucket = batch_bucket(batch)
        if self.attn_pair_heads is not None:
            return bool(self.attn_pair_heads) and bucket >= PAIR_HEADS_MIN_BATCH
        return tagged_pair_heads(bucket, max_context)

    def splits_for(self, max_context: int, batch: int = 1, mode: str | None = None) -> int:
        """Split-KV factor for a step. The tagged kernel (persistent, and its per-op
        launches) keeps a stage's attention tasks within one task per workgroup
        (16 // batch bucket splits, 32 // batch with tasks of both query heads, at
        most 16); the generic per-op stage kernels (lds_dma variant) need many
        workgroups per launch and keep one split per 256 positions (measured at C5,
        batch 8: 2358 us per step with 8 splits, 2692 us with 2)."""

        if self.persistent_variant == "tagged":
            bucket = batch_bucket(batch)
            pair = self.pair_heads_for(max_context, bucket)
            return tagged_attn_splits(max_context, self.min_attn_splits, bucket, pair_heads=pair)
        return auto_attn_splits(max_context, self.min_attn_splits, 1)

    def geometry_for(self, max_context: int, rows: int, mode: str | None = None) -> _Geometry:
        """The schedules a step of ``rows`` rows whose longest context is
        ``max_context`` runs: batch bucket, split-KV factor, attention task form."""

        return self._geometry(batch_bucket(rows), self.splits_for(max_context, rows, mode),
                              self.pair_heads_for(max_context, rows))

    # -- decode ----------------------------------------------------------------
    def decode_rows(self, input_ids, positions, block_tables, active_rows=None, logits=None,
                    mode: str | None = None, on_segment=None) -> list[int]:
        """One step for every row. ``input_ids``/``positions``: int64 device ``[rows]``
        (positions = pre-decode length); ``block_tables``: int32 device ``[rows, cols]``
        padded with 0. ``logits`` (optional bf16 ``[rows, vocab]``) receives the logits.
        ``on_segment(i, schedule)`` (persistent launch, diagnostics) is called after
        layer segment ``i`` has completed, with the workspace holding its outputs."""

        rows = int(input_ids.numel())
        if rows == 0:
            return []
        if rows > TG_MAX_BATCH:
            raise RuntimeError(
                f"decode_rows got {rows} rows but this decoder is sized for {TG_MAX_BATCH} (TG_MAX_BATCH); "
                "the backend's compatibility check should have rejected this batch upstream")
        cols = int(block_tables.size(1))
        if cols > self.max_pages:
            raise ValueError(
                f"block table has {cols} columns but the task-graph page_table stride is "
                f"{self.max_pages} (max_model_len // block_size)")
        geo = self.geometry_for(cols * self.block_size, rows, mode)
        if self.debug_bounds:
            self._audit_device_rows(input_ids, positions, block_tables, geo)
        self._ids[:rows].copy_(input_ids)
        self._seqlens[:rows].copy_(positions)
        self._table[:rows, :cols].copy_(block_tables)
        if active_rows is not None:
            mask = row_active_mask(active_rows, rows)
            self._row_active[:rows].copy_(torch.tensor(mask, dtype=torch.int32))
            self._mask_dirty = True
        elif self._mask_dirty:
            self._row_active.fill_(1)
            self._mask_dirty = False
        self._op_logits = logits
        self._launch(self._desc_for(rows, geo, logits=logits), geo, mode, on_segment)
        return self._read_status(rows)

    def decode_row(self, token_id: int, position: int, block_table) -> int:
        """Batch-1 step from host values (pinned staging, no per-step allocation)."""

        table = block_table.tolist() if torch.is_tensor(block_table) else list(block_table)
        cols = min(len(table), self.max_pages)
        if len(table) > self.max_pages:
            raise ValueError(f"block table has {len(table)} pages but the stride is {self.max_pages}")
        self.check_rows([token_id], [position], [table])
        self._host_ids[0] = int(token_id)
        self._host_pos[0] = int(position)
        tab = self._host_tables.numpy()
        tab[0, :cols] = table[:cols]
        tab[0, cols:] = 0
        self._stage_host_rows(1)
        if self._mask_dirty:
            self._row_active.fill_(1)
            self._mask_dirty = False
        # (the split rule sees the row's real context, known here; the block
        # table's width overstates it by up to a page)
        geo = self.geometry_for(int(position) + 1, 1)
        self._launch(self._desc_for(1, geo), geo)
        return int(self._read_status(1)[0])

    def decode_rows_host(self, input_ids: list[int], positions: list[int], block_tables: list[list[int]]) -> list[int]:
        """One step for every row from host lists (the engine's batch path). Same
        contract as :meth:`decode_rows`, but the rows are packed into pinned host
        buffers and copied without blocking, instead of being built as device
        tensors first."""

        rows = len(input_ids)
        if rows == 0:
            return []
        if rows > TG_MAX_BATCH:
            raise RuntimeError(
                f"decode_rows got {rows} rows but this decoder is sized for {TG_MAX_BATCH} (TG_MAX_BATCH); "
                "the backend's compatibility check should have rejected this batch upstream")
        if len(positions) != rows or len(block_tables) != rows:
            raise ValueError("input_ids, positions and block_tables must have one entry per row")
        cols = max(len(t) for t in block_tables)
        if cols > self.max_pages:
            raise ValueError(
                f"block table has {cols} columns but the task-graph page_table stride is "
                f"{self.max_pages} (max_model_len // block_size)")
        self.check_rows(input_ids, positions, block_tables)
        ids, pos, tab = self._host_ids.numpy(), self._host_pos.numpy(), self._host_tables.numpy()
        for r in range(rows):
            ids[r] = input_ids[r]
            pos[r] = positions[r]
            t = block_tables[r]
            tab[r, :len(t)] = t
            tab[r, len(t):] = 0
        self._stage_host_rows(rows)
        if self._mask_dirty:
            self._row_active.fill_(1)
            self._mask_dirty = False
        geo = self.geometry_for(max(int(p) for p in positions) + 1, rows)  # (real contexts, as decode_row)
        self._launch(self._desc_for(rows, geo), geo)
        return self._read_status(rows)

    def step(self, token_id: int, position: int | None = None, block_table=None) -> int:
        if position is None or block_table is None:
            raise ValueError("task-graph decode requires position and block_table")
        return self.decode_row(token_id, position, block_table)

    def step_batch(self, input_token_ids, positions, block_tables) -> list[int]:
        return self.decode_rows(input_token_ids, positions, block_tables)

    # -- device-resident loop (benchmarks) --------------------------------------
    def stage_rows(self, input_ids, positions, block_tables) -> None:
        """Load a batch into the decoder's own buffers for :meth:`run_steps`."""

        rows = int(input_ids.numel())
        cols = int(block_tables.size(1))
        self._ids[:rows].copy_(input_ids)
        self._seqlens[:rows].copy_(positions)
        self._table[:rows, :cols].copy_(block_tables)
        self._row_active.fill_(1)
        self._mask_dirty = False

    def prepare_steps(self, rows: int, max_context: int, mode: str = "persistent"):
        """Return a zero-argument callable that runs one device-resident step
        (token fed back, position advanced on the device, no host sync)."""

        geo = self.geometry_for(max_context, rows, mode)
        desc = self._desc_for(rows, geo, flags=native.FLAG_ADVANCE)
        if mode == "graph":
            handle = self._capture(desc, geo, self._stream_ptr())
            self._owned_graphs = getattr(self, "_owned_graphs", []) + [handle]
            return lambda: native.check(self._lib.mkd_graph_launch(handle, self._stream_ptr()))
        return lambda: self._launch(desc, geo, mode)

    def check_device_error(self) -> None:
        self._read_status(0)

    def tokens(self, rows: int) -> list[int]:
        return self._read_status(rows)

    def close(self) -> None:
        for geo in self._geometries.values():
            if geo.graph is not None:
                self._lib.mkd_graph_destroy(geo.graph[1])
                geo.graph = None
        for h in getattr(self, "_owned_graphs", []):
            self._lib.mkd_graph_destroy(h)
        self._owned_graphs = []
