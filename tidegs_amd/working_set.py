"""Resident working set on the GPU: materialization and writeback (drop-in).

TideGS keeps each GPU working-set buffer as six component tensors
(``GPUBuffer``, ``strategies/tide_engine/double_buffer_gpu.py:258-311``) and
moves rows between them with Triton kernels.  Here a buffer is ONE fp32 table
in CACHE column order (xyz | scaling | rotation | opacity | dc | rest) with a
row pitch of 64 floats by default (every row one 256-byte line; 59 = dense),
the same table ``TideStep`` and ``GPUResidentAdam`` consume, plus the int64
local->global id of every row.  The component tensors of the reference are
column views of it (``ResidentBuffer.xyz`` ...).

``ResidentWorkingSet`` holds the GPU side of ``DoubleBufferGPUWorkingSet`` and
``GPUWorkingSetManager``:

* ``materialize``              - ``_materialize_from_block_reader`` (double_buffer_gpu.py:974-1107)
* ``copy_resident_blocks``     - ``_copy_resident_blocks`` (:811-872)
* ``finalize_retained_blocks`` - the resident refresh of :874-923
* ``fill_streamed_global_ids`` - ``_fill_streamed_global_ids`` (:928-963)
* ``stage_updated_blocks``     - dirty-row packing + one D2H copy (gpu_working_set.py:895-988)
* ``stage_block_bounds``       - per-block xyz bounds + one D2H copy (gpu_working_set.py:990-1062)
* ``build_block_starts`` / ``global_to_local`` (double_buffer_gpu.py:212-255, :479-492)

Every row move is one launch of the native mover (``tgs_ws_*`` in
``include/tidegs_amd.h``) on the caller's current stream; there is no CPU
path.  The host keeps only the block bookkeeping, as the reference does.
The N+1 prefetch threads, host caches and storage I/O around these calls
stay with the caller.
"""
from __future__ import annotations

import enum
import threading
from dataclasses import dataclass, field
from typing import Dict, List, Optional, Sequence

import torch

from . import _native as N

CACHE_COLUMNS = {"xyz": slice(0, 3), "scaling": slice(3, 6), "rotation": slice(6, 10),
                 "opacity": slice(10, 11), "features_dc": slice(11, 14),
                 "features_rest": slice(14, 59)}
ROW_PITCH = 64


class BlockLayout(enum.Enum):
    """Column order of a 59-wide packed block (storage/block_reader.py:30-44)."""

    UNIFIED = "unified"  # xyz | opacity | scaling | rotation | dc | rest
    CACHE = "cache"      # xyz | scaling | rotation | opacity | dc | rest


def _layout_code(layout) -> int:
    value = getattr(layout, "value", layout)
    if value == "cache":
        return 0
    if value == "unified":
        return 1
    raise ValueError(f"Unsupported block layout: {layout!r}")


def allocate_table(rows: int, device, pitch: int = ROW_PITCH) -> torch.Tensor:
    """A [rows, 59] fp32 view of [rows, pitch] storage (pitch 59 or 64)."""
    if pitch not in (59, 64):
        raise ValueError("row pitch must be 59 or 64")
    storage = torch.empty((rows, pitch), dtype=torch.float32, device=device)
    return storage[:, :59]


def table_pitch(table: torch.Tensor) -> int:
    if table.dim() != 2 or table.shape[1] != 59 or table.stride(1) != 1 \
            or table.stride(0) not in (59, 64) or table.dtype != torch.float32:
        raise ValueError("a resident table is a [M,59] fp32 view with row pitch 59 or 64")
    return int(table.stride(0))


@dataclass
class ResidentBuffer:
    """One working-set buffer (the GPUBuffer of double_buffer_gpu.py:258-311)."""

    table: Optional[torch.Tensor] = None             # [M,59], CACHE order
    local_to_global_idx: Optional[torch.Tensor] = None  # [M] int64
    _block_starts: Optional[torch.Tensor] = None
    loaded_blocks: List[int] = field(default_factory=list)
    num_gaussians: int = 0
    filters_local: List[torch.Tensor] = field(default_factory=list)
    block_to_local_slice: Dict[int, slice] = field(default_factory=dict)
    resident_blocks: List[int] = field(default_factory=list)
    streamed_blocks: List[int] = field(default_factory=list)
    evicted_blocks: List[int] = field(default_factory=list)

    def _col(self, name):
        return None if self.table is None else self.table[:, CACHE_COLUMNS[name]]

    xyz = property(lambda self: self._col("xyz"))
    scaling = property(lambda self: self._col("scaling"))
    rotation = property(lambda self: self._col("rotation"))
    opacity = property(lambda self: self._col("opacity"))
    features_dc = property(lambda self: self._col("features_dc"))
    features_rest = property(lambda self: self._col("features_rest"))

    def is_empty(self) -> bool:
        return self.table is None

    def clear(self) -> None:
        self.table = None
        self.local_to_global_idx = None
        self._block_starts = None
        self.loaded_blocks = []
        self.filters_local = []
        self.block_to_local_slice = {}
        self.resident_blocks = []
        self.streamed_blocks = []
        self.evicted_blocks = []
        self.num_gaussians = 0


@dataclass(frozen=True)
class ResidentHandoffResult:
    """Outcome of making retained blocks ready (double_buffer_gpu.py:314-319)."""

    ready_blocks: int
    copied_blocks: int


@dataclass
class PendingBlockWriteback:
    """Packed dirty rows and their (block id, row count) plans; ``wait()``
    returns the host copy once the D2H copy has landed."""

    plans: List[tuple]
    packed_gpu: torch.Tensor
    packed_cpu: Optional[torch.Tensor]
    ready_event: Optional[torch.cuda.Event]

    def wait(self):
        if self.ready_event is not None:
            self.ready_event.synchronize()
        return self.plans, self.packed_cpu


@dataclass
class PendingBlockBounds:
    """Per-block bounds [n,6] (min xyz, max xyz) awaiting one D2H copy
    (gpu_working_set.py:119-133)."""

    block_ids: List[int]
    cpu_bounds: Optional[torch.Tensor]
    ready_event: Optional[torch.cuda.Event]
    gpu_bounds: Optional[torch.Tensor] = None

    def wait(self):
        if self.ready_event is not None:
            self.ready_event.synchronize()
        return self.block_ids, self.cpu_bounds


def _i64(device, *columns) -> torch.Tensor:
    """Index arrays of equal length as one [k, n] int64 device tensor, uploaded
    with one asynchronous copy from pinned memory (row i = columns[i])."""
    cols = [list(c) for c in columns]
    host = torch.empty((len(cols), len(cols[0])), dtype=torch.int64, pin_memory=True)
    for i, c in enumerate(cols):
        host[i] = torch.as_tensor(c, dtype=torch.int64)
    return host.to(device, non_blocking=True)


class ResidentWorkingSet:
    """GPU materialization / writeback of resident blocks of ``block_size`` rows
    out of ``num_total_gaussians`` (block b holds global rows
    ``b*block_size .. min((b+1)*block_size, N)``)."""

    def __init__(self, num_total_gaussians: int, block_size: int = 4096, device="cuda",
                 row_pitch: int = ROW_PITCH):
        if row_pitch not in (59, 64):
            raise ValueError("row_pitch must be 59 or 64")
        if block_size <= 0 or num_total_gaussians < 0:
            raise ValueError("block_size must be > 0 and num_total_gaussians >= 0")
        self.num_total = int(num_total_gaussians)
        self.block_size = int(block_size)
        self.num_blocks = -(-self.num_total // self.block_size)
        self.device = torch.device(device)
        self.row_pitch = row_pitch
        self._staging_lock = threading.Lock()
        self._host_staging: Optional[torch.Tensor] = None
        self._host_staging_event: Optional[torch.cuda.Event] = None
        self.stats = {"batched_materializations": 0, "batched_h2d_calls": 0,
                      "batched_resident_blocks": 0, "batched_streamed_blocks": 0,
                      "resident_refresh_blocks": 0, "batched_writebacks": 0,
                      "batched_writeback_rows": 0, "bounds_updates": 0}

    # ------------------------------------------------------------------ helpers
    def block_length(self, block_id: int) -> int:
        return min(self.block_size, self.num_total - int(block_id) * self.block_size)

    def allocate(self, target: ResidentBuffer, num_rows: int) -> None:
        """Fresh table and id storage (_allocate_target_tensors, :737-749)."""
        target.table = allocate_table(num_rows, self.device, self.row_pitch)
        target.local_to_global_idx = torch.empty(num_rows, dtype=torch.int64, device=self.device)

    def _stream(self):
        return N.stream_handle(self.device)

    # ------------------------------------------------------------- row moves
    def copy_resident_blocks(self, source: ResidentBuffer, target: ResidentBuffer,
                             block_ids: Sequence[int], target_slices: Dict[int, slice]) -> int:
        """Copy whole kept blocks, ids included (double_buffer_gpu.py:811-872)."""
        if not block_ids:
            return 0
        num_rows = sum(target_slices[b].stop - target_slices[b].start for b in block_ids)
        src_starts, dst_starts = _i64(self.device,
                                      (source.block_to_local_slice[b].start for b in block_ids),
                                      (target_slices[b].start for b in block_ids))
        N.call("tgs_ws_copy_rows", N.ptr(source.table), table_pitch(source.table),
               N.ptr(source.local_to_global_idx), N.ptr(src_starts), N.ptr(dst_starts),
               len(block_ids), num_rows, self.block_size, N.ptr(target.table),
               table_pitch(target.table), N.ptr(target.local_to_global_idx), self._stream())
        return num_rows

    def fill_streamed_global_ids(self, target: ResidentBuffer, block_ids: Sequence[int],
                                 target_offset: int, num_rows: int) -> None:
        """Ids of streamed (cold) rows (double_buffer_gpu.py:928-963)."""
        if not block_ids:
            return
        ids = _i64(self.device, block_ids)[0]
        N.call("tgs_ws_fill_global_ids", N.ptr(ids), len(block_ids),
               N.ptr(target.local_to_global_idx), target_offset, num_rows, self.block_size,
               self._stream())

    def unpack_streamed_rows(self, packed_gpu: torch.Tensor, layout, target: ResidentBuffer,
                             target_offset: int, block_ids: Optional[Sequence[int]] = None) -> None:
        """Unpack [rows,59] CACHE/UNIFIED rows into the table from target_offset
        (double_buffer_gpu.py:1060-1082); with ``block_ids`` the cold ids are
        written in the same pass."""
        N.require_cuda(packed_gpu, names=["packed_gpu"])
        if packed_gpu.dim() != 2 or packed_gpu.shape[1] != 59 or packed_gpu.dtype != torch.float32:
            raise ValueError(f"packed rows must be fp32 [rows,59], got {tuple(packed_gpu.shape)}")
        rows = int(packed_gpu.shape[0])
        if target_offset + rows > target.table.shape[0]:
            raise ValueError("streamed rows overrun the target table")
        ids = None
        if block_ids is not None:
            ids = _i64(self.device, block_ids)[0]
            if -(-rows // self.block_size) > len(block_ids):
                raise ValueError("fewer block ids than streamed blocks")
        N.call("tgs_ws_unpack_rows", N.ptr(packed_gpu), _layout_code(layout), rows,
               N.ptr(target.table), table_pitch(target.table), target_offset, N.ptr(ids),
               0 if ids is None else len(block_ids), self.block_size,
               None if ids is None else N.ptr(target.local_to_global_idx), self._stream())

    # ----------------------------------------------------------- lookups
    def build_block_starts(self, block_to_local_slice: Dict[int, slice]) -> torch.Tensor:
        """[num_blocks] int64, local start of each loaded block or -1 (:212-233)."""
        out = torch.empty(max(self.num_blocks, 1), dtype=torch.int64, device=self.device)
        items = [(int(b), int(s.start)) for b, s in block_to_local_slice.items()]
        ids = starts = None
        if items:
            ids, starts = _i64(self.device, (b for b, _ in items), (s for _, s in items))
        N.call("tgs_ws_build_block_starts", N.ptr(ids), N.ptr(starts), len(items), N.ptr(out),
               out.shape[0], self._stream())
        return out[:self.num_blocks]

    def global_to_local(self, buffer: ResidentBuffer, global_ids: torch.Tensor) -> torch.Tensor:
        """Working-set-local index of each global id, -1 when its block is not
        loaded (double_buffer_gpu.py:479-492, :236-255)."""
        if buffer._block_starts is None:
            raise RuntimeError("global_to_local called before the block-start table was built")
        g = global_ids.to(device=self.device, dtype=torch.int64).contiguous()
        out = torch.empty_like(g)
        if self.num_blocks == 0:
            return out.fill_(-1)
        N.call("tgs_ws_global_to_local", N.ptr(g), g.numel(), N.ptr(buffer._block_starts),
               self.num_blocks, self.block_size, N.ptr(out), self._stream())
        return out

    # ------------------------------------------------------ materialization
    def _host_rows(self, rows: int) -> torch.Tensor:
        with self._staging_lock:
            if self._host_staging_event is not None:
                self._host_staging_event.synchronize()
            if self._host_staging is None or self._host_staging.shape[0] < rows:
                self._host_staging = torch.empty((max(rows, 1), 59), dtype=torch.float32,
                                                 pin_memory=True)
            return self._host_staging[:rows]

    def _read_streamed(self, block_reader, streamed_blocks, block_lengths, rows):
        """Packed CPU rows of the streamed blocks in order (:1010-1057)."""
        staging = self._host_rows(rows)
        read_batch = getattr(block_reader, "read_batch", None)
        if callable(read_batch):
            batch = read_batch(streamed_blocks, out=staging)
            packed = batch.tensor
            if tuple(packed.shape) != (rows, 59):
                raise ValueError(f"Invalid N+1 block batch shape {tuple(packed.shape)}; "
                                 f"expected {(rows, 59)}")
            for b in streamed_blocks:
                sl = batch.block_slices.get(b)
                if sl is None or sl.stop - sl.start != block_lengths[b]:
                    raise ValueError(f"Invalid N+1 batch slice for block {b}: got={sl}, "
                                     f"expected_rows={block_lengths[b]}")
            return packed
        blocks = block_reader.read_blocks(streamed_blocks)
        missing = [b for b in streamed_blocks if b not in blocks]
        if missing:
            raise KeyError(f"BlockReader omitted {len(missing)} N+1 blocks; "
                           f"first missing={missing[:8]}")
        offset = 0
        for b in streamed_blocks:
            n = block_lengths[b]
            staging[offset:offset + n].copy_(blocks[b][:n])
            offset += n
        return staging

    def materialize(self, source: Optional[ResidentBuffer], sorted_visible_blocks: Sequence[int],
                    resident_set, evicted_set=(), allow_resident_copy: bool = True,
                    block_reader=None, defer_resident_copy: bool = False,
                    target: Optional[ResidentBuffer] = None) -> ResidentBuffer:
        """Build the next working set: kept resident blocks first (copied from
        ``source``), then the streamed blocks in ascending id order, read from
        ``block_reader`` (``.layout`` and ``read_batch``/``read_blocks`` of
        storage/block_reader.py), uploaded once and unpacked on the GPU
        (double_buffer_gpu.py:974-1107)."""
        target = target if target is not None else ResidentBuffer()
        visible = set(int(b) for b in sorted_visible_blocks)
        resident_blocks = sorted(
            b for b in visible & set(int(x) for x in resident_set)
            if allow_resident_copy and source is not None and not source.is_empty()
            and b in source.block_to_local_slice)
        streamed_blocks = sorted(visible - set(resident_blocks))
        target_order = resident_blocks + streamed_blocks
        lengths = {b: self.block_length(b) for b in target_order}
        invalid = [b for b, n in lengths.items() if n <= 0]
        if invalid:
            raise ValueError(f"Invalid block IDs during N+1 materialization: {invalid}")
        target.block_to_local_slice = {}
        offset = 0
        for b in target_order:
            target.block_to_local_slice[b] = slice(offset, offset + lengths[b])
            offset += lengths[b]
        self.allocate(target, offset)
        resident_rows = sum(lengths[b] for b in resident_blocks)
        if not defer_resident_copy:
            self.copy_resident_blocks(source, target, resident_blocks, target.block_to_local_slice)
        streamed_rows = 0
        if streamed_blocks:
            if block_reader is None:
                raise ValueError("streamed blocks need a block_reader")
            streamed_rows = sum(lengths[b] for b in streamed_blocks)
            packed_cpu = self._read_streamed(block_reader, streamed_blocks, lengths, streamed_rows)
            packed_gpu = torch.empty((streamed_rows, 59), dtype=torch.float32, device=self.device)
            packed_gpu.copy_(packed_cpu, non_blocking=packed_cpu.is_pinned())
            if packed_cpu.is_pinned():
                ev = torch.cuda.Event()
                ev.record(torch.cuda.current_stream(self.device))
                self._host_staging_event = ev
            self.unpack_streamed_rows(packed_gpu, block_reader.layout, target, resident_rows,
                                      block_ids=streamed_blocks)
            self.stats["batched_h2d_calls"] += 1
        target.loaded_blocks = target_order
        target.num_gaussians = resident_rows + streamed_rows
        target.resident_blocks = resident_blocks
        target.streamed_blocks = streamed_blocks
        target.evicted_blocks = sorted(int(b) for b in evicted_set)
        target._block_starts = self.build_block_starts(target.block_to_local_slice)
        self.stats["batched_materializations"] += 1
        self.stats["batched_resident_blocks"] += len(resident_blocks)
        self.stats["batched_streamed_blocks"] += len(streamed_blocks)
        return target

    def finalize_retained_blocks(self, source: ResidentBuffer, target: ResidentBuffer,
                                 block_ids: Sequence[int]) -> ResidentHandoffResult:
        """Refresh retained blocks of ``target`` from the (since updated)
        ``source`` (double_buffer_gpu.py:874-923, non-persistent path)."""
        if source.is_empty() or target.is_empty() or not block_ids:
            return ResidentHandoffResult(0, 0)
        refresh = sorted(int(b) for b in set(block_ids)
                         if int(b) in source.block_to_local_slice
                         and int(b) in target.block_to_local_slice)
        if not refresh:
            return ResidentHandoffResult(0, 0)
        self.copy_resident_blocks(source, target, refresh, target.block_to_local_slice)
        self.stats["resident_refresh_blocks"] += len(refresh)
        return ResidentHandoffResult(len(refresh), len(refresh))

    # ------------------------------------------------------------ writeback
    def _plans(self, buffer: ResidentBuffer, block_ids):
        plans = []
        for b in sorted(set(int(x) for x in block_ids)):
            sl = buffer.block_to_local_slice.get(b)
            if sl is None:
                continue
            count = min(self.block_length(b), int(sl.stop - sl.start))
            if count > 0:
                plans.append((b, int(sl.start), count))
        return plans

    def stage_updated_blocks(self, buffer: ResidentBuffer, updated_block_ids,
                             to_host: bool = True) -> Optional[PendingBlockWriteback]:
        """Pack the rows of updated blocks into one [rows,59] CACHE-order
        array and (``to_host``) start one D2H copy into pinned memory
        (gpu_working_set.py:895-988)."""
        if buffer.is_empty() or not updated_block_ids:
            return None
        plans = self._plans(buffer, updated_block_ids)
        if not plans:
            return None
        counts = [c for _, _, c in plans]
        total = sum(counts)
        out_starts, acc = [], 0
        for c in counts:
            out_starts.append(acc)
            acc += c
        packed_gpu = torch.empty((total, 59), dtype=torch.float32, device=self.device)
        src_starts, row_counts, out_st = _i64(self.device, (s for _, s, _ in plans), counts,
                                              out_starts)
        N.call("tgs_ws_pack_rows", N.ptr(buffer.table), table_pitch(buffer.table),
               N.ptr(src_starts), N.ptr(row_counts), N.ptr(out_st), len(plans), self.block_size,
               N.ptr(packed_gpu), self._stream())
        packed_cpu, ev = None, None
        if to_host:
            packed_cpu = torch.empty((total, 59), dtype=torch.float32, pin_memory=True)
            packed_cpu.copy_(packed_gpu, non_blocking=True)
            ev = torch.cuda.Event()
            ev.record(torch.cuda.current_stream(self.device))
        self.stats["batched_writebacks"] += 1
        self.stats["batched_writeback_rows"] += total
        return PendingBlockWriteback([(b, c) for b, _, c in plans], packed_gpu, packed_cpu, ev)

    def stage_block_bounds(self, buffer: ResidentBuffer, block_ids,
                           to_host: bool = True) -> Optional[PendingBlockBounds]:
        """Per-block xyz min/max of the listed loaded blocks
        (gpu_working_set.py:990-1062)."""
        if buffer.is_empty() or not block_ids:
            return None
        plans = self._plans(buffer, block_ids)
        if not plans:
            return None
        starts, lengths = _i64(self.device, (s for _, s, _ in plans), (c for _, _, c in plans))
        bounds = torch.empty((len(plans), 6), dtype=torch.float32, device=self.device)
        N.call("tgs_ws_block_bounds", N.ptr(buffer.table), table_pitch(buffer.table),
               N.ptr(starts), N.ptr(lengths), len(plans), self.block_size, N.ptr(bounds),
               self._stream())
        cpu, ev = None, None
        if to_host:
            cpu = torch.empty((len(plans), 6), dtype=torch.float32, pin_memory=True)
            cpu.copy_(bounds, non_blocking=True)
            ev = torch.cuda.Event()
            ev.record(torch.cuda.current_stream(self.device))
        self.stats["bounds_updates"] += len(plans)
        return PendingBlockBounds([b for b, _, _ in plans], cpu, ev, bounds)

    def get_stats(self) -> dict:
        return dict(self.stats)
