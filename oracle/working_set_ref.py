"""CPU restatement of TideGS's resident-set materialization and writeback.

Test oracle only (see ``oracle/__init__.py``).

The reference keeps each GPU working-set buffer as six component tensors
(``GPUBuffer``, ``strategies/tide_engine/double_buffer_gpu.py:258-311``) and
moves rows with flat Triton kernels that index one value at a time
(``value offset -> row = offset // 59, column = offset % 59``).  The
functions below restate those kernels on numpy component dictionaries, value
index by value index, so the HIP mover (one table, row pitch 59 or 64) is
checked against the reference's own indexing:

* ``copy_resident_rows``  - ``_copy_resident_rows_kernel`` (double_buffer_gpu.py:41-128)
* ``fill_cold_global_ids`` - ``_fill_cold_global_ids_kernel`` (:130-149)
* ``unpack_streamed_rows`` - ``_unpack_streamed_rows_kernel`` (:151-210)
* ``component_columns``   - ``_component_columns`` (:714-735)
* ``build_block_starts`` / ``global_ids_to_local`` (:212-255)
* ``pack_resident_rows``  - ``_pack_resident_rows_kernel`` (gpu_working_set.py:33-87,
  grid of ``stage_updated_blocks`` :952-966)
* ``resident_block_bounds`` - ``_resident_block_bounds_kernel`` (gpu_working_set.py:89-116)
* ``materialize``         - the layout logic of ``_materialize_from_block_reader``
  (double_buffer_gpu.py:974-1107) and ``finalize_retained_blocks`` (:874-923)

Pinned by (tests/test_oracle_working_set.py): the known answers of the
reference's ``tests/test_double_buffer_materialization.py`` (CACHE and
UNIFIED materialization of a 14-row scene with a partial block, the resident
refresh, ``global_to_local``, the persistent-slot copy), pack/unpack round
trips against ``np.concatenate`` of the components, bounds against
``np.min``/``np.max``, and ``global_ids_to_local`` against a dictionary
lookup on random ids (negative and out-of-range ids included).
"""
from __future__ import annotations

from typing import Dict, List, Sequence

import numpy as np

NAMES = ("xyz", "scaling", "rotation", "opacity", "features_dc", "features_rest")
WIDTHS = {"xyz": 3, "scaling": 3, "rotation": 4, "opacity": 1, "features_dc": 3, "features_rest": 45}


def component_columns(layout: str) -> Dict[str, slice]:
    """Column slices of a 59-wide packed row (double_buffer_gpu.py:714-735)."""
    if layout == "unified":
        return {"xyz": slice(0, 3), "opacity": slice(3, 4), "scaling": slice(4, 7),
                "rotation": slice(7, 11), "features_dc": slice(11, 14),
                "features_rest": slice(14, 59)}
    if layout == "cache":
        return {"xyz": slice(0, 3), "scaling": slice(3, 6), "rotation": slice(6, 10),
                "opacity": slice(10, 11), "features_dc": slice(11, 14),
                "features_rest": slice(14, 59)}
    raise ValueError(f"unsupported block layout {layout!r}")


def empty_components(rows: int) -> Dict[str, np.ndarray]:
    return {n: np.zeros((rows, WIDTHS[n]), np.float32) for n in NAMES}


def components_of_table(table: np.ndarray) -> Dict[str, np.ndarray]:
    """Split a CACHE-order [M, >=59] table into the six component arrays."""
    cols = component_columns("cache")
    return {n: np.ascontiguousarray(table[:, cols[n]]) for n in NAMES}


def table_of_components(comp: Dict[str, np.ndarray]) -> np.ndarray:
    return np.concatenate([comp[n] for n in NAMES], axis=1)


# Column masks of the flat kernels (double_buffer_gpu.py:75-80): CACHE column
# range of each component.
_RANGES = {"xyz": (0, 3), "scaling": (3, 6), "rotation": (6, 10), "opacity": (10, 11),
           "features_dc": (11, 14), "features_rest": (14, 59)}


def _masks(column):
    for name in NAMES:
        lo, hi = _RANGES[name]
        m = (column >= lo) & (column < hi)
        yield name, m, column[m] - lo


def copy_resident_rows(src, src_gids, src_starts, dst_starts, num_rows, block_rows, dst, dst_gids):
    """double_buffer_gpu.py:41-128: one value per offset over num_rows*59."""
    offsets = np.arange(num_rows * 59, dtype=np.int64)
    row = offsets // 59
    column = offsets - row * 59
    block_position = row // block_rows
    row_in_block = row - block_position * block_rows
    source_row = np.asarray(src_starts, np.int64)[block_position] + row_in_block
    target_row = np.asarray(dst_starts, np.int64)[block_position] + row_in_block
    for name, m, c in _masks(column):
        dst[name][target_row[m], c] = src[name][source_row[m], c]
    first = column == 0
    dst_gids[target_row[first]] = src_gids[source_row[first]]


def fill_cold_global_ids(block_ids, dst_gids, target_offset, num_rows, block_rows):
    """double_buffer_gpu.py:130-149."""
    row = np.arange(num_rows, dtype=np.int64)
    block_position = row // block_rows
    row_in_block = row - block_position * block_rows
    dst_gids[target_offset + row] = np.asarray(block_ids, np.int64)[block_position] * block_rows + row_in_block


def unpack_streamed_rows(packed, dst, target_offset, num_rows, unified):
    """double_buffer_gpu.py:151-210 (SOURCE_UNIFIED remaps columns 3..10)."""
    offsets = np.arange(num_rows * 59, dtype=np.int64)
    row = offsets // 59
    column = offsets - row * 59
    source_column = column.copy()
    if unified:
        source_column = np.where((column >= 3) & (column < 10), column + 1, source_column)
        source_column = np.where(column == 10, 3, source_column)
    flat = np.asarray(packed, np.float32).reshape(-1)
    value = flat[row * 59 + source_column]
    target_row = target_offset + row
    for name, m, c in _masks(column):
        dst[name][target_row[m], c] = value[m]


def pack_resident_rows(src, src_starts, row_counts, out_starts, out, block_rows):
    """gpu_working_set.py:33-87 with the grid of :952-966
    (len(plans) x cdiv(block_rows*59, 256) programs of 256 values)."""
    n_values = -(-block_rows * 59 // 256) * 256
    flat = out.reshape(-1)
    for b in range(len(src_starts)):
        offsets = np.arange(n_values, dtype=np.int64)
        offsets = offsets[offsets < int(row_counts[b]) * 59]
        row = offsets // 59
        column = offsets - row * 59
        source_row = int(src_starts[b]) + row
        output_offset = (int(out_starts[b]) + row) * 59 + column
        for name, m, c in _masks(column):
            flat[output_offset[m]] = src[name][source_row[m], c]


def resident_block_bounds(xyz, starts, lengths, block_rows):
    """gpu_working_set.py:89-116: masked rows read as +-1e20."""
    out = np.zeros((len(starts), 6), np.float32)
    for b, (start, length) in enumerate(zip(starts, lengths)):
        rows = int(start) + np.arange(block_rows)
        mask = np.arange(block_rows) < int(length)
        for axis in range(3):
            lo = np.full(block_rows, 1.0e20, np.float32)
            hi = np.full(block_rows, -1.0e20, np.float32)
            lo[mask] = xyz[rows[mask], axis]
            hi[mask] = xyz[rows[mask], axis]
            out[b, axis] = lo.min()
            out[b, 3 + axis] = hi.max()
    return out


def build_block_starts(block_to_local_slice: Dict[int, slice], num_blocks: int) -> np.ndarray:
    """double_buffer_gpu.py:212-233."""
    starts = np.full(num_blocks, -1, np.int64)
    for block_id, sl in block_to_local_slice.items():
        if 0 <= int(block_id) < num_blocks:
            starts[int(block_id)] = int(sl.start)
    return starts


def global_ids_to_local(global_ids, block_starts, block_size):
    """double_buffer_gpu.py:236-255 (floor division, -1 when unloaded)."""
    g = np.asarray(global_ids, np.int64)
    num_blocks = block_starts.shape[0]
    block_ids = np.floor_divide(g, block_size)
    within = g - block_ids * block_size
    safe = np.clip(block_ids, 0, num_blocks - 1)
    starts = block_starts[safe]
    invalid = (block_ids != safe) | (starts < 0)
    local = starts + within
    local[invalid] = -1
    return local


class BufferRef:
    """The parts of GPUBuffer (double_buffer_gpu.py:258-311) the moves touch."""

    def __init__(self):
        self.comp: Dict[str, np.ndarray] | None = None
        self.gids: np.ndarray | None = None
        self.block_to_local_slice: Dict[int, slice] = {}
        self.loaded_blocks: List[int] = []
        self.resident_blocks: List[int] = []
        self.streamed_blocks: List[int] = []
        self.evicted_blocks: List[int] = []
        self.num_gaussians = 0
        self.block_starts: np.ndarray | None = None


def copy_resident_blocks(source: BufferRef, target: BufferRef, block_ids: Sequence[int],
                         target_slices: Dict[int, slice], block_rows: int) -> int:
    """double_buffer_gpu.py:811-872 (the Triton branch)."""
    if not block_ids:
        return 0
    num_rows = sum(target_slices[b].stop - target_slices[b].start for b in block_ids)
    src_starts = [source.block_to_local_slice[b].start for b in block_ids]
    dst_starts = [target_slices[b].start for b in block_ids]
    copy_resident_rows(source.comp, source.gids, src_starts, dst_starts, num_rows, block_rows,
                       target.comp, target.gids)
    return num_rows


def materialize(source: BufferRef | None, sorted_visible_blocks: Sequence[int], resident_set,
                evicted_set, allow_resident_copy: bool, read_blocks, layout: str,
                num_total: int, block_rows: int, defer_resident_copy: bool = False) -> BufferRef:
    """double_buffer_gpu.py:974-1107 with a reader returning {block: [len,59]}."""
    num_blocks = -(-num_total // block_rows)
    visible = set(int(b) for b in sorted_visible_blocks)
    resident_blocks = sorted(
        b for b in visible & set(resident_set)
        if allow_resident_copy and source is not None and source.comp is not None
        and b in source.block_to_local_slice)
    streamed_blocks = sorted(visible - set(resident_blocks))
    target_order = resident_blocks + streamed_blocks
    lengths = {b: min(block_rows, num_total - b * block_rows) for b in target_order}
    invalid = [b for b, n in lengths.items() if n <= 0]
    if invalid:
        raise ValueError(f"Invalid block IDs during N+1 materialization: {invalid}")
    target = BufferRef()
    offset = 0
    for b in target_order:
        target.block_to_local_slice[b] = slice(offset, offset + lengths[b])
        offset += lengths[b]
    target.comp = empty_components(offset)
    target.gids = np.zeros(offset, np.int64)
    resident_rows = sum(lengths[b] for b in resident_blocks)
    if not defer_resident_copy:
        copy_resident_blocks(source, target, resident_blocks, target.block_to_local_slice,
                             block_rows)
    streamed_rows = 0
    if streamed_blocks:
        blocks = read_blocks(streamed_blocks)
        packed = np.concatenate([np.asarray(blocks[b], np.float32)[:lengths[b]]
                                 for b in streamed_blocks], axis=0)
        streamed_rows = packed.shape[0]
        unpack_streamed_rows(packed, target.comp, resident_rows, streamed_rows, layout == "unified")
        fill_cold_global_ids(streamed_blocks, target.gids, resident_rows, streamed_rows, block_rows)
    target.loaded_blocks = target_order
    target.num_gaussians = resident_rows + streamed_rows
    target.resident_blocks = resident_blocks
    target.streamed_blocks = streamed_blocks
    target.evicted_blocks = sorted(evicted_set)
    target.block_starts = build_block_starts(target.block_to_local_slice, num_blocks)
    return target


def stage_updated_blocks(buffer: BufferRef, updated_block_ids, num_total: int, block_rows: int):
    """gpu_working_set.py:895-988: (plans, packed [rows,59] CACHE order)."""
    plans, local_starts = [], []
    for b in sorted(set(int(x) for x in updated_block_ids)):
        sl = buffer.block_to_local_slice.get(b)
        if sl is None:
            continue
        expected = min(block_rows, num_total - b * block_rows)
        count = min(expected, sl.stop - sl.start)
        if count <= 0:
            continue
        plans.append((b, count))
        local_starts.append(sl.start)
    if not plans:
        return None
    counts = [c for _, c in plans]
    out_starts = np.cumsum([0] + counts[:-1])
    out = np.zeros((sum(counts), 59), np.float32)
    pack_resident_rows(buffer.comp, local_starts, counts, out_starts, out, block_rows)
    return plans, out


def stage_block_bounds(buffer: BufferRef, block_ids, num_total: int, block_rows: int):
    """gpu_working_set.py:990-1062: (block ids, bounds [n,6])."""
    plans = []
    for b in sorted(set(int(x) for x in block_ids)):
        sl = buffer.block_to_local_slice.get(b)
        if sl is None:
            continue
        count = min(min(block_rows, num_total - b * block_rows), sl.stop - sl.start)
        if count > 0:
            plans.append((b, sl.start, count))
    if not plans:
        return None
    bounds = resident_block_bounds(buffer.comp["xyz"], [p[1] for p in plans],
                                   [p[2] for p in plans], block_rows)
    return [p[0] for p in plans], bounds


def finalize_retained_blocks(source: BufferRef, target: BufferRef, block_ids,
                             block_rows: int) -> int:
    """double_buffer_gpu.py:874-923 (non-persistent path): refresh the rows of
    blocks loaded in both buffers from the active one; returns blocks copied."""
    refresh = sorted(int(b) for b in set(block_ids)
                     if int(b) in source.block_to_local_slice
                     and int(b) in target.block_to_local_slice)
    copy_resident_blocks(source, target, refresh, target.block_to_local_slice, block_rows)
    return len(refresh)
