"""Resident-block Adam / Sophia for the TideGS working set (drop-in).

``GPUResidentAdam`` serves the call sites of
``strategies/tide_engine/gpu_resident_optimizer.py:73-513`` (constructed and
stepped from ``runtime.py:1732-1791``) with the same behaviour:

* moments exist only for resident blocks; every resident block owns a state
  slot with its own step counter and bias correction (``:302-337``);
* eviction discards the slot's moments, re-admission cold-starts them
  (``:219-264``);
* gradients are divided by the batch size; ``step()`` returns the same stats
  dictionaries and ``get_stats()`` the same keys.

The design differs.  The host side is one :class:`SlotTable` of parallel
numpy arrays (owner block, step count, warm flag, row count per slot; the
resident blocks sorted with their slot and residency streak), so admission,
eviction and the per-step slot update are a handful of vectorised operations
whatever the number of blocks.  The device side is ONE launch for all 59
columns (``tgs_resident_adam_step``) with the row -> slot lookup done on the
GPU, and moments stored as ``[slots * block_size, 64]`` tables in the
resident table's column order (a touched row's state is one 256-byte span of
two whole cache lines).  The per-slot bias terms are uploaded whole from a
pinned staging table; two staging tables alternate and each waits for its
previous copy before it is rewritten, so back-to-back steps without a host
synchronisation cannot race an upload.

``GPUResidentSophia`` keeps the same slots with a diagonal-Hessian EMA in
place of the second moment (Liu et al. 2023; no TideGS counterpart).
"""
from __future__ import annotations

import copy
import ctypes
from typing import Any, Callable, Dict, Optional, Sequence, Tuple

import numpy as np
import torch

from . import _native as N

# First column of each learning-rate group in TideGS's unified column order
# (xyz 0-2, opacity 3, scaling 4-6, rotation 7-10, dc 11-13, rest 14-58), used
# to read a 59-entry expanded ``columns_lr``.
_GROUP_FIRST_COLUMN = np.array([0, 3, 4, 7, 11, 14])
# logical state per row: two moments of 59 fp32 values
_STATE_BYTES_PER_ROW = 59 * 2 * 4
# state column of each component: the resident table's CACHE order
# (storage/block_reader.py:35-44), shared by the [N,59] table and its gradient
# rows, so that runs of rows stream as flat spans
_STATE_COLUMNS = {"xyz": 0, "scaling": 3, "rotation": 6, "opacity": 10, "features_dc": 11,
                  "features_rest": 14}


def component_learning_rates(columns_lr, specs) -> Dict[str, float]:
    """Learning rate of each component from ``optimizer.columns_lr``: six
    grouped values, or 59 per-column values of which each group's first
    column is taken (``gaussian_model.py:721-728`` builds them)."""
    if columns_lr is None:
        raise RuntimeError("[GPUResidentAdam] the optimizer carries no columns_lr")
    if torch.is_tensor(columns_lr):
        columns_lr = columns_lr.detach().to("cpu", torch.float32).numpy()
    lr = np.asarray(columns_lr, dtype=np.float32).reshape(-1)
    if lr.size == 59:
        lr = lr[_GROUP_FIRST_COLUMN]
    elif lr.size != 6:
        raise RuntimeError(
            f"[GPUResidentAdam] columns_lr holds {lr.size} values: give 6 (one per parameter "
            "group) or 59 (one per column)")
    return {name: float(lr[group]) for name, _, _, group in specs}


class SlotTable:
    """Host bookkeeping of the optimizer's state slots.

    Per slot: ``owner`` (block id, -1 when free), ``steps`` (updates since the
    block's admission), ``warm`` (moments initialised by a step since
    admission) and ``rows`` (the block's row count when it was first touched).
    Per resident block, sorted by id: ``blocks``, ``block_slot`` and
    ``streak`` (consecutive resident sets that held it).  Free slots are
    handed out lowest first."""

    def __init__(self):
        self.owner = np.empty(0, np.int64)
        self.steps = np.empty(0, np.int64)
        self.warm = np.empty(0, bool)
        self.rows = np.empty(0, np.int64)
        self.blocks = np.empty(0, np.int64)
        self.block_slot = np.empty(0, np.int64)
        self.streak = np.empty(0, np.int64)
        self.ended_streak_sum = 0    # streaks of blocks that have left the set
        self.ended_streak_count = 0
        self.evicted_warm = 0        # slots discarded with initialised moments

    @property
    def capacity(self) -> int:
        return int(self.owner.size)

    def add_slots(self, n: int) -> None:
        self.owner = np.concatenate([self.owner, np.full(n, -1, np.int64)])
        self.steps = np.concatenate([self.steps, np.zeros(n, np.int64)])
        self.warm = np.concatenate([self.warm, np.zeros(n, bool)])
        self.rows = np.concatenate([self.rows, np.zeros(n, np.int64)])

    def _reset(self, slots: np.ndarray, owner) -> None:
        self.owner[slots] = owner
        self.steps[slots] = 0
        self.warm[slots] = False
        self.rows[slots] = 0

    def retarget(self, wanted: Sequence[int], reserve: Callable[[int], None]) -> np.ndarray:
        """Make ``wanted`` the resident set: release the slots of blocks that
        leave (closing their streaks), extend the streaks of blocks that stay,
        give arriving blocks (ascending) the lowest free slots after
        ``reserve(len(wanted))`` has grown the table if needed.  Returns the
        arriving blocks' slots (their moments must be cleared)."""
        new = np.unique(np.fromiter((int(b) for b in wanted), dtype=np.int64))
        stays = np.isin(self.blocks, new, assume_unique=True)
        leaving = self.block_slot[~stays]
        ended = self.streak[~stays]
        self.ended_streak_sum += int(ended.sum())
        self.ended_streak_count += int(np.count_nonzero(ended))
        self.evicted_warm += int(np.count_nonzero(self.warm[leaving]))
        self._reset(leaving, -1)
        kept = self.blocks[stays]
        arriving = np.setdiff1d(new, kept, assume_unique=True)
        reserve(int(new.size))
        slots = np.flatnonzero(self.owner < 0)[: arriving.size]
        self._reset(slots, arriving)
        merged = np.concatenate([kept, arriving])
        order = np.argsort(merged, kind="stable")
        self.blocks = merged[order]
        self.block_slot = np.concatenate([self.block_slot[stays], slots])[order]
        self.streak = np.concatenate([self.streak[stays] + 1,
                                      np.ones(arriving.size, np.int64)])[order]
        return slots

    def slots_of(self, block_ids: np.ndarray) -> np.ndarray:
        """Slot of each block id, -1 where the block is not resident."""
        block_ids = np.asarray(block_ids, np.int64)
        if self.blocks.size == 0:
            return np.full(block_ids.shape, -1, np.int64)
        pos = np.minimum(np.searchsorted(self.blocks, block_ids), self.blocks.size - 1)
        return np.where(self.blocks[pos] == block_ids, self.block_slot[pos], -1)

    def advance(self, slots: np.ndarray, block_rows: np.ndarray,
                touched: np.ndarray) -> Tuple[int, int]:
        """One update of ``slots`` (distinct), whose blocks hold ``block_rows``
        rows of which ``touched`` were updated: warm the cold ones (recording
        their row counts), count the step.  Returns (cold slots, their touched
        rows)."""
        cold = ~self.warm[slots]
        cold_slots = slots[cold]
        self.warm[cold_slots] = True
        self.rows[cold_slots] = block_rows[cold]
        self.steps[slots] += 1
        return int(cold_slots.size), int(touched[cold].sum())

    def live_state(self) -> Tuple[int, int]:
        """(blocks with initialised moments, their logical state bytes)."""
        return int(np.count_nonzero(self.warm)), int(self.rows[self.warm].sum()) * \
            _STATE_BYTES_PER_ROW

    def mean_streak(self) -> float:
        total = self.ended_streak_sum + int(self.streak.sum())
        count = self.ended_streak_count + int(self.streak.size)
        return float(total) / max(1, count)


class _Layout:
    """The working set's blocks in row order: ``[start, stop)`` slices, block
    ids and state slots as numpy arrays plus the device copies the kernels
    read (starts, ends, slots as int64)."""

    def __init__(self, manager, table: SlotTable, device):
        ids, starts, stops = [], [], []
        for b in manager.loaded_blocks:
            sl = manager.block_to_gpu_slice.get(int(b))
            if sl is not None:
                ids.append(int(b))
                starts.append(int(sl.start))
                stops.append(int(sl.stop))
        if not ids:
            raise RuntimeError("[GPUResidentAdam] the working set holds no blocks to update")
        order = np.argsort(np.asarray(starts, np.int64), kind="stable")
        self.block_ids = np.asarray(ids, np.int64)[order]
        self.starts = np.asarray(starts, np.int64)[order]
        self.stops = np.asarray(stops, np.int64)[order]
        self.slots = table.slots_of(self.block_ids)
        missing = self.block_ids[self.slots < 0]
        if missing.size:
            raise RuntimeError(
                f"[GPUResidentAdam] block {int(missing[0])} is loaded but was never made "
                "resident (set_resident_blocks), so it has no state slot")
        dev = torch.from_numpy(np.stack([self.starts, self.stops, self.slots])).to(device)
        self.d_starts, self.d_stops, self.d_slots = dev[0], dev[1], dev[2]

    def __len__(self) -> int:
        return int(self.block_ids.size)


class GPUResidentAdam:
    """Adam with moments stored only for the current resident block set."""

    # (component, attribute on the Gaussians, width, learning-rate group):
    # the reference optimizer's component table, which callers index
    COMPONENT_SPECS = (
        ("xyz", "_xyz", 3, 0),
        ("opacity", "_opacity", 1, 1),
        ("scaling", "_scaling", 3, 2),
        ("rotation", "_rotation", 4, 3),
        ("features_dc", "_features_dc", 3, 4),
        ("features_rest", "_features_rest", 45, 5),
    )
    TOTAL_WIDTH = sum(spec[2] for spec in COMPONENT_SPECS)
    # moment table row pitch: 64 floats = two whole 128-byte lines per row
    STATE_PITCH = 64
    _STATE_COLS = _STATE_COLUMNS
    # kernel component order = state column order
    _LAUNCH_ORDER = tuple(sorted(COMPONENT_SPECS, key=lambda spec: _STATE_COLUMNS[spec[0]]))
    # learning-rate order of tgs_tide_project_bwd_update (CACHE column groups)
    _FUSED_LR_ORDER = ("xyz", "scaling", "rotation", "opacity", "features_dc", "features_rest")

    def __init__(self, batch_size: int = 1, block_size: int = 4096, capacity_blocks: int = 0,
                 device: str = "cuda"):
        self.batch_size = int(batch_size)
        self.block_size = int(block_size)
        self.capacity_blocks = max(0, int(capacity_blocks))
        self.device = torch.device(device)
        self.state_mode = "resident_blocks"
        self.kernel_hooks = None  # optional (before, after) callables around the launch
        self.slots = SlotTable()
        self._epoch = 0            # bumps on every set_resident_blocks
        self._layout_key = None
        self._layout_cached: Optional[_Layout] = None
        self._exp_avg: Optional[torch.Tensor] = None     # [slots*block, 64]
        self._exp_avg_sq: Optional[torch.Tensor] = None  # [slots*block, 64]
        # per-slot bias terms [2, slots] (1 - b1^t, sqrt(1 - b2^t)): host values,
        # their device copy, and two pinned staging tables for the uploads,
        # each with the event of its last copy
        self._bias_host = np.zeros((2, 0), np.float32)
        self._bias_terms: Optional[torch.Tensor] = None
        self._staging = []
        self._staging_turn = 0
        self._counts_dev: Optional[torch.Tensor] = None
        self._counts_host: Optional[torch.Tensor] = None
        self._fused_lrs = None
        self._error_flag = torch.zeros(1, dtype=torch.int32, device=self.device)
        self._counters = {"cold_restarts": 0, "optimizer_rows_touched_total": 0,
                          "cold_restarted_rows_touched_total": 0}

    # ---- state storage -------------------------------------------------------
    @property
    def _allocated_slots(self) -> int:
        return self.slots.capacity

    def _reserve(self, required: int) -> None:
        """Grow to hold ``required`` slots: to max(required, capacity_blocks,
        twice the current size), keeping every existing slot's contents."""
        have = self.slots.capacity
        if required <= have:
            return
        target = max(required, self.capacity_blocks, 2 * have, 1)
        rows = target * self.block_size
        grown = []
        for old in (self._exp_avg, self._exp_avg_sq):
            t = torch.empty((rows, self.STATE_PITCH), dtype=torch.float32, device=self.device)
            if old is not None:
                t[: old.shape[0]].copy_(old)
            grown.append(t)
        self._exp_avg, self._exp_avg_sq = grown
        for _, event in self._staging:  # no upload may still read the old tables
            if event is not None:
                event.synchronize()
        self._bias_host = np.concatenate(
            [self._bias_host, np.zeros((2, target - have), np.float32)], axis=1)
        self._bias_terms = torch.from_numpy(self._bias_host).to(self.device)
        pin = self.device.type == "cuda"
        self._staging = [[torch.empty((2, target), dtype=torch.float32, pin_memory=pin), None]
                         for _ in range(2)]
        self.slots.add_slots(target - have)

    def _clear_moments(self, slots: np.ndarray) -> None:
        """Zero both moment tables over the given slots, one fill per run of
        consecutive slots (a fill kernel, no memset nodes)."""
        if slots.size == 0:
            return
        slots = np.unique(slots)
        breaks = np.flatnonzero(np.diff(slots) != 1) + 1
        words = self.block_size * self.STATE_PITCH
        stream = N.stream_handle(self.device)
        for run in np.split(slots, breaks):
            first, count = int(run[0]), int(run.size)
            for table in (self._exp_avg, self._exp_avg_sq):
                N.call("tgs_fill_u32", table.data_ptr() + 4 * first * words, count * words, 0,
                       stream)

    def _upload_bias_terms(self, slots: np.ndarray, beta1: float, beta2: float) -> None:
        """Refresh the bias terms of ``slots`` from their step counts
        (``1 - b1^t``, ``sqrt(1 - b2^t)`` in float64, stored as float32) and
        queue the whole table's upload from the staging table whose previous
        copy has finished."""
        t = self.slots.steps[slots].astype(np.float64)
        self._bias_host[0, slots] = 1.0 - beta1 ** t
        self._bias_host[1, slots] = np.sqrt(1.0 - beta2 ** t)
        turn = self._staging[self._staging_turn]
        self._staging_turn ^= 1
        if turn[1] is not None:
            turn[1].synchronize()
        turn[0].numpy()[:] = self._bias_host
        self._bias_terms.copy_(turn[0], non_blocking=True)
        if self.device.type == "cuda":
            turn[1] = torch.cuda.Event()
            turn[1].record(torch.cuda.current_stream(self.device))

    # ---- resident set --------------------------------------------------------
    def set_resident_blocks(self, block_ids) -> None:
        """Make ``block_ids`` the resident set (``gpu_resident_optimizer.py:219-264``
        behaviour): leaving blocks lose their moments, arriving blocks start
        cold in freshly cleared slots."""
        arriving = self.slots.retarget(block_ids, self._reserve)
        self._clear_moments(arriving)
        self._epoch += 1

    def slot_of(self, block_id: int) -> int:
        """State slot of a resident block (-1 if it is not resident)."""
        return int(self.slots.slots_of(np.array([block_id]))[0])

    def _layout(self, manager) -> _Layout:
        """The block layout, rebuilt when the resident set, the working-set
        manager, its block count or its ``layout_version`` changes."""
        key = (self._epoch, id(manager), id(manager.block_to_gpu_slice),
               len(manager.block_to_gpu_slice), len(manager.loaded_blocks),
               getattr(manager, "layout_version", None))
        if key != self._layout_key:
            self._layout_cached = _Layout(manager, self.slots, self.device)
            self._layout_key = key
        return self._layout_cached

    # ---- per-step bookkeeping --------------------------------------------------
    @staticmethod
    def _hyper(gaussians) -> Tuple[float, float, float]:
        group = gaussians.optimizer.param_groups[0]
        beta1, beta2 = group["betas"]
        return float(beta1), float(beta2), float(group["eps"])

    def _count_touches(self, layout: _Layout, rows: torch.Tensor) -> torch.Tensor:
        """Queue the per-layout-block count of ``rows`` (ascending) on the
        device stream and its copy into pinned host memory; the host tensor is
        valid after the stream's next synchronisation."""
        n = len(layout)
        if self._counts_dev is None or self._counts_dev.numel() < n:
            size = max(n, 64)
            self._counts_dev = torch.empty(size, dtype=torch.int64, device=self.device)
            self._counts_host = torch.empty(size, dtype=torch.int64,
                                            pin_memory=self.device.type == "cuda")
        N.call("tgs_block_touch_counts", rows.numel(), N.ptr(rows),
               1 if rows.dtype == torch.int64 else 0, N.ptr(layout.d_starts),
               N.ptr(layout.d_stops), n, N.ptr(self._counts_dev), N.stream_handle(self.device))
        host = self._counts_host[:n]
        host.copy_(self._counts_dev[:n], non_blocking=True)
        return host

    def _apply_counts(self, layout: _Layout, counts: np.ndarray, n_rows: int, beta1: float,
                      beta2: float) -> Dict[str, Any]:
        """Advance the slots of the touched blocks and refresh their bias
        terms (``gpu_resident_optimizer.py:302-337`` behaviour); returns the
        step's stats dictionary."""
        if counts.shape[0] != len(layout) or int(counts.sum()) != int(n_rows):
            raise RuntimeError(
                "[GPUResidentAdam] a touched row lies outside every resident block of the layout")
        hit = np.flatnonzero(counts > 0)
        slots = layout.slots[hit]
        cold_slots, cold_rows = self.slots.advance(
            slots, layout.stops[hit] - layout.starts[hit], counts[hit])
        if slots.size:
            self._upload_bias_terms(slots, beta1, beta2)
        self._counters["cold_restarts"] += cold_slots
        self._counters["cold_restarted_rows_touched_total"] += cold_rows
        self._counters["optimizer_rows_touched_total"] += int(n_rows)
        return {"updated_blocks": int(hit.size),
                "updated_block_ids": layout.block_ids[hit].tolist(),
                "touched_rows": int(n_rows),
                "cold_rows": int(cold_rows)}

    # ---- stand-alone update -------------------------------------------------
    @staticmethod
    def _row_view(t: torch.Tensor, width: int, name: str) -> Tuple[int, int]:
        """(pointer, row stride) of a [rows, width] tensor with unit column stride."""
        if t.dim() == 1 and width == 1:
            if t.stride(0) != 1:
                raise RuntimeError(f"[GPUResidentAdam] {name} must have unit stride")
            return t.data_ptr(), 1
        if t.dim() != 2 or t.shape[1] != width or (t.shape[0] > 1 and t.stride(1) != 1):
            raise RuntimeError(
                f"[GPUResidentAdam] {name}: parameters and gradients must be [rows, {width}] "
                f"with contiguous rows (got shape {tuple(t.shape)}, stride {t.stride()})")
        return t.data_ptr(), max(t.stride(0), width)

    def _component_tables(self, gaussians, grads):
        """ctypes arrays of the launch: parameter, gradient and moment pointers,
        widths, row strides (param, grad, state) and learning rates."""
        lrs_by_name = component_learning_rates(getattr(gaussians.optimizer, "columns_lr", None),
                                               self.COMPONENT_SPECS)
        n = len(self._LAUNCH_ORDER)
        ptrs = [(ctypes.c_void_p * n)() for _ in range(4)]
        widths = (ctypes.c_int32 * n)()
        strides = (ctypes.c_int64 * (3 * n))()
        lrs = (ctypes.c_float * n)()
        for k, (name, attr, width, _) in enumerate(self._LAUNCH_ORDER):
            if name not in grads:
                raise KeyError(f"[GPUResidentAdam] no gradient for component {name!r}")
            pp, ps = self._row_view(getattr(gaussians, attr).data, width, name)
            gp, gs = self._row_view(grads[name], width, name)
            col = 4 * self._STATE_COLS[name]
            ptrs[0][k], ptrs[1][k] = pp, gp
            ptrs[2][k] = self._exp_avg.data_ptr() + col
            ptrs[3][k] = self._exp_avg_sq.data_ptr() + col
            widths[k] = width
            strides[3 * k:3 * k + 3] = [ps, gs, self.STATE_PITCH]
            lrs[k] = lrs_by_name[name]
        return ptrs, widths, strides, lrs

    def _kernel_args(self, gaussians, grads, beta1, beta2, eps, iteration):
        ptrs, widths, strides, lrs = self._component_tables(gaussians, grads)
        head = (N.ptr(self._bias_terms[0]), N.ptr(self._bias_terms[1]))
        tail = (beta1, beta2, eps, float(self.batch_size))
        return "tgs_resident_adam_step", head, (len(self._LAUNCH_ORDER), *ptrs, widths, strides,
                                                 lrs), tail

    def step(self, iteration: int, gaussians, sparse_grad_local_ids: torch.Tensor,
             sparse_grad_components: Dict[str, torch.Tensor]) -> Dict[str, Any]:
        """Update the touched rows (ascending, unique local ids) with their
        gradient rows; returns ``{"updated_blocks", "updated_block_ids",
        "touched_rows", "cold_rows"}``."""
        if (sparse_grad_local_ids is None or sparse_grad_components is None
                or sparse_grad_local_ids.numel() == 0):
            return {"updated_blocks": 0, "updated_block_ids": [], "touched_rows": 0,
                    "cold_rows": 0}
        manager = getattr(gaussians, "gpu_working_set_manager", None)
        if manager is None or manager.local_to_global_idx is None:
            raise RuntimeError(
                "[GPUResidentAdam] the Gaussians carry no gpu_working_set_manager "
                "(with local_to_global_idx)")
        rows = sparse_grad_local_ids.to(self.device)
        if rows.dtype not in (torch.int32, torch.int64):
            rows = rows.to(torch.int64)
        rows = rows.contiguous()
        layout = self._layout(manager)
        beta1, beta2, eps = self._hyper(gaussians)
        kernel, head, comps, tail = self._kernel_args(gaussians, sparse_grad_components, beta1,
                                                      beta2, eps, iteration)
        counts = self._count_touches(layout, rows)
        torch.cuda.current_stream(self.device).synchronize()
        stats = self._apply_counts(layout, counts.numpy(), rows.numel(), beta1, beta2)
        hooks = self.kernel_hooks
        if hooks:
            hooks[0]()
        N.call(kernel, rows.numel(), N.ptr(rows), 1 if rows.dtype == torch.int64 else 0,
               N.ptr(layout.d_starts), N.ptr(layout.d_stops), N.ptr(layout.d_slots), len(layout),
               self.block_size, *head, *comps, *tail, N.ptr(self._error_flag),
               N.stream_handle(self.device))
        if hooks:
            hooks[1]()
        return stats

    # ---- update fused into the gradient launch ------------------------------
    # A caller that computes the touched rows' gradients on the GPU applies the
    # update inside that launch (tgs_tide_project_bwd_update) instead of
    # materialising the gradient rows: launch_touch_counts() once the touched
    # rows exist, fused_update_args() before the fused launch.
    def _fused_mode(self, iteration: int) -> Tuple[int, float, int]:
        """(optimizer id, rho, update_hessian) of tgs_tide_project_bwd_update."""
        return 0, 0.0, 1

    def launch_touch_counts(self, gaussians, local_rows: torch.Tensor) -> torch.Tensor:
        """Per-block touched-row counts of ``local_rows`` (ascending, unique),
        computed on the device stream and copied to pinned host memory without
        waiting; valid after the caller's next synchronisation."""
        if local_rows.dtype not in (torch.int32, torch.int64):
            raise RuntimeError("[GPUResidentAdam] touched rows must be int32 or int64")
        layout = self._layout(gaussians.gpu_working_set_manager)
        return self._count_touches(layout, local_rows.contiguous())

    def fused_update_args(self, iteration: int, gaussians, n_rows: int,
                          counts_host: torch.Tensor) -> Tuple[tuple, Dict[str, Any]]:
        """Advance the touched slots (as step() does) and return the optimizer
        arguments of tgs_tide_project_bwd_update (``block_starts`` through
        ``error_flag``) with step()'s stats dictionary."""
        layout = self._layout(gaussians.gpu_working_set_manager)
        lrs_by_name = component_learning_rates(getattr(gaussians.optimizer, "columns_lr", None),
                                               self.COMPONENT_SPECS)
        beta1, beta2, eps = self._hyper(gaussians)
        stats = self._apply_counts(layout, counts_host.numpy(), n_rows, beta1, beta2)
        mode, rho, update_h = self._fused_mode(iteration)
        self._fused_lrs = (ctypes.c_float * 6)(*[lrs_by_name[k] for k in self._FUSED_LR_ORDER])
        args = (N.ptr(layout.d_starts), N.ptr(layout.d_stops), N.ptr(layout.d_slots),
                len(layout), self.block_size, N.ptr(self._bias_terms[0]),
                N.ptr(self._bias_terms[1]), N.ptr(self._exp_avg), N.ptr(self._exp_avg_sq),
                self.STATE_PITCH, self._fused_lrs, mode, beta1, beta2, eps,
                float(self.batch_size), rho, update_h, N.ptr(self._error_flag))
        return args, stats

    # ---- snapshot / restore ----------------------------------------------------
    def snapshot(self) -> Dict[str, Any]:
        """A copy of the whole optimizer state (moment tables on the device,
        slot bookkeeping, bias terms and counters on the host), for
        :meth:`restore`.  The resident set must not change in between."""
        torch.cuda.current_stream(self.device).synchronize()
        return {"exp_avg": None if self._exp_avg is None else self._exp_avg.clone(),
                "exp_avg_sq": None if self._exp_avg_sq is None else self._exp_avg_sq.clone(),
                "bias_host": self._bias_host.copy(), "slots": copy.deepcopy(self.slots),
                "counters": dict(self._counters), "epoch": self._epoch}

    def restore(self, snap: Dict[str, Any]) -> None:
        """Put back a :meth:`snapshot` in place (device copies queued on the
        current stream; the tables keep their addresses)."""
        if snap["epoch"] != self._epoch or snap["slots"].capacity != self.slots.capacity:
            raise RuntimeError("[GPUResidentAdam] restore: the resident set changed since the "
                               "snapshot")
        for table, saved in ((self._exp_avg, snap["exp_avg"]),
                             (self._exp_avg_sq, snap["exp_avg_sq"])):
            if saved is not None:
                table.copy_(saved)
        for _, event in self._staging:  # no queued upload may still read the host table
            if event is not None:
                event.synchronize()
        self._bias_host[...] = snap["bias_host"]
        self._bias_terms.copy_(torch.from_numpy(self._bias_host))
        self.slots = copy.deepcopy(snap["slots"])
        self._counters = dict(snap["counters"])

    # ---- stats ----------------------------------------------------------------
    def get_stats(self) -> Dict[str, Any]:
        """The reference's stats keys; also raises if a launch flagged a row
        outside every resident block."""
        if int(self._error_flag.item()) != 0:
            raise RuntimeError(
                "[GPUResidentAdam] a touched row lies outside every resident block of the layout")
        live_blocks, live_bytes = self.slots.live_state()
        return {
            "state_mode": self.state_mode,
            "resident_target_blocks": int(self.slots.blocks.size),
            "resident_state_blocks": live_blocks,
            "resident_state_bytes": live_bytes,
            "allocated_state_bytes": self.slots.capacity * self.block_size *
            self.STATE_PITCH * 2 * 4,
            "cold_restarts": self._counters["cold_restarts"],
            "state_evictions": self.slots.evicted_warm,
            "optimizer_rows_touched_total": self._counters["optimizer_rows_touched_total"],
            "cold_restarted_rows_touched_total":
                self._counters["cold_restarted_rows_touched_total"],
            "mean_resident_streak": self.slots.mean_streak(),
        }


class GPUResidentSophia(GPUResidentAdam):
    """Sophia-style update on the same resident slots (second moment -> Hessian EMA).

    ``m = b1 m + (1-b1) g``; every ``hessian_interval`` iterations
    ``h = b2 h + (1-b2) g*g``; ``p -= lr * clamp(m / max(h, eps), -rho, rho)``.
    ``g`` is the gradient divided by the batch size, as in GPUResidentAdam.
    """

    def __init__(self, batch_size: int = 1, block_size: int = 4096, capacity_blocks: int = 0,
                 device: str = "cuda", rho: float = 0.04, hessian_interval: int = 1):
        super().__init__(batch_size, block_size, capacity_blocks, device)
        self.rho = float(rho)
        self.hessian_interval = max(1, int(hessian_interval))

    def _update_hessian(self, iteration: int) -> int:
        return 1 if int(iteration) % self.hessian_interval == 0 else 0

    def _fused_mode(self, iteration: int) -> Tuple[int, float, int]:
        return 1, self.rho, self._update_hessian(iteration)

    def _kernel_args(self, gaussians, grads, beta1, beta2, eps, iteration):
        ptrs, widths, strides, lrs = self._component_tables(gaussians, grads)
        tail = (beta1, beta2, eps, self.rho, float(self.batch_size),
                self._update_hessian(iteration))
        return "tgs_resident_sophia_step", (), (len(self._LAUNCH_ORDER), *ptrs, widths, strides,
                                                 lrs), tail
