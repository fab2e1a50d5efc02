"""Resident-block Adam / Sophia for the TideGS working set (drop-in).

``GPUResidentAdam`` mirrors ``strategies/tide_engine/gpu_resident_optimizer.py:73-513``:
moments exist only for resident blocks, each resident block owns a state slot
with its own step counter and bias correction (``:302-337``), eviction discards
the slot and re-admission cold-starts it (``:219-264``), gradients are divided by
the batch size, and ``step()`` returns the same stats dicts.  The host keeps
that bookkeeping; the update of all 59 columns runs as ONE HIP launch
(``tgs_resident_adam_step``) instead of six Triton launches, with the
row -> slot mapping resolved on the GPU.

Moments live in one ``[slots * block_size, 64]`` array per moment (59 columns
in the resident table's CACHE order plus 5 padding columns), so a touched
row's state is one 256-byte span of two whole cache lines.

``GPUResidentSophia`` uses the same slots with a diagonal-Hessian EMA instead of
the second moment (Liu et al. 2023; no TideGS counterpart, see the kernel).
"""
from __future__ import annotations

import ctypes
import math
from typing import Any, Dict, List, Optional, Tuple

import numpy as np
import torch

from . import _native as N


class GPUResidentAdam:
    """Adam with moments stored only for the current resident block set."""

    COMPONENT_SPECS = (
        ("xyz", "_xyz", 3, 0),
        ("opacity", "_opacity", 1, 1),
        ("scaling", "_scaling", 3, 2),
        ("rotation", "_rotation", 4, 3),
        ("features_dc", "_features_dc", 3, 4),
        ("features_rest", "_features_rest", 45, 5),
    )
    TOTAL_WIDTH = sum(spec[2] for spec in COMPONENT_SPECS)
    # Row pitch of the moment tables: 64 floats, so that every state row is two
    # whole 128-byte lines (a 59-float row straddles three lines, and the
    # partial lines cost a read-modify-write on every update).
    STATE_PITCH = 64
    # Column offsets of each component inside the unified state rows: the
    # resident table's CACHE column order (storage/block_reader.py:35-44), so
    # that a [N,59] parameter table, its [T,59] gradient rows and the state rows
    # share one column layout (the kernel then streams runs of rows as flat
    # spans).  The state layout is internal to this class.
    _STATE_COLS = {"xyz": 0, "scaling": 3, "rotation": 6, "opacity": 10, "features_dc": 11,
                   "features_rest": 14}
    # components in state-column order (the kernel's component order)
    _order = []
    for _spec in COMPONENT_SPECS:
        _order.append((_STATE_COLS[_spec[0]], _spec))
    _order.sort()
    _LAUNCH_ORDER = tuple(_item[1] for _item in _order)
    del _order, _spec

    def __init__(self, batch_size: int = 1, block_size: int = 4096, capacity_blocks: int = 0,
                 device: str = "cuda"):
        self.batch_size = int(batch_size)
        self.block_size = int(block_size)
        self.capacity_blocks = max(0, int(capacity_blocks))
        self.device = torch.device(device)
        self.state_mode = "resident_blocks"

        self._resident_blocks = set()
        self._resident_streaks: Dict[int, int] = {}
        self._completed_streak_total = 0
        self._completed_streak_count = 0

        self._allocated_slots = 0
        self._block_to_slot: Dict[int, int] = {}
        self._slot_to_block: List[Optional[int]] = []
        self._free_slots: List[int] = []
        # per state slot (numpy, so that a step updates all touched slots at once)
        self._slot_steps = np.zeros(0, dtype=np.int64)
        self._slot_initialized = np.zeros(0, dtype=bool)
        self._slot_row_counts = np.zeros(0, dtype=np.int64)
        self._layout_key = None   # cached block layout (see _layout_tables)
        self._layout_cached = None
        self._resident_epoch = 0
        self._exp_avg: Optional[torch.Tensor] = None     # [slots*block, STATE_PITCH]
        self._exp_avg_sq: Optional[torch.Tensor] = None  # [slots*block, STATE_PITCH]
        self._bias_correction1: Optional[torch.Tensor] = None
        self._denom_scale: Optional[torch.Tensor] = None
        self._error_flag = torch.zeros(1, dtype=torch.int32, device=self.device)

        self._logical_state_blocks = 0
        self._logical_state_bytes = 0
        self._stats = {
            "state_mode": "resident_blocks",
            "resident_target_blocks": 0,
            "resident_state_blocks": 0,
            "resident_state_bytes": 0,
            "allocated_state_bytes": 0,
            "cold_restarts": 0,
            "state_evictions": 0,
            "optimizer_rows_touched_total": 0,
            "cold_restarted_rows_touched_total": 0,
            "mean_resident_streak": 0.0,
        }

    # ---- bookkeeping (host) -------------------------------------------------
    def _physical_state_bytes(self) -> int:
        return int(self._allocated_slots * self.block_size * self.STATE_PITCH * 2 * 4)

    def _update_state_stats(self) -> None:
        self._stats["resident_target_blocks"] = len(self._resident_blocks)
        self._stats["resident_state_blocks"] = int(self._logical_state_blocks)
        self._stats["resident_state_bytes"] = int(self._logical_state_bytes)
        self._stats["allocated_state_bytes"] = self._physical_state_bytes()
        streak_total = self._completed_streak_total + sum(self._resident_streaks.values())
        streak_count = self._completed_streak_count + len(self._resident_streaks)
        self._stats["mean_resident_streak"] = float(streak_total) / max(1, streak_count)

    def _normalize_columns_lr(self, columns_lr) -> Dict[str, float]:
        if columns_lr is None:
            raise RuntimeError("[GPUResidentAdam] optimizer.columns_lr is required")
        if torch.is_tensor(columns_lr):
            cols = columns_lr.detach().to(device="cpu", dtype=torch.float32)
        else:
            cols = torch.tensor(columns_lr, dtype=torch.float32)
        cols = cols.flatten().contiguous()
        if cols.numel() == 6:
            grouped = cols
        elif cols.numel() == 59:
            grouped = cols[torch.tensor([0, 3, 4, 7, 11, 14])]
        else:
            raise RuntimeError(
                f"[GPUResidentAdam] Unexpected columns_lr width={cols.numel()}; "
                "expected 6 grouped or 59 expanded entries"
            )
        return {name: float(grouped[g].item()) for name, _, _, g in self.COMPONENT_SPECS}

    def _ensure_storage(self, required_slots: int) -> None:
        if required_slots <= self._allocated_slots:
            return
        target = max(required_slots, self.capacity_blocks, max(1, self._allocated_slots * 2))
        old_slots = self._allocated_slots
        old_rows = old_slots * self.block_size
        new_rows = target * self.block_size
        avg = torch.empty((new_rows, self.STATE_PITCH), dtype=torch.float32, device=self.device)
        avg_sq = torch.empty_like(avg)
        if old_rows:
            avg[:old_rows].copy_(self._exp_avg)
            avg_sq[:old_rows].copy_(self._exp_avg_sq)
        bias = torch.empty((target,), dtype=torch.float32, device=self.device)
        denom = torch.empty((target,), dtype=torch.float32, device=self.device)
        if old_slots:
            bias[:old_slots].copy_(self._bias_correction1)
            denom[:old_slots].copy_(self._denom_scale)
        self._exp_avg, self._exp_avg_sq = avg, avg_sq
        self._bias_correction1, self._denom_scale = bias, denom
        self._slot_to_block.extend([None] * (target - old_slots))
        grow = target - old_slots
        self._slot_steps = np.concatenate([self._slot_steps, np.zeros(grow, dtype=np.int64)])
        self._slot_initialized = np.concatenate([self._slot_initialized, np.zeros(grow, dtype=bool)])
        self._slot_row_counts = np.concatenate([self._slot_row_counts,
                                                np.zeros(grow, dtype=np.int64)])
        # host mirrors of the bias tables (the source of truth, uploaded whole
        # after each step's update), pinned for asynchronous copies
        pin = self.device.type == "cuda"
        bias_host = torch.zeros(target, dtype=torch.float32, pin_memory=pin)
        denom_host = torch.zeros(target, dtype=torch.float32, pin_memory=pin)
        if old_slots:
            bias_host[:old_slots].copy_(self._bias_host[:old_slots])
            denom_host[:old_slots].copy_(self._denom_host[:old_slots])
        self._bias_host, self._denom_host = bias_host, denom_host
        self._free_slots.extend(range(target - 1, old_slots - 1, -1))
        self._allocated_slots = target

    def _clear_slots(self, slots: List[int]) -> None:
        """Zero the moments of the given slots: one fill per run of consecutive slots."""
        row_words = self.block_size * self.STATE_PITCH
        s = N.stream_handle(self.device)
        ordered = sorted(set(int(x) for x in slots))
        i = 0
        while i < len(ordered):
            j = i
            while j + 1 < len(ordered) and ordered[j + 1] == ordered[j] + 1:
                j += 1
            first, count = ordered[i], j - i + 1
            for buf in (self._exp_avg, self._exp_avg_sq):
                N.call("tgs_fill_u32", buf.data_ptr() + first * row_words * 4, count * row_words, 0,
                       s)
            i = j + 1

    def set_resident_blocks(self, block_ids: List[int]) -> None:
        next_resident = {int(b) for b in block_ids}
        previous = set(self._resident_blocks)
        evicted = previous - next_resident
        kept = previous & next_resident
        incoming = next_resident - previous

        for block_id in evicted:
            streak = int(self._resident_streaks.pop(block_id, 0))
            if streak > 0:
                self._completed_streak_total += streak
                self._completed_streak_count += 1
            slot = self._block_to_slot.pop(block_id)
            if self._slot_initialized[slot]:
                self._stats["state_evictions"] += 1
                self._logical_state_blocks -= 1
                self._logical_state_bytes -= int(self._slot_row_counts[slot]) * self.TOTAL_WIDTH * 2 * 4
            self._slot_to_block[slot] = None
            self._slot_steps[slot] = 0
            self._slot_initialized[slot] = False
            self._slot_row_counts[slot] = 0
            self._free_slots.append(slot)

        for block_id in kept:
            self._resident_streaks[block_id] = self._resident_streaks.get(block_id, 0) + 1
        for block_id in incoming:
            self._resident_streaks[block_id] = 1

        self._ensure_storage(len(next_resident))
        incoming_slots: List[int] = []
        for block_id in sorted(incoming):
            if not self._free_slots:
                self._ensure_storage(self._allocated_slots + 1)
            slot = self._free_slots.pop()
            self._block_to_slot[block_id] = slot
            self._slot_to_block[slot] = block_id
            self._slot_steps[slot] = 0
            self._slot_initialized[slot] = False
            self._slot_row_counts[slot] = 0
            incoming_slots.append(slot)
        self._clear_slots(incoming_slots)
        self._resident_blocks = next_resident
        self._resident_epoch += 1
        self._update_state_stats()

    def _layout(self, manager) -> List[Tuple[int, int, int, int]]:
        layout = []
        for block_id in manager.loaded_blocks:
            block_id = int(block_id)
            block_slice = manager.block_to_gpu_slice.get(block_id)
            if block_slice is None:
                continue
            slot = self._block_to_slot.get(block_id)
            if slot is None:
                raise RuntimeError(
                    f"[GPUResidentAdam] loaded block {block_id} has no resident state slot")
            layout.append((int(block_slice.start), int(block_slice.stop), block_id, slot))
        layout.sort(key=lambda item: item[0])
        if not layout:
            raise RuntimeError("[GPUResidentAdam] working set contains no resident blocks")
        return layout

    def _layout_tables(self, manager):
        """The sorted block layout (the reference's per-step searchsorted table,
        gpu_resident_optimizer.py:266-300) with its device copies.  Rebuilt when
        the resident set changes (set_resident_blocks) or the working-set
        manager, its block count or its ``layout_version`` (if it has one) does."""
        key = (self._resident_epoch, id(manager), id(manager.block_to_gpu_slice),
               len(manager.block_to_gpu_slice), len(manager.loaded_blocks),
               getattr(manager, "layout_version", None))
        if key != self._layout_key:
            layout = self._layout(manager)
            arr = np.array(layout, dtype=np.int64).reshape(-1, 4)
            table = torch.from_numpy(np.ascontiguousarray(arr[:, [0, 1, 3]].T)).to(self.device)
            self._layout_cached = (layout, arr, table[0], table[1], table[2])
            self._layout_key = key
        return self._layout_cached

    def _touched_counts(self, n_layout, starts, ends, local_rows, index_is_i64) -> np.ndarray:
        counts = torch.empty(n_layout, dtype=torch.int64, device=self.device)
        N.call("tgs_block_touch_counts", local_rows.numel(), N.ptr(local_rows), index_is_i64,
               N.ptr(starts), N.ptr(ends), n_layout, N.ptr(counts), N.stream_handle(self.device))
        return counts.cpu().numpy()

    def _update_touched_slot_metadata(self, arr: np.ndarray, counts: np.ndarray, beta1: float,
                                      beta2: float):
        """Advance the step of every slot with touched rows and refresh its bias
        terms (gpu_resident_optimizer.py:302-337); returns (touched layout rows,
        cold rows)."""
        hit = np.nonzero(counts > 0)[0]
        slots = arr[hit, 3]
        cold = ~self._slot_initialized[slots]
        cold_slots = slots[cold]
        cold_rows = int(counts[hit][cold].sum())
        if cold_slots.size:
            row_counts = arr[hit, 1][cold] - arr[hit, 0][cold]
            self._slot_initialized[cold_slots] = True
            self._slot_row_counts[cold_slots] = row_counts
            self._logical_state_blocks += int(cold_slots.size)
            self._logical_state_bytes += int(row_counts.sum()) * self.TOTAL_WIDTH * 2 * 4
            self._stats["cold_restarts"] += int(cold_slots.size)
            self._stats["cold_restarted_rows_touched_total"] += cold_rows
        if slots.size:
            self._slot_steps[slots] += 1
            steps = self._slot_steps[slots].astype(np.float64)
            bias = self._bias_host.numpy()
            denom = self._denom_host.numpy()
            bias[slots] = 1.0 - beta1 ** steps
            denom[slots] = np.sqrt(1.0 - beta2 ** steps)
            n = self._allocated_slots
            self._bias_correction1.copy_(self._bias_host[:n], non_blocking=True)
            self._denom_scale.copy_(self._denom_host[:n], non_blocking=True)
        return hit, cold_rows

    # ---- fused update --------------------------------------------------------
    @staticmethod
    def _row_view(t: torch.Tensor, width: int, name: str) -> Tuple[int, int]:
        """(pointer, row stride) of a [rows, width] tensor with unit column stride."""
        if t.dim() == 1 and width == 1:
            if t.stride(0) != 1:
                raise RuntimeError(f"[GPUResidentAdam] {name} must have unit stride")
            return t.data_ptr(), 1
        if t.dim() != 2 or t.shape[1] != width or (t.shape[0] > 1 and t.stride(1) != 1):
            raise RuntimeError(
                f"[GPUResidentAdam] {name} parameter and gradient must be contiguous "
                f"[rows, {width}] rows (got shape {tuple(t.shape)}, stride {t.stride()})")
        return t.data_ptr(), max(t.stride(0), width)

    def _launch(self, kernel: str, n_rows, local_rows, index_is_i64, starts, ends, slots,
                n_layout, param_views, grads, component_lrs, extra_args):
        n = len(self._LAUNCH_ORDER)
        params_p = (ctypes.c_void_p * n)()
        grads_p = (ctypes.c_void_p * n)()
        m_p = (ctypes.c_void_p * n)()
        v_p = (ctypes.c_void_p * n)()
        widths = (ctypes.c_int32 * n)()
        strides = (ctypes.c_int64 * (3 * n))()
        lrs = (ctypes.c_float * n)()
        for k, (name, _, width, _) in enumerate(self._LAUNCH_ORDER):
            pp, ps = self._row_view(param_views[name], width, name)
            gp, gs = self._row_view(grads[name], width, name)
            col = self._STATE_COLS[name]
            params_p[k], grads_p[k] = pp, gp
            m_p[k] = self._exp_avg.data_ptr() + 4 * col
            v_p[k] = self._exp_avg_sq.data_ptr() + 4 * col
            widths[k] = width
            strides[3 * k + 0], strides[3 * k + 1], strides[3 * k + 2] = ps, gs, self.STATE_PITCH
            lrs[k] = component_lrs[name]
        hooks = getattr(self, "kernel_hooks", None)
        if hooks:
            hooks[0]()
        if kernel == "tgs_resident_adam_step":
            args = (n_rows, N.ptr(local_rows), index_is_i64, N.ptr(starts), N.ptr(ends), N.ptr(slots),
                    n_layout, self.block_size, N.ptr(self._bias_correction1),
                    N.ptr(self._denom_scale), n, params_p, grads_p, m_p, v_p, widths, strides, lrs,
                    *extra_args, N.ptr(self._error_flag), N.stream_handle(self.device))
        else:
            args = (n_rows, N.ptr(local_rows), index_is_i64, N.ptr(starts), N.ptr(ends), N.ptr(slots),
                    n_layout, self.block_size, n, params_p, grads_p, m_p, v_p, widths, strides, lrs,
                    *extra_args, N.ptr(self._error_flag), N.stream_handle(self.device))
        N.call(kernel, *args)
        if hooks:
            hooks[1]()

    def _prepare(self, iteration, gaussians, sparse_grad_local_ids, sparse_grad_components):
        manager = getattr(gaussians, "gpu_working_set_manager", None)
        if manager is None or manager.local_to_global_idx is None:
            raise RuntimeError(
                "[GPUResidentAdam] gpu_working_set_manager with local_to_global_idx is required")
        local_rows = sparse_grad_local_ids.to(device=self.device)
        if local_rows.dtype not in (torch.int64, torch.int32):
            local_rows = local_rows.to(torch.int64)
        local_rows = local_rows.contiguous()
        index_is_i64 = 1 if local_rows.dtype == torch.int64 else 0
        layout, arr, starts, ends, slots = self._layout_tables(manager)
        for name, _, _, _ in self.COMPONENT_SPECS:
            if name not in sparse_grad_components:
                raise KeyError(
                    f"[GPUResidentAdam] Missing sparse_grad_components[{name!r}] at iter={iteration}")
        return manager, local_rows, index_is_i64, layout, arr, starts, ends, slots

    def _touched(self, arr, starts, ends, local_rows, idx64):
        """Per-block touched counts; rows outside every resident block raise here,
        before any update, as the reference's slot lookup does (:275-279).  The
        rows must be sorted (TideGS passes unique ids)."""
        counts = self._touched_counts(len(arr), starts, ends, local_rows, idx64)
        if int(counts.sum()) != local_rows.numel():
            raise RuntimeError(
                "[GPUResidentAdam] a touched row lies outside every resident block of the layout")
        return counts

    def _check_error(self):
        """Device-side guard of the update kernel (a row that misses every block);
        read lazily, since the host check in _touched already covers sorted rows."""
        if int(self._error_flag.item()) != 0:
            raise RuntimeError(
                "[GPUResidentAdam] a touched row lies outside every resident block of the layout")

    def step(self, iteration: int, gaussians, sparse_grad_local_ids: torch.Tensor,
             sparse_grad_components: Dict[str, torch.Tensor]) -> Dict[str, Any]:
        empty = {"updated_blocks": 0, "updated_block_ids": [], "touched_rows": 0, "cold_rows": 0}
        if sparse_grad_local_ids is None or sparse_grad_components is None:
            return empty
        if sparse_grad_local_ids.numel() == 0:
            return empty
        manager, local_rows, idx64, layout, arr, starts, ends, slots = self._prepare(
            iteration, gaussians, sparse_grad_local_ids, sparse_grad_components)
        counts = self._touched(arr, starts, ends, local_rows, idx64)
        component_lrs = self._normalize_columns_lr(getattr(gaussians.optimizer, "columns_lr", None))
        beta1, beta2 = gaussians.optimizer.param_groups[0]["betas"]
        beta1, beta2 = float(beta1), float(beta2)
        eps = float(gaussians.optimizer.param_groups[0]["eps"])
        hit, cold_rows = self._update_touched_slot_metadata(arr, counts, beta1, beta2)
        param_views = {name: getattr(gaussians, attr).data for name, attr, _, _ in self.COMPONENT_SPECS}
        self._launch("tgs_resident_adam_step", local_rows.numel(), local_rows, idx64, starts, ends,
                     slots, len(layout), param_views, sparse_grad_components, component_lrs,
                     (beta1, beta2, eps, float(self.batch_size)))
        touched_rows = int(local_rows.numel())
        self._stats["optimizer_rows_touched_total"] += touched_rows
        self._update_state_stats()
        return {
            "updated_blocks": int(hit.size),
            "updated_block_ids": arr[hit, 2].tolist(),
            "touched_rows": touched_rows,
            "cold_rows": int(cold_rows),
        }

    # ---- update fused into the gradient launch --------------------------------
    # A caller that computes the touched rows' gradients on the GPU can apply
    # the update inside that launch (tgs_tide_project_bwd_update) instead of
    # materialising the gradients for step().  The host bookkeeping is step()'s:
    # launch_touch_counts() once the touched rows exist, fused_update_args()
    # before the fused launch.
    _FUSED_LR_ORDER = ("xyz", "scaling", "rotation", "opacity", "features_dc", "features_rest")

    def _fused_mode(self, iteration: int) -> Tuple[int, float, int]:
        """(optimizer id, rho, update_hessian) of tgs_tide_project_bwd_update."""
        return 0, 0.0, 1

    def launch_touch_counts(self, gaussians, local_rows: torch.Tensor) -> torch.Tensor:
        """Per-block touched-row counts of ``local_rows`` (ascending, unique),
        computed on the device stream and copied to pinned host memory without
        waiting.  The returned host tensor is valid once the stream has passed
        this point (after the caller's next synchronisation)."""
        manager = gaussians.gpu_working_set_manager
        layout, arr, starts, ends, slots = self._layout_tables(manager)
        local_rows = local_rows.contiguous()
        if local_rows.dtype not in (torch.int32, torch.int64):
            raise RuntimeError("[GPUResidentAdam] touched rows must be int32 or int64")
        n = len(arr)
        dev = getattr(self, "_fused_counts", None)
        if dev is None or dev.numel() < n:
            pin = self.device.type == "cuda"
            self._fused_counts = dev = torch.empty(n, dtype=torch.int64, device=self.device)
            self._fused_counts_host = torch.empty(n, dtype=torch.int64, pin_memory=pin)
        N.call("tgs_block_touch_counts", local_rows.numel(), N.ptr(local_rows),
               1 if local_rows.dtype == torch.int64 else 0, N.ptr(starts), N.ptr(ends), n,
               N.ptr(dev), N.stream_handle(self.device))
        host = self._fused_counts_host[:n]
        host.copy_(dev[:n], non_blocking=True)
        return host

    def fused_update_args(self, iteration: int, gaussians, n_rows: int,
                          counts_host: torch.Tensor) -> Tuple[tuple, Dict[str, Any]]:
        """Advance the touched slots' steps and bias terms (as step() does) and
        return the optimizer arguments of tgs_tide_project_bwd_update (from
        ``block_starts`` to ``error_flag``) and step()'s stats dict."""
        manager = gaussians.gpu_working_set_manager
        layout, arr, starts, ends, slots = self._layout_tables(manager)
        counts = counts_host.numpy()
        if counts.shape[0] != len(arr) or int(counts.sum()) != int(n_rows):
            raise RuntimeError(
                "[GPUResidentAdam] a touched row lies outside every resident block of the layout")
        component_lrs = self._normalize_columns_lr(getattr(gaussians.optimizer, "columns_lr", None))
        beta1, beta2 = gaussians.optimizer.param_groups[0]["betas"]
        beta1, beta2 = float(beta1), float(beta2)
        eps = float(gaussians.optimizer.param_groups[0]["eps"])
        hit, cold_rows = self._update_touched_slot_metadata(arr, counts, beta1, beta2)
        mode, rho, update_h = self._fused_mode(iteration)
        lrs = (ctypes.c_float * 6)(*[component_lrs[name] for name in self._FUSED_LR_ORDER])
        self._fused_lrs = lrs  # kept alive until the next call
        args = (N.ptr(starts), N.ptr(ends), N.ptr(slots), len(layout), self.block_size,
                N.ptr(self._bias_correction1), N.ptr(self._denom_scale), N.ptr(self._exp_avg),
                N.ptr(self._exp_avg_sq), self.STATE_PITCH, lrs, mode, beta1, beta2, eps,
                float(self.batch_size), rho, update_h, N.ptr(self._error_flag))
        self._stats["optimizer_rows_touched_total"] += int(n_rows)
        self._update_state_stats()
        return args, {
            "updated_blocks": int(hit.size),
            "updated_block_ids": arr[hit, 2].tolist(),
            "touched_rows": int(n_rows),
            "cold_rows": int(cold_rows),
        }

    def get_stats(self) -> Dict[str, Any]:
        self._check_error()
        self._update_state_stats()
        return dict(self._stats)


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

    def _fused_mode(self, iteration: int) -> Tuple[int, float, int]:
        return 1, self.rho, 1 if (int(iteration) % self.hessian_interval) == 0 else 0

    def step(self, iteration: int, gaussians, sparse_grad_local_ids: torch.Tensor,
             sparse_grad_components: Dict[str, torch.Tensor]) -> Dict[str, Any]:
        empty = {"updated_blocks": 0, "updated_block_ids": [], "touched_rows": 0, "cold_rows": 0}
        if sparse_grad_local_ids is None or sparse_grad_components is None:
            return empty
        if sparse_grad_local_ids.numel() == 0:
            return empty
        manager, local_rows, idx64, layout, arr, starts, ends, slots = self._prepare(
            iteration, gaussians, sparse_grad_local_ids, sparse_grad_components)
        counts = self._touched(arr, starts, ends, local_rows, idx64)
        component_lrs = self._normalize_columns_lr(getattr(gaussians.optimizer, "columns_lr", None))
        beta1, beta2 = gaussians.optimizer.param_groups[0]["betas"]
        eps = float(gaussians.optimizer.param_groups[0]["eps"])
        hit, cold_rows = self._update_touched_slot_metadata(arr, counts, float(beta1), float(beta2))
        update_h = 1 if (int(iteration) % self.hessian_interval) == 0 else 0
        param_views = {name: getattr(gaussians, attr).data for name, attr, _, _ in self.COMPONENT_SPECS}
        self._launch("tgs_resident_sophia_step", local_rows.numel(), local_rows, idx64, starts, ends,
                     slots, len(layout), param_views, sparse_grad_components, component_lrs,
                     (float(beta1), float(beta2), eps, self.rho, float(self.batch_size), update_h))
        touched_rows = int(local_rows.numel())
        self._stats["optimizer_rows_touched_total"] += touched_rows
        self._update_state_stats()
        return {
            "updated_blocks": int(hit.size),
            "updated_block_ids": arr[hit, 2].tolist(),
            "touched_rows": touched_rows,
            "cold_rows": int(cold_rows),
        }
