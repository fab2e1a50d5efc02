"""Fused per-batch TideGS training step on a resident ``[N, 59]`` table.

One call of :meth:`TideStep.step` does what a TideGS batch does on the GPU
(``strategies/tide_engine/engine.py:1435-2737`` + ``runtime.py:1741-1791``):
per-camera visibility filters (packed-projection rule), the touched-row set,
projection + SH colours, tile intersection and sort, alpha compositing, the
L1 + SSIM loss (``base_engine.py:464-488``), the full backward into compact
``[T, 59]`` row gradients, and the resident Adam (or Sophia) update of the
touched rows.  Every stage is a HIP kernel from ``libtidegs_amd.so``; this
module only sequences them and owns the buffers.

The per-camera loop of the reference becomes one launch per stage over the
whole batch: parameters do not change between the cameras of a batch, so the
gradients are the same, and each touched row accumulates its cameras in the
reference's camera order.

The host reads three small results per step (the reference syncs for all
three, ``isect_tiles.cu:166``, ``base_engine.py:407``,
``gpu_resident_optimizer.py:296``), each while the GPU has queued work behind
it, so the GPU never waits for the host: the visibility totals while the
projection runs (its launch covers every row and reads the touched-row count
on the device), the per-camera intersection counts (sums of the tile
rectangles' areas, known right after the projection) while the depth sort
runs, and the optimizer's per-block touch counts while the rasterizers run.
By default the optimizer update runs inside the projection-backward launch
(``tgs_tide_project_bwd_update``), so the compact gradient rows never reach
memory; ``fuse_update=False`` keeps the two-launch form (gradient rows, then
``GPUResidentAdam.step``).
"""
from __future__ import annotations

import ctypes
import math
import types
from dataclasses import dataclass, field
from typing import Dict, Optional

import torch

from . import _native as N
from .resident_optim import GPUResidentAdam, GPUResidentSophia

ROW = 59
# Row pitch of the compact gradient rows: whole 256-byte lines (see
# scenes.padded_table for the resident table's padded layout).
GRAD_PITCH = 64
# CACHE-order column slices of the optimizer components (unified names)
_CACHE_COLS = {
    "xyz": (0, 3),
    "scaling": (3, 6),
    "rotation": (6, 10),
    "opacity": (10, 11),
    "features_dc": (11, 14),
    "features_rest": (14, 59),
}


class _Manager:
    """Working-set view expected by GPUResidentAdam: all blocks resident."""

    def __init__(self, n_rows: int, block_size: int, device):
        n_blocks = -(-n_rows // block_size)
        self.loaded_blocks = list(range(n_blocks))
        self.block_to_gpu_slice = {
            b: slice(b * block_size, min(n_rows, (b + 1) * block_size)) for b in range(n_blocks)
        }
        self.local_to_global_idx = torch.empty(0, device=device)  # identity mapping


class _TableGaussians:
    """Component attributes as column views of the CACHE-order table."""

    def __init__(self, table, manager, columns_lr, betas, eps):
        self.gpu_working_set_manager = manager
        for name, (a, b) in _CACHE_COLS.items():
            setattr(self, "_" + name, table[:, a:b])
        self.optimizer = types.SimpleNamespace(columns_lr=columns_lr,
                                               param_groups=[{"betas": betas, "eps": eps}])


@dataclass
class StepStats:
    n_cameras: int
    visible_per_camera: list
    touched_rows: int
    entries: int
    n_isects: int
    loss_sums: torch.Tensor = field(repr=False)  # [C, 2] double on device
    optimizer: dict = field(default_factory=dict)
    isects_per_camera: list = field(default_factory=list)

    def losses(self, width: int, height: int, lambda_dssim: float = 0.2):
        s = self.loss_sums.double().cpu()
        n = 3.0 * width * height
        return [float((1 - lambda_dssim) * s[c, 0] / n + lambda_dssim * (1 - s[c, 1] / n))
                for c in range(s.shape[0])]


# Index widths of the fused step: entries, visits and the per-block count scan
# are 32-bit (the scan's total is V + T + V <= (2C + 1) N), and intersection
# keys, flatten ids and the per-tile offsets are int32 as in the reference's
# rasterizer (rasterize_to_pixels_fwd.cu: int32 tile ranges).
MAX_ISECTS = (1 << 31) - 1


def check_batch_capacity(n_rows: int, n_cams: int) -> None:
    """Refuse a batch whose 32-bit entry/visit counts could wrap."""
    if (2 * int(n_cams) + 1) * int(n_rows) >= (1 << 32):
        raise ValueError(
            f"TideStep: {n_rows} rows x {n_cams} cameras exceeds the 32-bit entry counts "
            f"((2C+1)*N must stay below 2^32); use fewer cameras per batch")


def check_isect_count(n_isects: int) -> None:
    """Refuse an intersection count that does not fit the int32 tile ranges."""
    if not 0 <= int(n_isects) <= MAX_ISECTS:
        raise RuntimeError(
            f"TideStep: {n_isects} intersections in one batch exceed the int32 range of the "
            f"tile offsets and flatten ids (max {MAX_ISECTS}); use fewer cameras per batch")


# ulps of slack around the visibility pass's depth-key range (its depths and
# the projection's are the same float expression)
DEPTH_KEY_SLACK = 256
RANGE_SLOTS = 64  # {min, max} pairs the visibility pass spreads the range over


def depth_key_range(lo: int, hi: int) -> tuple:
    """(key_base, key_bits) of the depth sort from the smallest and largest
    visible depth keys (uint32 float bits): every key of [lo - slack,
    hi + slack] maps below 2^key_bits - 1, where the culled entries' sentinel
    0xffffffff ties after them; (0, 32) when nothing is visible."""
    lo, hi = lo & 0xFFFFFFFF, hi & 0xFFFFFFFF
    if hi < lo:
        return 0, 32
    base = max(0, lo - DEPTH_KEY_SLACK)
    top = min(hi + DEPTH_KEY_SLACK, 0xFFFFFFFE)
    return base, min((top - base + 1).bit_length(), 32)


def depth_range_holds(slots, key_base: int, key_bits: int) -> bool:
    """True when every depth key the projection wrote (the min / max over its
    {min, max} slot pairs, sentinels excluded) ranks below the ranked sort's
    cap: key_base <= key < key_base + 2^key_bits - 1."""
    slots = [v & 0xFFFFFFFF for v in slots]
    lo, hi = min(slots[0::2]), max(slots[1::2])
    if hi < lo:  # no key written
        return True
    cap = (1 << key_bits) - 1
    return key_base <= lo and hi - key_base < cap


def _segments(offsets) -> "ctypes.Array":
    """Host uint32 array of segment offsets for tgs_segmented_sort_pairs_u32."""
    return (ctypes.c_uint32 * len(offsets))(*[int(o) for o in offsets])


class TideStep:
    """Fused TideGS batch step (forward, backward, resident optimizer) on one GPU."""

    TILE = 16

    def __init__(self, params: torch.Tensor, width: int, height: int, batch_size: int,
                 block_size: int = 4096, sh_degree: int = 3, columns_lr=None,
                 betas=(0.9, 0.999), eps: float = 1e-15, lr_scale_mode: str = "sqrt",
                 eps2d: float = 0.3, near_plane: float = 0.01, far_plane: float = 1e10,
                 radius_clip: float = 0.0, lambda_dssim: float = 0.2,
                 backgrounds: Optional[torch.Tensor] = None, optimizer: str = "adam",
                 sophia_rho: float = 0.04, gt_div: float = 255.0, keep_isect_ids: bool = False,
                 fuse_update: bool = True):
        if params.dim() != 2 or params.shape[1] != ROW or params.dtype != torch.float32:
            raise ValueError("params must be a float32 [N, 59] table (CACHE column order)")
        if not params.is_cuda or params.stride(1) != 1 or not ROW <= params.stride(0) <= 64:
            raise ValueError("params must be a GPU table with contiguous rows at a pitch of "
                             "59..64 floats (59: dense, 64: padded to 256-byte rows)")
        self.params = params
        self.row_stride = int(params.stride(0))
        self.device = params.device
        self.W, self.H = int(width), int(height)
        self.tw = -(-self.W // self.TILE)
        self.th = -(-self.H // self.TILE)
        self.bsz = int(batch_size)
        self.sh_degree = int(sh_degree)
        self.eps2d, self.near, self.far = float(eps2d), float(near_plane), float(far_plane)
        self.radius_clip = float(radius_clip)
        self.lambda_dssim = float(lambda_dssim)
        self.gt_div = float(gt_div)
        self.backgrounds = backgrounds
        self.keep_isect_ids = bool(keep_isect_ids)  # materialise gsplat's isect keys (tests)
        # step(): optimizer update inside the projection-backward launch (True)
        # or as its own launch over materialised gradient rows (False)
        self.fuse_update = bool(fuse_update)
        n = params.shape[0]
        # TideGS hyper-parameter scaling (gaussian_model.py:855-888)
        if columns_lr is None:
            columns_lr = [1.6e-4, 0.05, 5e-3, 1e-3, 2.5e-3, 2.5e-3 / 20.0]
        cols = torch.tensor(columns_lr, dtype=torch.float32)
        if lr_scale_mode == "sqrt":
            scale = math.sqrt(self.bsz)
            cols = cols * scale
            eps = eps / scale
            betas = tuple(b ** self.bsz for b in betas)
        elif lr_scale_mode == "linear":
            cols = cols * self.bsz
        self.manager = _Manager(n, block_size, self.device)
        self.gaussians = _TableGaussians(params, self.manager, cols, betas, eps)
        opt_cls = GPUResidentSophia if optimizer == "sophia" else GPUResidentAdam
        kw = {"rho": sophia_rho} if optimizer == "sophia" else {}
        self.optimizer = opt_cls(batch_size=self.bsz, block_size=block_size,
                                 capacity_blocks=len(self.manager.loaded_blocks),
                                 device=str(self.device), **kw)
        self.optimizer.set_resident_blocks(self.manager.loaded_blocks)
        self._iteration = 0
        self._bufs: Dict[str, torch.Tensor] = {}
        self.last: Dict[str, torch.Tensor] = {}
        self._timing = False
        self._count_pairs = False
        self._events = []
        self.stage_ms: Dict[str, float] = {}
        self.last_visible_entries = 0
        self.last_live_pairs = 0  # composited (Gaussian, pixel) pairs of the last counting step
        self.last_depth_key_bits = 32  # key bits of the last step's depth sort
        # steps whose projected depth keys fell outside the visibility pass's
        # range, so that the depth sort was redone on all 32 bits
        self.depth_sort_repairs = 0

    # ---- stage timing (HIP events on the launch stream) ----------------------
    def _begin(self, name: str):
        if self._timing:
            ev = torch.cuda.Event(enable_timing=True)
            ev.record()
            self._events.append([name, ev, None])

    def _end(self):
        if self._timing:
            ev = torch.cuda.Event(enable_timing=True)
            ev.record()
            self._events[-1][2] = ev

    def _collect(self):
        torch.cuda.synchronize(self.device)
        out: Dict[str, float] = {}
        for name, a, b in self._events:
            out[name] = out.get(name, 0.0) + a.elapsed_time(b)
        self._events = []
        self.stage_ms = out

    # ---- buffers ----------------------------------------------------------
    def _buf(self, name: str, numel: int, dtype) -> torch.Tensor:
        b = self._bufs.get(name)
        if b is None or b.numel() < numel or b.dtype != dtype:
            b = torch.empty(max(1, int(numel * 1.25) if b is not None else numel), dtype=dtype,
                            device=self.device)
            self._bufs[name] = b
        return b[:numel]

    def _pinned(self, name: str, numel: int, dtype) -> torch.Tensor:
        """Pinned host buffer for an asynchronous device-to-host copy."""
        key = "host_" + name
        b = self._bufs.get(key)
        if b is None or b.numel() < numel or b.dtype != dtype:
            b = torch.empty(numel, dtype=dtype, pin_memory=True)
            self._bufs[key] = b
        return b[:numel]

    def _record(self) -> torch.cuda.Event:
        ev = torch.cuda.Event()
        ev.record(torch.cuda.current_stream(self.device))
        return ev

    # ---- stages -----------------------------------------------------------
    def forward_backward(self, viewmats: torch.Tensor, Ks: torch.Tensor, gt: torch.Tensor,
                         count_pairs: bool = False):
        """Everything up to the compact gradients; returns (touched, grads, stats).
        ``count_pairs`` as for :meth:`step` (the per-pixel counts are left in
        ``self.last["n_contrib"]``)."""
        self._count_pairs = bool(count_pairs)
        try:
            return self._run(viewmats, Ks, gt, update=False)
        finally:
            self._count_pairs = False

    def _run(self, viewmats: torch.Tensor, Ks: torch.Tensor, gt: torch.Tensor, update: bool):
        """The batch's stages.  With ``update`` the last stage applies the
        optimizer to the touched rows in the projection-backward launch
        (tgs_tide_project_bwd_update) and no gradient rows are returned."""
        C = viewmats.shape[0]
        if not 1 <= C <= 32:
            raise ValueError("1..32 cameras per batch")
        s = N.stream_handle(self.device)
        P = self.params
        n = P.shape[0]
        check_batch_capacity(n, C)
        W, H, tw, th = self.W, self.H, self.tw, self.th
        viewmats = viewmats.to(self.device, torch.float32).contiguous()
        Ks = Ks.to(self.device, torch.float32).contiguous()
        campos = self._buf("campos", 3 * C, torch.float32).view(C, 3)
        self._begin("camera_centers")
        N.call("tgs_tide_camera_centers", C, N.ptr(viewmats), N.ptr(campos), s)
        self._end()
        gt = gt.to(self.device, torch.float32).contiguous()
        lib = N.load()

        # 1. visibility masks + per-block counts, scan, compaction
        nb = lib.tgs_tide_row_blocks(n)
        masks = self._buf("masks", n, torch.int32)
        counts = self._buf("counts", (C + 2) * nb, torch.int32)
        self._begin("visibility")
        # totals [C+3+128]: V_c..., T, sum V, visits (compaction), then 64
        # {min, max} pairs of the depth keys' range (visibility)
        totals = self._buf("totals", C + 3 + 2 * RANGE_SLOTS, torch.int32)
        N.call("tgs_tide_visibility", n, N.ptr(P), self.row_stride, C, N.ptr(viewmats), N.ptr(Ks),
               N.ptr(campos),
               W, H, self.eps2d, self.near, self.far, self.radius_clip, N.ptr(masks),
               N.ptr(counts), N.ptr(totals) + 4 * (C + 3), s)
        offs = self._buf("offs", (C + 2) * nb, torch.int32)
        ws = self._buf("scan_ws", lib.tgs_scan_workspace_size((C + 2) * nb), torch.uint8)
        N.call("tgs_exclusive_scan_u32", N.ptr(counts), N.ptr(offs), (C + 2) * nb, N.ptr(ws),
               ws.numel(), s)
        entries = self._buf("entries", C * n, torch.int32)
        visits = self._buf("visits", C * n, torch.int32)
        touched = self._buf("touched", n, torch.int32)
        visit_base = self._buf("visit_base", n + 1, torch.int32)
        cam_offsets = self._buf("cam_offsets", C + 1, torch.int32)
        N.call("tgs_tide_compact", n, C, N.ptr(masks), N.ptr(counts), N.ptr(offs), N.ptr(entries),
               N.ptr(touched), N.ptr(visit_base), N.ptr(visits), N.ptr(totals),
               N.ptr(cam_offsets), s)
        self._end()
        # the totals (V per camera, T, V) go to the host while the projection
        # runs: its launch covers every row and reads T on the device
        tot_host = self._pinned("totals", C + 3 + 2 * RANGE_SLOTS, torch.int32)
        tot_host.copy_(totals, non_blocking=True)
        totals_ready = self._record()

        # 2. projection + SH colours for every (camera, visible row), one pass over
        #    the touched rows; depth keys and tile rectangles for the sort.
        #    Entry buffers hold the C * N entries a batch can have at most.
        n_buckets = C * th * tw
        cap_v = C * n
        splats = self._buf("splats", cap_v * 12, torch.float32)
        dkeys = self._buf("depth_keys", cap_v, torch.int32)
        rects = self._buf("entry_rects", cap_v, torch.int64)
        # the projection also sums the per-camera intersection counts (the
        # rectangles' areas); they go to the host while the depth sort runs
        isect_tot = self._buf("isect_totals", C, torch.int64)
        # and the range of the depth keys it writes, to check the depth sort's
        # range (taken from the visibility pass) against
        proj_range = self._buf("proj_range", 2 * RANGE_SLOTS, torch.int32)
        self._begin("project_fwd")
        N.call("tgs_tide_project_fwd", n, N.ptr(totals) + 4 * C, N.ptr(touched),
               N.ptr(visit_base), N.ptr(visits), N.ptr(masks), C, N.ptr(P), self.row_stride,
               N.ptr(viewmats), N.ptr(Ks), N.ptr(campos), W, H, self.eps2d, self.near, self.far,
               0.0, self.sh_degree, self.TILE, tw, th, N.ptr(splats), N.ptr(dkeys), N.ptr(rects),
               N.ptr(isect_tot), N.ptr(proj_range), s)
        self._end()
        isect_host = self._pinned("isect_totals", C, torch.int64)
        isect_host.copy_(isect_tot, non_blocking=True)
        range_host = self._pinned("proj_range", 2 * RANGE_SLOTS, torch.int32)
        range_host.copy_(proj_range, non_blocking=True)
        isects_ready = self._record()

        totals_ready.synchronize()  # host read 1: the projection keeps the GPU busy
        tot = tot_host.tolist()
        V = tot[C + 1]
        T = tot[C]
        if update and T:
            # per-block touch counts for the optimizer's slot bookkeeping
            self._begin("touch_counts")
            counts_host = self.optimizer.launch_touch_counts(self.gaussians, touched[:T])
            self._end()
            counts_ready = self._record()

        # 3. intersections in the reference's (camera, tile, depth, entry) order:
        #    depth sort of the entries per camera; each block of depth-ordered
        #    entries' intersections counted by the tile-bit sort's first digit
        #    (scanned: every (camera, digit, block)'s first slot); the emission
        #    fused with that first pass; the remaining tile-bit pass per
        #    camera; bucket offsets
        cam_segs = _segments([sum(tot[:c]) for c in range(C + 1)])
        dkeys2 = self._buf("depth_keys2", cap_v, torch.int32)
        rects2 = self._buf("entry_rects2", cap_v, torch.int64)
        tile_bits = (tw * th).bit_length()
        hist_words = max(int(lib.tgs_tide_isect_fused_hist_words(C, cam_segs, tile_bits)), 1)
        fe_hist = self._buf("fused_hist", hist_words, torch.int32)
        fe_scan = self._buf("fused_hist_scan", hist_words, torch.int32)
        ws = self._buf("scan_ws2", lib.tgs_scan_workspace_size(hist_words), torch.uint8)
        self._begin("isect_scan")
        key_base, key_bits = 0, 32
        if V:
            sel = ctypes.c_int(0)
            dws = self._buf("sort_ws", lib.tgs_segmented_sort_workspace_size(V, C), torch.uint8)
            # depth keys ranked relative to the visible range: 25 bits at cfg3,
            # four 6-7 bit passes instead of four 8-bit ones
            rng = [v & 0xFFFFFFFF for v in tot[C + 3:]]
            key_base, key_bits = depth_key_range(min(rng[0::2]), max(rng[1::2]))
            N.call("tgs_segmented_sort_pairs_u32_range", N.ptr(dkeys), N.ptr(rects),
                   N.ptr(dkeys2), N.ptr(rects2), 8, V, C, cam_segs, key_base, key_bits,
                   N.ptr(dws), dws.numel(), ctypes.byref(sel), s)
            if sel.value:
                dkeys, rects, dkeys2, rects2 = dkeys2, rects2, dkeys, rects
            N.call("tgs_tide_isect_fused_count", C, cam_segs, N.ptr(rects), tw, tile_bits,
                   N.ptr(fe_hist), hist_words, s)
            N.call("tgs_exclusive_scan_u32", N.ptr(fe_hist), N.ptr(fe_scan), hist_words,
                   N.ptr(ws), ws.numel(), s)
        self._end()
        self.last_depth_key_bits = key_bits
        isects_ready.synchronize()  # host read 2: the depth sort keeps the GPU busy
        if V and not depth_range_holds(range_host.tolist(), key_base, key_bits):
            # a projected key outside the visibility pass's range (plus slack)
            # tied with its neighbours in the ranked sort; a stable sort on all
            # 32 bits of the ranked result restores the (depth, entry) order,
            # since equal keys kept their input order in the ranked sort
            self.depth_sort_repairs += 1
            self._begin("depth_sort_repair")
            sel = ctypes.c_int(0)
            N.call("tgs_segmented_sort_pairs_u32", N.ptr(dkeys), N.ptr(rects), N.ptr(dkeys2),
                   N.ptr(rects2), 8, V, C, cam_segs, 0, 32, N.ptr(dws), dws.numel(),
                   ctypes.byref(sel), s)
            if sel.value:
                dkeys, rects, dkeys2, rects2 = dkeys2, rects2, dkeys, rects
            N.call("tgs_tide_isect_fused_count", C, cam_segs, N.ptr(rects), tw, tile_bits,
                   N.ptr(fe_hist), hist_words, s)
            N.call("tgs_exclusive_scan_u32", N.ptr(fe_hist), N.ptr(fe_scan), hist_words,
                   N.ptr(ws), ws.numel(), s)
            self._end()
        per_cam = isect_host.tolist()
        isect_segs = [0]
        for k in per_cam:
            isect_segs.append(isect_segs[-1] + int(k))
        n_isects = isect_segs[C]
        check_isect_count(n_isects)
        cap = max(n_isects, 1)
        keys = self._buf("keys", cap, torch.int32)
        keys2 = self._buf("keys2", cap, torch.int32)
        fids = self._buf("fids", cap, torch.int32)
        fids2 = self._buf("fids2", cap, torch.int32)
        offsets = self._buf("offsets", n_buckets, torch.int32)
        self._begin("isect_sort")
        if n_isects:
            # intersections written in the order of the tile-bit sort's first
            # pass, then its remaining passes
            N.call("tgs_tide_isect_fused_scatter", C, cam_segs, N.ptr(rects), tw, tile_bits,
                   N.ptr(fe_scan), hist_words, n_isects, N.ptr(keys), N.ptr(fids), s)
            w1 = int(lib.tgs_tide_isect_fused_digit_bits(tile_bits))
            if tile_bits > w1:
                tws = self._buf("sort_ws2", lib.tgs_segmented_sort_workspace_size(n_isects, C),
                                torch.uint8)
                sel = ctypes.c_int(0)
                N.call("tgs_segmented_sort_pairs_u32", N.ptr(keys), N.ptr(fids), N.ptr(keys2),
                       N.ptr(fids2), 4, n_isects, C, _segments(isect_segs), w1, tile_bits,
                       N.ptr(tws), tws.numel(), ctypes.byref(sel), s)
                if sel.value:
                    keys, fids = keys2, fids2
        N.call("tgs_tide_offset_encode", n_isects, N.ptr(keys), C, tw, th, tile_bits,
               N.ptr(offsets), s)
        self._end()
        isect_ids = None
        if self.keep_isect_ids:
            isect_ids = self._buf("isect_ids", cap, torch.int64)
            N.call("tgs_tide_isect_ids", n_isects, N.ptr(keys), N.ptr(fids), N.ptr(splats),
                   N.ptr(isect_ids), s)

        # 4. rasterize, loss, loss backward, rasterize backward
        images = self._buf("images", C * H * W * 3, torch.float32)
        alphas = self._buf("alphas", C * H * W, torch.float32)
        last_ids = self._buf("last_ids", C * H * W, torch.int32)
        bg = self.backgrounds
        # the backward's per-entry gradient records, zeroed by the forward launch
        sg_words = (max(V, 1) * 9 + 3) // 4 * 4
        sgrads = self._buf("splat_grads", sg_words, torch.float32)
        self._begin("raster_fwd")
        # with timing, also each pixel's composited-Gaussian count (the live
        # (Gaussian, pixel) pairs the backward replays)
        n_contrib = self._buf("n_contrib", C * H * W, torch.int32) if self._count_pairs else None
        N.call("tgs_tide_rasterize_fwd", C, N.ptr(splats), N.ptr(bg), W, H, tw, th,
               N.ptr(offsets), N.ptr(fids), n_isects, N.ptr(images), N.ptr(alphas),
               N.ptr(last_ids), N.ptr(n_contrib), N.ptr(sgrads), sg_words, s)
        self._end()
        sums = self._buf("loss_sums", 2 * C, torch.float64)
        v_images = self._buf("v_images", C * H * W * 3, torch.float32)
        self._begin("loss")
        N.call("tgs_fill_u32", N.ptr(sums), 4 * C, 0, s)
        N.call("tgs_tide_loss", C, H, W, N.ptr(images), N.ptr(gt), self.gt_div,
               self.lambda_dssim, N.ptr(sums), N.ptr(v_images), s)
        self._end()
        self._begin("raster_bwd")
        N.call("tgs_tide_rasterize_bwd", C, N.ptr(splats), N.ptr(bg), W, H, tw, th,
               N.ptr(offsets), N.ptr(fids), n_isects, N.ptr(alphas), N.ptr(last_ids),
               N.ptr(v_images), None, N.ptr(sgrads), s)
        self._end()

        # 5. per touched row: projection + SH + activation backward (and, with
        #    update, the resident optimizer step of the row in the same launch)
        grads = None
        opt_stats: dict = {}
        if update:
            if T:
                self._iteration += 1
                # slot bookkeeping and the bias-term upload (host work that
                # overlaps the raster backward; the bracket shows what of it
                # reaches the GPU's timeline)
                self._begin("optimizer_host")
                counts_ready.synchronize()
                opt_args, opt_stats = self.optimizer.fused_update_args(
                    self._iteration, self.gaussians, T, counts_host)
                self._end()
                self._begin("project_bwd_update")
                N.call("tgs_tide_project_bwd_update", T, N.ptr(touched), N.ptr(visit_base),
                       N.ptr(visits), N.ptr(masks), C, N.ptr(P), self.row_stride,
                       N.ptr(viewmats), N.ptr(Ks), N.ptr(campos), W, H, self.eps2d, self.near,
                       self.far, 0.0, self.sh_degree, N.ptr(sgrads), *opt_args, s)
                self._end()
        else:
            grads = self._buf("grads", max(T, 1) * GRAD_PITCH, torch.float32).view(-1, GRAD_PITCH)
            grads = grads[:T, :ROW]
            self._begin("project_bwd")
            N.call("tgs_tide_project_bwd", T, N.ptr(touched), N.ptr(visit_base), N.ptr(visits),
                   N.ptr(masks), C, N.ptr(P), self.row_stride, N.ptr(viewmats), N.ptr(Ks),
                   N.ptr(campos), W, H, self.eps2d, self.near, self.far, 0.0, self.sh_degree,
                   N.ptr(sgrads), N.ptr(grads), GRAD_PITCH, s)
            self._end()
        if self._timing:
            self.last_visible_entries = int((splats[: V * 12].view(-1, 12)[:, 7] > 0).sum())
        if self._count_pairs:
            self.last_live_pairs = int(n_contrib.sum(dtype=torch.int64))
        self.last = dict(masks=masks, entries=entries[:V], cam_offsets=cam_offsets,
                         touched=touched[:T], visit_base=visit_base[:T + 1], visits=visits[:V],
                         splats=splats[: V * 12].view(-1, 12),
                         isect_ids=isect_ids[:n_isects] if isect_ids is not None else None,
                         flatten_ids=fids[:n_isects], offsets=offsets[:n_buckets].view(C, th, tw),
                         images=images.view(C, H, W, 3), alphas=alphas.view(C, H, W),
                         last_ids=last_ids.view(C, H, W), v_images=v_images.view(C, H, W, 3),
                         splat_grads=sgrads[: V * 9].view(-1, 9), grads=grads, campos=campos,
                         n_contrib=n_contrib.view(C, H, W) if n_contrib is not None else None)
        stats = StepStats(n_cameras=C, visible_per_camera=tot[:C], touched_rows=T, entries=V,
                          n_isects=n_isects, loss_sums=sums.view(C, 2), optimizer=opt_stats,
                          isects_per_camera=[isect_segs[c + 1] - isect_segs[c] for c in range(C)])
        return touched[:T], grads, stats

    def snapshot(self) -> dict:
        """A copy of everything a step changes (the resident table, the
        optimizer's moments and slot bookkeeping, the iteration count), so
        that :meth:`restore` can run a step again from the same scene state."""
        torch.cuda.current_stream(self.device).synchronize()
        return {"params": self.params.clone(), "optimizer": self.optimizer.snapshot(),
                "iteration": self._iteration}

    def restore(self, snap: dict) -> None:
        """Put a :meth:`snapshot` back in place (device copies queued on the
        current stream)."""
        self.params.copy_(snap["params"])
        self.optimizer.restore(snap["optimizer"])
        self._iteration = snap["iteration"]

    def optimizer_step(self, touched: torch.Tensor, grads: torch.Tensor) -> dict:
        self._iteration += 1
        comps = {name: grads[:, a:b] for name, (a, b) in _CACHE_COLS.items()}
        return self.optimizer.step(self._iteration, self.gaussians, touched, comps)

    def step(self, viewmats: torch.Tensor, Ks: torch.Tensor, gt: torch.Tensor,
             timing: bool = False, count_pairs: bool = False) -> StepStats:
        """One batch: forward, backward and the resident optimizer update.

        With ``timing`` the stages are bracketed by HIP events on the launch
        stream and their times (ms) are left in ``self.stage_ms``.  With
        ``count_pairs`` the forward also counts each pixel's composited
        Gaussians (a slower variant of its walk) and leaves their sum in
        ``self.last_live_pairs``.
        """
        self._timing = bool(timing)
        self._count_pairs = bool(count_pairs)
        self._events = []
        try:
            if self.fuse_update:
                _, _, stats = self._run(viewmats, Ks, gt, update=True)
            else:
                touched, grads, stats = self._run(viewmats, Ks, gt, update=False)
                if self._timing:
                    self.optimizer.kernel_hooks = (lambda: self._begin("adam"), self._end)
                stats.optimizer = self.optimizer_step(touched, grads) if touched.numel() else {}
            if self._timing:
                self._collect()
        finally:
            self._timing = False
            self._count_pairs = False
            self.optimizer.kernel_hooks = None
        return stats
