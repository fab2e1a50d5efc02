"""Drop-in replacements for the gsplat ops TideGS imports.

Call sites served unchanged (``strategies/tide_engine/engine.py:217-223``,
``strategies/base_engine.py:9-15``)::

    from tidegs_amd.gsplat_ops import (fully_fused_projection, spherical_harmonics,
                                       isect_tiles, isect_offset_encode,
                                       rasterize_to_pixels)

Names, keyword signatures, return tuples and autograd behaviour follow
gsplat 1.0's ``gsplat/cuda/_wrapper.py`` contract as used by TideGS
(``engine.py:480-561``): projection is differentiable w.r.t. means / quats /
scales (or covars) and optionally viewmats; SH w.r.t. dirs and coeffs;
rasterization w.r.t. means2d, conics, colors, opacities and backgrounds.
Every op runs the MI355X HIP kernels of ``libtidegs_amd.so``; GPU tensors are
required and there is no CPU path.
"""
from __future__ import annotations

import ctypes
import math
from typing import Optional, Tuple

import torch
from torch import Tensor

from . import _native as N

_SUPPORTED_CHANNELS = (1, 2, 3, 4, 8, 16, 32)
_CHUNK = 32  # channels per launch above 32


def _pad_channels(ch: int) -> int:
    """The smallest instantiated channel count >= ch (ch <= 32)."""
    return next(d for d in _SUPPORTED_CHANNELS if d >= ch)


def _pad_last(t: Optional[Tensor], width: int) -> Optional[Tensor]:
    """``t`` zero-padded along its last dimension to ``width`` (contiguous)."""
    if t is None:
        return None
    if t.shape[-1] == width:
        return t.contiguous()
    pad = torch.zeros(*t.shape[:-1], width - t.shape[-1], dtype=t.dtype, device=t.device)
    return torch.cat([t, pad], -1).contiguous()


def _channel_chunks(ch: int):
    """(first channel, channels, launched channels) of each launch: one launch
    up to 32 channels, else consecutive runs of 32 and a padded remainder."""
    if ch <= _CHUNK:
        return [(0, ch, _pad_channels(ch))]
    return [(s, min(_CHUNK, ch - s), _pad_channels(min(_CHUNK, ch - s)))
            for s in range(0, ch, _CHUNK)]


def _pixel_mask(masks: Tensor, tile_size: int, height: int, width: int) -> Tensor:
    """[C, H, W] bool: the tile mask of every pixel."""
    m = masks.to(torch.bool)
    return m.repeat_interleave(tile_size, 1).repeat_interleave(tile_size, 2)[:, :height, :width]


def _stream() -> int:
    return N.stream_handle()


# ---------------------------------------------------------------------------
# fully_fused_projection
# ---------------------------------------------------------------------------


class _FullyFusedProjection(torch.autograd.Function):
    @staticmethod
    def forward(ctx, means, covars, quats, scales, viewmats, Ks, width, height, eps2d,
                near_plane, far_plane, radius_clip, calc_compensations):
        C, Nn = viewmats.shape[0], means.shape[0]
        dev = means.device
        radii = torch.empty((C, Nn), dtype=torch.int32, device=dev)
        means2d = torch.empty((C, Nn, 2), dtype=torch.float32, device=dev)
        depths = torch.empty((C, Nn), dtype=torch.float32, device=dev)
        conics = torch.empty((C, Nn, 3), dtype=torch.float32, device=dev)
        comps = torch.empty((C, Nn), dtype=torch.float32, device=dev) if calc_compensations else None
        N.call(
            "tgs_fully_fused_projection_fwd", C, Nn, N.ptr(means), N.ptr(covars), N.ptr(quats),
            N.ptr(scales), N.ptr(viewmats), N.ptr(Ks), int(width), int(height), float(eps2d),
            float(near_plane), float(far_plane), float(radius_clip), N.ptr(radii),
            N.ptr(means2d), N.ptr(depths), N.ptr(conics), N.ptr(comps), _stream(),
        )
        ctx.save_for_backward(means, covars, quats, scales, viewmats, Ks, radii, conics, comps)
        ctx.width, ctx.height, ctx.eps2d = int(width), int(height), float(eps2d)
        ctx.mark_non_differentiable(radii)
        return radii, means2d, depths, conics, comps

    @staticmethod
    def backward(ctx, v_radii, v_means2d, v_depths, v_conics, v_comps):
        means, covars, quats, scales, viewmats, Ks, radii, conics, comps = ctx.saved_tensors
        C, Nn = viewmats.shape[0], means.shape[0]

        def _c(t, like):
            return torch.zeros_like(like) if t is None else t.contiguous()

        v_means2d = _c(v_means2d, radii.unsqueeze(-1).expand(C, Nn, 2).float())
        v_depths = _c(v_depths, radii.float())
        v_conics = _c(v_conics, conics)
        v_comps = v_comps.contiguous() if (v_comps is not None and comps is not None) else None
        v_means = torch.empty_like(means)
        v_covars = torch.empty_like(covars) if covars is not None else None
        v_quats = torch.empty_like(quats) if covars is None else None
        v_scales = torch.empty_like(scales) if covars is None else None
        v_viewmats = torch.zeros_like(viewmats) if ctx.needs_input_grad[4] else None
        N.call(
            "tgs_fully_fused_projection_bwd", C, Nn, N.ptr(means), N.ptr(covars), N.ptr(quats),
            N.ptr(scales), N.ptr(viewmats), N.ptr(Ks), ctx.width, ctx.height, ctx.eps2d,
            N.ptr(radii), N.ptr(conics), N.ptr(comps), N.ptr(v_means2d), N.ptr(v_depths),
            N.ptr(v_conics), N.ptr(v_comps), N.ptr(v_means), N.ptr(v_covars), N.ptr(v_quats),
            N.ptr(v_scales), N.ptr(v_viewmats), _stream(),
        )
        return (v_means, v_covars, v_quats, v_scales, v_viewmats, None, None, None, None, None,
                None, None, None)


class _FullyFusedProjectionPacked(torch.autograd.Function):
    """Packed projection (fully_fused_projection_packed_fwd.cu / _bwd.cu): the
    surviving (camera, Gaussian) entries as COO arrays."""

    @staticmethod
    def forward(ctx, means, covars, quats, scales, viewmats, Ks, width, height, eps2d,
                near_plane, far_plane, radius_clip, sparse_grad, calc_compensations):
        C, Nn = viewmats.shape[0], means.shape[0]
        dev = means.device
        s = _stream()
        lib = N.load()
        nb = int(lib.tgs_fully_fused_projection_packed_blocks(Nn))
        n_blocks = max(C * nb, 1)
        counts = torch.zeros(n_blocks, dtype=torch.int32, device=dev)
        offsets = torch.zeros(n_blocks, dtype=torch.int32, device=dev)
        args = (N.ptr(means), N.ptr(covars), N.ptr(quats), N.ptr(scales), N.ptr(viewmats),
                N.ptr(Ks), int(width), int(height), float(eps2d), float(near_plane),
                float(far_plane), float(radius_clip))
        nnz = 0
        if C * Nn:
            N.call("tgs_fully_fused_projection_packed_count", C, Nn, *args, N.ptr(counts), s)
            ws = torch.empty(int(lib.tgs_scan_workspace_size(n_blocks)), dtype=torch.uint8,
                             device=dev)
            N.call("tgs_exclusive_scan_u32", N.ptr(counts), N.ptr(offsets), n_blocks, N.ptr(ws),
                   ws.numel(), s)
            # host read of the entry count, as the reference's block_accum[-1].item()
            nnz = int((offsets[-1] + counts[-1]).item())
        indptr = torch.empty(C + 1, dtype=torch.int32, device=dev)
        camera_ids = torch.empty(nnz, dtype=torch.int64, device=dev)
        gaussian_ids = torch.empty(nnz, dtype=torch.int64, device=dev)
        radii = torch.empty(nnz, dtype=torch.int32, device=dev)
        means2d = torch.empty((nnz, 2), dtype=torch.float32, device=dev)
        depths = torch.empty(nnz, dtype=torch.float32, device=dev)
        conics = torch.empty((nnz, 3), dtype=torch.float32, device=dev)
        comps = torch.zeros(nnz, dtype=torch.float32, device=dev) if calc_compensations else None
        N.call("tgs_fully_fused_projection_packed_fwd", C, Nn, *args, N.ptr(offsets), nnz,
               N.ptr(indptr), N.ptr(camera_ids), N.ptr(gaussian_ids), N.ptr(radii),
               N.ptr(means2d), N.ptr(depths), N.ptr(conics), N.ptr(comps), s)
        ctx.save_for_backward(means, covars, quats, scales, viewmats, Ks, camera_ids,
                              gaussian_ids, conics, comps)
        ctx.width, ctx.height, ctx.eps2d = int(width), int(height), float(eps2d)
        ctx.sparse_grad = bool(sparse_grad)
        ctx.mark_non_differentiable(indptr, camera_ids, gaussian_ids, radii)
        return indptr, camera_ids, gaussian_ids, radii, means2d, depths, conics, comps

    @staticmethod
    def backward(ctx, v_indptr, v_camera_ids, v_gaussian_ids, v_radii, v_means2d, v_depths,
                 v_conics, v_comps):
        (means, covars, quats, scales, viewmats, Ks, camera_ids, gaussian_ids, conics,
         comps) = ctx.saved_tensors
        C, Nn = viewmats.shape[0], means.shape[0]
        nnz = camera_ids.numel()
        dev = means.device

        def _c(t, shape):
            return torch.zeros(shape, dtype=torch.float32, device=dev) if t is None else \
                t.contiguous()

        v_means2d = _c(v_means2d, (nnz, 2))
        v_depths = _c(v_depths, (nnz,))
        v_conics = _c(v_conics, (nnz, 3))
        v_comps = v_comps.contiguous() if (v_comps is not None and comps is not None) else None
        rows = nnz if ctx.sparse_grad else Nn
        v_means = torch.zeros((rows, 3), dtype=torch.float32, device=dev)
        v_covars = torch.zeros((rows, 6), dtype=torch.float32, device=dev) \
            if covars is not None else None
        v_quats = torch.zeros((rows, 4), dtype=torch.float32, device=dev) if covars is None else None
        v_scales = torch.zeros((rows, 3), dtype=torch.float32, device=dev) if covars is None else None
        v_viewmats = torch.zeros_like(viewmats) if ctx.needs_input_grad[4] else None
        N.call("tgs_fully_fused_projection_packed_bwd", C, Nn, nnz, N.ptr(means), N.ptr(covars),
               N.ptr(quats), N.ptr(scales), N.ptr(viewmats), N.ptr(Ks), ctx.width, ctx.height,
               ctx.eps2d, N.ptr(camera_ids), N.ptr(gaussian_ids), N.ptr(conics), N.ptr(comps),
               N.ptr(v_means2d), N.ptr(v_depths), N.ptr(v_conics), N.ptr(v_comps),
               int(ctx.sparse_grad), N.ptr(v_means), N.ptr(v_covars), N.ptr(v_quats),
               N.ptr(v_scales), N.ptr(v_viewmats), _stream())
        if ctx.sparse_grad:
            # gsplat's sparse gradients: COO tensors over the Gaussian rows
            idx = gaussian_ids[None]

            def _sp(v, shape):
                return None if v is None else torch.sparse_coo_tensor(idx, v, shape)

            v_means = _sp(v_means, means.shape)
            v_covars = _sp(v_covars, covars.shape) if covars is not None else None
            v_quats = _sp(v_quats, quats.shape) if quats is not None else None
            v_scales = _sp(v_scales, scales.shape) if scales is not None else None
        return (v_means, v_covars, v_quats, v_scales, v_viewmats, None, None, None, None, None,
                None, None, None, None)


def fully_fused_projection(
    means: Tensor,
    covars: Optional[Tensor] = None,
    quats: Optional[Tensor] = None,
    scales: Optional[Tensor] = None,
    viewmats: Tensor = None,
    Ks: Tensor = None,
    width: int = None,
    height: int = None,
    eps2d: float = 0.3,
    near_plane: float = 0.01,
    far_plane: float = 1e10,
    radius_clip: float = 0.0,
    packed: bool = False,
    sparse_grad: bool = False,
    calc_compensations: bool = False,
) -> Tuple[Tensor, ...]:
    """EWA projection of 3D Gaussians (gsplat fully_fused_projection).

    Non-packed: ``(radii [C,N] i32, means2d [C,N,2], depths [C,N], conics [C,N,3],
    compensations [C,N] or None)`` (``engine.py:480``).  Packed: the surviving
    entries under the packed radius rule, camera-major and Gaussian-ascending,
    as gsplat 1.0's 7-tuple ``(camera_ids [nnz] i64, gaussian_ids [nnz] i64,
    radii [nnz] i32, means2d [nnz,2], depths [nnz], conics [nnz,3],
    compensations [nnz] or None)`` (``base_engine.py:112-121,329-340``).
    ``sparse_grad`` (packed only) returns the Gaussian gradients as COO tensors.
    """
    if sparse_grad and not packed:
        raise ValueError("sparse_grad requires packed=True")
    assert means.dim() == 2 and means.shape[-1] == 3, means.shape
    if covars is None:
        assert quats is not None and scales is not None, "need covars or quats + scales"
    means = means.contiguous()
    covars = covars.contiguous() if covars is not None else None
    quats = quats.contiguous() if quats is not None else None
    scales = scales.contiguous() if scales is not None else None
    viewmats = viewmats.contiguous()
    Ks = Ks.contiguous()
    N.require_cuda(means, covars, quats, scales, viewmats, Ks,
                   names=["means", "covars", "quats", "scales", "viewmats", "Ks"])
    if packed:
        _, camera_ids, gaussian_ids, radii, means2d, depths, conics, comps = \
            _FullyFusedProjectionPacked.apply(means, covars, quats, scales, viewmats, Ks, width,
                                              height, eps2d, near_plane, far_plane, radius_clip,
                                              sparse_grad, calc_compensations)
        return camera_ids, gaussian_ids, radii, means2d, depths, conics, comps
    return _FullyFusedProjection.apply(means, covars, quats, scales, viewmats, Ks, width, height,
                                       eps2d, near_plane, far_plane, radius_clip,
                                       calc_compensations)


# ---------------------------------------------------------------------------
# spherical_harmonics
# ---------------------------------------------------------------------------


class _SphericalHarmonics(torch.autograd.Function):
    @staticmethod
    def forward(ctx, degrees_to_use, dirs, coeffs, masks):
        n = dirs.numel() // 3
        K = coeffs.shape[-2]
        colors = torch.empty_like(dirs)
        N.call("tgs_compute_sh_fwd", n, K, int(degrees_to_use), N.ptr(dirs), N.ptr(coeffs),
               N.ptr(masks), N.ptr(colors), _stream())
        ctx.save_for_backward(dirs, coeffs, masks)
        ctx.degrees_to_use = int(degrees_to_use)
        return colors

    @staticmethod
    def backward(ctx, v_colors):
        dirs, coeffs, masks = ctx.saved_tensors
        n = dirs.numel() // 3
        K = coeffs.shape[-2]
        v_colors = v_colors.contiguous()
        v_coeffs = torch.empty_like(coeffs)
        v_dirs = torch.empty_like(dirs) if ctx.needs_input_grad[1] else None
        N.call("tgs_compute_sh_bwd", n, K, ctx.degrees_to_use, N.ptr(dirs), N.ptr(coeffs),
               N.ptr(masks), N.ptr(v_colors), N.ptr(v_coeffs), N.ptr(v_dirs), _stream())
        return None, v_dirs, v_coeffs, None


def spherical_harmonics(degrees_to_use: int, dirs: Tensor, coeffs: Tensor,
                        masks: Optional[Tensor] = None) -> Tensor:
    """Real SH colors up to ``degrees_to_use`` (gsplat spherical_harmonics).

    dirs [..., 3], coeffs [..., K, 3] -> colors [..., 3] (``engine.py:508-512``).
    """
    assert (degrees_to_use + 1) ** 2 <= coeffs.shape[-2], coeffs.shape
    assert dirs.shape[:-1] == coeffs.shape[:-2], (dirs.shape, coeffs.shape)
    assert dirs.shape[-1] == 3 and coeffs.shape[-1] == 3
    if masks is not None:
        assert masks.shape == dirs.shape[:-1], masks.shape
        masks = masks.contiguous().to(torch.bool).view(torch.uint8)
    dirs = dirs.contiguous()
    coeffs = coeffs.contiguous()
    N.require_cuda(dirs, coeffs, masks, names=["dirs", "coeffs", "masks"])
    return _SphericalHarmonics.apply(degrees_to_use, dirs, coeffs, masks)


# ---------------------------------------------------------------------------
# isect_tiles / isect_offset_encode
# ---------------------------------------------------------------------------


def _bit_width(v: int) -> int:
    return int(v).bit_length()


@torch.no_grad()
def isect_tiles(
    means2d: Tensor,
    radii: Tensor,
    depths: Tensor,
    tile_size: int,
    tile_width: int,
    tile_height: int,
    sort: bool = True,
    packed: bool = False,
    n_cameras: Optional[int] = None,
    camera_ids: Optional[Tensor] = None,
    gaussian_ids: Optional[Tensor] = None,
    double_buffer: bool = True,
) -> Tuple[Tensor, Tensor, Tensor]:
    """Gaussian-tile intersections sorted by (camera, tile, depth).

    Returns ``(tiles_per_gauss [C,N] or [nnz] i32, isect_ids [I] i64,
    flatten_ids [I] i32)``; bit-exact with gsplat's isect_tiles
    (``isect_tiles.cu:100-232``).
    """
    if packed:
        nnz = means2d.shape[0]
        assert n_cameras is not None and camera_ids is not None and gaussian_ids is not None
        C = int(n_cameras)
        total, Nn = nnz, 0
        cam_ids = camera_ids.contiguous().to(torch.int64)
    else:
        C, Nn = means2d.shape[0], means2d.shape[1]
        total = C * Nn
        cam_ids = None
    dev = means2d.device
    means2d = means2d.contiguous()
    radii = radii.contiguous()
    depths = depths.contiguous()
    N.require_cuda(means2d, radii, depths, cam_ids, names=["means2d", "radii", "depths", "camera_ids"])
    assert means2d.dtype == torch.float32 and depths.dtype == torch.float32
    assert radii.dtype == torch.int32

    n_tiles = tile_width * tile_height
    tile_n_bits = _bit_width(n_tiles)
    cam_n_bits = _bit_width(C)
    assert tile_n_bits + cam_n_bits <= 32, "camera and tile ids need more than 32 bits"
    s = _stream()
    tiles_per_gauss = torch.empty(radii.shape, dtype=torch.int32, device=dev)
    if total == 0:
        return (tiles_per_gauss, torch.empty(0, dtype=torch.int64, device=dev),
                torch.empty(0, dtype=torch.int32, device=dev))
    N.call("tgs_isect_tiles_count", total, N.ptr(means2d), N.ptr(radii), tile_size, tile_width,
           tile_height, N.ptr(tiles_per_gauss), s)
    cum = torch.empty(total, dtype=torch.int64, device=dev)
    ws = torch.empty(N.load().tgs_scan_workspace_size(total), dtype=torch.uint8, device=dev)
    N.call("tgs_inclusive_scan_i32_i64", N.ptr(tiles_per_gauss), N.ptr(cum), total, N.ptr(ws),
           ws.numel(), s)
    n_isects = int(cum[-1].item())
    isect_ids = torch.empty(n_isects, dtype=torch.int64, device=dev)
    flatten_ids = torch.empty(n_isects, dtype=torch.int32, device=dev)
    if n_isects:
        N.call("tgs_isect_tiles_emit", total, Nn, N.ptr(cam_ids), N.ptr(means2d), N.ptr(radii),
               N.ptr(depths), N.ptr(cum), tile_size, tile_width, tile_height, tile_n_bits,
               N.ptr(isect_ids), N.ptr(flatten_ids), s)
    if n_isects and sort:
        isect_ids, flatten_ids = radix_sort_pairs(isect_ids, flatten_ids,
                                                  end_bit=32 + tile_n_bits + cam_n_bits)
    return tiles_per_gauss, isect_ids, flatten_ids


def radix_sort_pairs(keys: Tensor, values: Tensor, begin_bit: int = 0,
                     end_bit: int = 64) -> Tuple[Tensor, Tensor]:
    """Stable ascending sort of int64 keys (on bits [begin_bit, end_bit)) with int32 values."""
    n = keys.numel()
    dev = keys.device
    k_alt = torch.empty_like(keys)
    v_alt = torch.empty_like(values)
    ws = torch.empty(max(1, N.load().tgs_radix_sort_workspace_size(n)), dtype=torch.uint8, device=dev)
    sel = ctypes.c_int(0)
    N.call("tgs_radix_sort_pairs", N.ptr(keys), N.ptr(values), N.ptr(k_alt), N.ptr(v_alt), n,
           begin_bit, end_bit, N.ptr(ws), ws.numel(), ctypes.byref(sel), _stream())
    return (k_alt, v_alt) if sel.value else (keys, values)


@torch.no_grad()
def isect_offset_encode(isect_ids: Tensor, n_cameras: int, tile_width: int,
                        tile_height: int) -> Tensor:
    """Per-(camera, tile) start offsets into the sorted intersections, [C, th, tw] i32."""
    isect_ids = isect_ids.contiguous()
    N.require_cuda(isect_ids, names=["isect_ids"])
    offsets = torch.empty((n_cameras, tile_height, tile_width), dtype=torch.int32,
                          device=isect_ids.device)
    N.call("tgs_isect_offset_encode", isect_ids.numel(), N.ptr(isect_ids), n_cameras,
           tile_width, tile_height, N.ptr(offsets), _stream())
    return offsets


# ---------------------------------------------------------------------------
# rasterize_to_pixels
# ---------------------------------------------------------------------------


def _packed_splats(means2d, conics, colors, opacities) -> Tensor:
    """gsplat's SoA splat tensors as the 48-byte records [n, 12] of the packed
    rasterizer kernels (one gather per staged Gaussian instead of four)."""
    n = opacities.numel()
    rec = torch.empty((max(n, 1), 12), dtype=torch.float32, device=means2d.device)
    N.call("tgs_pack_splats", n, N.ptr(means2d), N.ptr(conics), N.ptr(colors), N.ptr(opacities),
           N.ptr(rec), _stream())
    return rec


class _RasterizeToPixels(torch.autograd.Function):
    """3 channels at tile 16 without absgrad (TideGS's case) run the packed
    record kernels; every other shape runs the SoA kernels, other channel
    counts zero-padded to an instantiated one.  Above 32 channels the kernels
    run once per run of 32 channels: compositing (T, alphas, last ids) is the
    same in every launch, the colour outputs and gradients are per launch, and
    the geometry gradients, linear in each channel's share of dL/dalpha,
    accumulate over the launches (dL/dalpha and the background term enter
    the first launch only).  ``masks`` [C, tile rows, tile columns] (False =
    skip the tile): the tile's pixels take the background (or zero) with
    alpha 0 and pass no gradient."""

    @staticmethod
    def forward(ctx, means2d, conics, colors, opacities, backgrounds, width, height, tile_size,
                isect_offsets, flatten_ids, absgrad, masks):
        C = isect_offsets.shape[0]
        th, tw = isect_offsets.shape[1], isect_offsets.shape[2]
        ch = colors.shape[-1]
        dev = means2d.device
        render_alphas = torch.empty((C, height, width, 1), dtype=torch.float32, device=dev)
        last_ids = torch.empty((C, height, width), dtype=torch.int32, device=dev)
        records = None
        if ch == 3 and tile_size == 16 and not absgrad:
            render_colors = torch.empty((C, height, width, ch), dtype=torch.float32, device=dev)
            records = _packed_splats(means2d, conics, colors, opacities)
            N.call("tgs_tide_rasterize_fwd", C, N.ptr(records), N.ptr(backgrounds), width, height,
                   tw, th, N.ptr(isect_offsets), N.ptr(flatten_ids), flatten_ids.numel(),
                   N.ptr(render_colors), N.ptr(render_alphas), N.ptr(last_ids), None, None, 0,
                   _stream())
        else:
            outs = []
            for s0, w, cw in _channel_chunks(ch):
                col = _pad_last(colors[..., s0:s0 + w], cw)
                bg = _pad_last(backgrounds[:, s0:s0 + w], cw) if backgrounds is not None else None
                rc = torch.empty((C, height, width, cw), dtype=torch.float32, device=dev)
                N.call("tgs_rasterize_to_pixels_fwd", C, cw, N.ptr(means2d), N.ptr(conics),
                       N.ptr(col), N.ptr(opacities), N.ptr(bg), width, height, tile_size,
                       tw, th, N.ptr(isect_offsets), N.ptr(flatten_ids), flatten_ids.numel(),
                       N.ptr(rc), N.ptr(render_alphas), N.ptr(last_ids), _stream())
                outs.append(rc if cw == w else rc[..., :w])
            render_colors = outs[0] if len(outs) == 1 else torch.cat(outs, -1)
            render_colors = render_colors.contiguous()
        kernel_alphas = render_alphas
        pmask = None
        if masks is not None:
            pmask = _pixel_mask(masks, tile_size, height, width)
            fill = (backgrounds[:, None, None, :] if backgrounds is not None
                    else torch.zeros((), dtype=torch.float32, device=dev))
            render_colors = torch.where(pmask[..., None], render_colors, fill)
            render_alphas = torch.where(pmask[..., None], render_alphas,
                                        torch.zeros((), dtype=torch.float32, device=dev))
        ctx.save_for_backward(means2d, conics, colors, opacities, backgrounds, isect_offsets,
                              flatten_ids, kernel_alphas, render_alphas, last_ids, records, pmask)
        ctx.width, ctx.height, ctx.tile_size, ctx.absgrad = width, height, tile_size, absgrad
        return render_colors, render_alphas

    @staticmethod
    def backward(ctx, v_render_colors, v_render_alphas):
        (means2d, conics, colors, opacities, backgrounds, isect_offsets, flatten_ids,
         render_alphas, out_alphas, last_ids, records, pmask) = ctx.saved_tensors
        C = isect_offsets.shape[0]
        th, tw = isect_offsets.shape[1], isect_offsets.shape[2]
        ch = colors.shape[-1]
        v_render_colors = (torch.zeros((C, ctx.height, ctx.width, ch), device=means2d.device)
                           if v_render_colors is None else v_render_colors.contiguous())
        v_out_colors = v_render_colors
        v_render_alphas = None if v_render_alphas is None else v_render_alphas.contiguous()
        if pmask is not None:
            # a skipped tile's pixels do not depend on the Gaussians
            v_render_colors = (v_render_colors * pmask[..., None]).contiguous()
            if v_render_alphas is not None:
                v_render_alphas = (v_render_alphas * pmask[..., None]).contiguous()
        v_means2d = torch.zeros_like(means2d)
        v_conics = torch.zeros_like(conics)
        v_colors = torch.zeros_like(colors)
        v_opacities = torch.zeros_like(opacities)
        v_abs = torch.zeros_like(means2d) if ctx.absgrad else None
        if records is not None:
            n = opacities.numel()
            grads = torch.zeros((max(n, 1), 9), dtype=torch.float32, device=means2d.device)
            N.call("tgs_tide_rasterize_bwd", C, N.ptr(records), N.ptr(backgrounds), ctx.width,
                   ctx.height, tw, th, N.ptr(isect_offsets), N.ptr(flatten_ids),
                   flatten_ids.numel(), N.ptr(render_alphas), N.ptr(last_ids),
                   N.ptr(v_render_colors), N.ptr(v_render_alphas), N.ptr(grads), _stream())
            N.call("tgs_unpack_splat_grads", n, N.ptr(grads), N.ptr(v_means2d), N.ptr(v_conics),
                   N.ptr(v_colors), N.ptr(v_opacities), _stream())
        else:
            for j, (s0, w, cw) in enumerate(_channel_chunks(ch)):
                col = _pad_last(colors[..., s0:s0 + w], cw)
                bg = _pad_last(backgrounds[:, s0:s0 + w], cw) if backgrounds is not None else None
                vrc = _pad_last(v_render_colors[..., s0:s0 + w], cw)
                vcol = v_colors if cw == ch else torch.zeros(
                    (*colors.shape[:-1], cw), dtype=torch.float32, device=means2d.device)
                N.call("tgs_rasterize_to_pixels_bwd", C, cw, N.ptr(means2d), N.ptr(conics),
                       N.ptr(col), N.ptr(opacities), N.ptr(bg), ctx.width, ctx.height,
                       ctx.tile_size, tw, th, N.ptr(isect_offsets), N.ptr(flatten_ids),
                       flatten_ids.numel(), N.ptr(render_alphas), N.ptr(last_ids),
                       N.ptr(vrc), N.ptr(v_render_alphas if j == 0 else None), N.ptr(v_abs),
                       N.ptr(v_means2d), N.ptr(v_conics), N.ptr(vcol), N.ptr(v_opacities),
                       _stream())
                if vcol is not v_colors:
                    v_colors[..., s0:s0 + w] = vcol[..., :w]
        if ctx.absgrad:
            ctx.saved_tensors[0].absgrad = v_abs
        v_backgrounds = None
        if ctx.needs_input_grad[4]:
            v_backgrounds = (v_out_colors * (1.0 - out_alphas)).sum(dim=(1, 2))
        return (v_means2d, v_conics, v_colors, v_opacities, v_backgrounds, None, None, None,
                None, None, None, None)


def rasterize_to_pixels(
    means2d: Tensor,
    conics: Tensor,
    colors: Tensor,
    opacities: Tensor,
    image_width: int,
    image_height: int,
    tile_size: int,
    isect_offsets: Tensor,
    flatten_ids: Tensor,
    backgrounds: Optional[Tensor] = None,
    masks: Optional[Tensor] = None,
    packed: bool = False,
    absgrad: bool = False,
) -> Tuple[Tensor, Tensor]:
    """Alpha-composite sorted Gaussians into pixels (gsplat rasterize_to_pixels).

    Returns ``(render_colors [C,H,W,D], render_alphas [C,H,W,1])``
    (``engine.py:550-561``).  Any channel count: up to 32 the kernels run at the
    next instantiated count (zero-padded channels, sliced back), above 32 once
    per run of 32 channels (the reference instantiates 1-5, 8, 9, 16, 17, 32,
    33, ... 512, 513: ``rasterize_to_pixels_fwd.cu:261-283``).  ``masks``
    [C, tile rows, tile columns]: tiles marked False render the background
    with alpha 0 and pass no gradient.
    """
    C = isect_offsets.shape[0]
    ch = colors.shape[-1]
    if packed:
        assert means2d.dim() == 2 and colors.dim() == 2
    else:
        assert means2d.shape[0] == C and colors.shape[:2] == means2d.shape[:2]
    if backgrounds is not None:
        assert backgrounds.shape == (C, ch), backgrounds.shape
    if absgrad and ch > _CHUNK:
        # |dL/dmean2d| per pixel needs every channel's share of dL/dalpha at once
        raise NotImplementedError("rasterize_to_pixels: absgrad with more than 32 channels")
    tile_width = math.ceil(image_width / float(tile_size))
    tile_height = math.ceil(image_height / float(tile_size))
    assert isect_offsets.shape == (C, tile_height, tile_width), isect_offsets.shape
    if masks is not None:
        assert masks.shape == (C, tile_height, tile_width), masks.shape
        masks = masks.to(means2d.device)
    means2d, conics, colors, opacities = (t.contiguous() for t in (means2d, conics, colors, opacities))
    backgrounds = backgrounds.contiguous() if backgrounds is not None else None
    isect_offsets = isect_offsets.contiguous()
    flatten_ids = flatten_ids.contiguous()
    N.require_cuda(means2d, conics, colors, opacities, backgrounds, isect_offsets, flatten_ids,
                   names=["means2d", "conics", "colors", "opacities", "backgrounds",
                          "isect_offsets", "flatten_ids"])
    return _RasterizeToPixels.apply(
        means2d, conics, colors, opacities, backgrounds, int(image_width), int(image_height),
        int(tile_size), isect_offsets, flatten_ids, absgrad, masks)
