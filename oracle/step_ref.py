"""CPU restatement of one TideGS training batch on a resident table.

Test oracle and CPU baseline only (see ``oracle/__init__.py``).  Follows the
reference's per-camera loop literally:

* filters: packed projection per camera, ascending Gaussian ids
  (``strategies/base_engine.py:329-425`` over
  ``gsplat/cuda/csrc/fully_fused_projection_packed_fwd.cu:19-131``)
* touched rows: union of the filters (``engine.py:1801-1827``)
* per camera (``engine.py:2255-2311`` -> ``pipeline_forward_one_step_shs_inplace``
  ``engine.py:458-571``): activations (``base_gaussian_model.py:35-50``),
  non-packed projection, SH colours ``clamp_min(sh + 0.5, 0)``, isect + sort,
  rasterize, loss ``0.8 L1 + 0.2 (1 - SSIM)`` (``base_engine.py:464-488``),
  then the backward of all of it and ``scatter_add_`` into the compact rows
  in camera order (``engine.py:2434-2469``).
* optional resident Adam of the touched rows (``oracle/optim_ref.py``).

Every piece is a function of the other oracle modules, each pinned in
tests/test_oracle_*.py; this module only composes them.
"""
from __future__ import annotations

import types

import numpy as np
import torch

from . import gsplat_ref as G
from . import raster_ref as R
from . import ssim_ref as S


def _split(params: torch.Tensor):
    xyz = params[:, 0:3]
    logs = params[:, 3:6]
    q = params[:, 6:10]
    logit = params[:, 10]
    sh = params[:, 11:59].reshape(-1, 16, 3)
    return xyz, logs, q, logit, sh


def packed_filters(params, viewmats, Ks, W, H, eps2d=0.3, near=0.01, far=1e10, radius_clip=0.0,
                   dtype=torch.float64):
    """Per-camera ascending row ids visible under the packed-projection rule.

    A row is in camera c's filter when gsplat's packed projection keeps it
    (``fully_fused_projection_packed_fwd.cu:50-131``, consumed as the filter at
    ``base_engine.py:329-425``): the radius of ``gsplat_ref.project_fwd(...,
    packed=True)`` is positive.  The rows' activations are TideGS's
    (``base_gaussian_model.py:35-50``: ``exp`` of the log-scales, the
    quaternion normalised as ``q / max(|q|, 1e-12)``)."""
    xyz, logs, q, _, _ = _split(params.to(dtype))
    qn = q / torch.clamp(q.norm(dim=-1, keepdim=True), min=1e-12)
    radii = G.project_fwd(xyz, qn, torch.exp(logs), viewmats, Ks, W, H, eps2d=eps2d,
                          near_plane=near, far_plane=far, radius_clip=radius_clip, dtype=dtype,
                          packed=True)[0]
    return [torch.nonzero(radii[c] > 0).flatten() for c in range(radii.shape[0])]


def packed_filter_ambiguous(params, viewmats, Ks, W, H, eps2d=0.3, near=0.01, far=1e10,
                            radius_clip=0.0, rel=2e-5):
    """[C, N] bool: entries whose packed-filter decision sits within float32
    rounding of a boundary, evaluated in float64.

    The GPU evaluates the rule in float32; the oracle in float64.  Far from a
    boundary both give the same decision; within a relative ``rel`` of one they
    may not.  An entry is flagged when any of these holds:

    * ``z`` within ``rel * (|p| + |t|)`` of the near or far plane;
    * ``det`` of the blurred covariance within ``rel * a d`` of zero;
    * ``3 sqrt(v1)`` within a relative ``rel`` of an integer (the radius, a
      ceiling, may then be one larger or smaller), where that changes the
      radius-clip or image-border decision;
    * the mean within ``rel`` (relative to its pixel magnitude) of flipping an
      image-border test at either candidate radius.

    Any difference between the GPU's filters and ``packed_filters`` must lie
    inside this set; ``tests/test_oracle_step.py`` checks that float32
    evaluations of the rule only ever differ from float64 there."""
    f64 = torch.float64
    xyz, logs, q, _, _ = _split(params.to(f64))
    qn = q / torch.clamp(q.norm(dim=-1, keepdim=True), min=1e-12)
    Sigma = G.covar_from_quat_scale(qn, torch.exp(logs))
    vm, Kd = viewmats.to(f64), Ks.to(f64)
    pc, m2d, a, b, d, det, _, _ = G.project_core(xyz, Sigma, vm, Kd, W, H, eps2d)
    z = pc[..., 2]
    scale_z = xyz.abs().sum(-1)[None] + vm[:, :3, 3].abs().sum(-1)[:, None] + 1.0
    amb = ((z - near).abs() <= rel * scale_z) | ((z - far).abs() <= rel * scale_z)
    amb |= det.abs() <= rel * (a * d).abs()
    bb = 0.5 * (a + d)
    v1 = bb + torch.sqrt(torch.clamp(bb * bb - det, min=0.1))
    rr = 3.0 * torch.sqrt(v1)
    r_lo = torch.ceil(rr * (1 - rel))
    r_hi = torch.ceil(rr * (1 + rel))
    fx, fy = Kd[:, 0, 0][:, None], Kd[:, 1, 1][:, None]
    cx, cy = Kd[:, 0, 2][:, None], Kd[:, 1, 2][:, None]
    tol_x = rel * ((m2d[..., 0] - cx).abs() + cx.abs() + 1.0)
    tol_y = rel * ((m2d[..., 1] - cy).abs() + cy.abs() + 1.0)
    outcomes = []
    for r in (r_lo, r_hi):
        for sx in (-1.0, 1.0):
            for sy in (-1.0, 1.0):
                mx = m2d[..., 0] + sx * tol_x
                my = m2d[..., 1] + sy * tol_y
                out = (mx + r <= 0) | (mx - r >= W) | (my + r <= 0) | (my - r >= H)
                outcomes.append(out | (r <= radius_clip))
    stack = torch.stack(outcomes)
    amb |= stack.any(0) != stack.all(0)
    return amb & torch.isfinite(rr)


def render_projection(params, rows, viewmat, K, W, H, eps2d=0.3, dtype=torch.float64):
    """The render projection of ``rows`` for one camera (gsplat non-packed
    rule, ``fully_fused_projection_fwd.cu:18-129``) with TideGS's activations:
    (radii [n], means2d [n,2], depths [n], 3 sqrt(v1) before the ceiling [n])."""
    p = params[rows].to(dtype)
    xyz, logs, q, _, _ = _split(p)
    qn = q / torch.clamp(q.norm(dim=-1, keepdim=True), min=1e-12)
    radii, m2d, depths, _, _ = G.project_fwd(xyz, qn, torch.exp(logs), viewmat[None].to(dtype),
                                             K[None].to(dtype), W, H, eps2d=eps2d, dtype=dtype)
    Sigma = G.covar_from_quat_scale(qn, torch.exp(logs))
    _, _, a, _, d, det, _, _ = G.project_core(xyz, Sigma, viewmat[None].to(dtype),
                                              K[None].to(dtype), W, H, eps2d)
    bb = 0.5 * (a + d)
    rr = 3.0 * torch.sqrt(bb + torch.sqrt(torch.clamp(bb * bb - det, min=0.01)))
    return radii[0], m2d[0], depths[0], rr[0]


def _render_entries(params, rows, viewmat, K, W, H, sh_degree, dtype):
    """Forward values of one camera's entries: TideGS's activations
    (``base_gaussian_model.py:35-50``), the render projection
    (``fully_fused_projection_fwd.cu:18-129``) and the SH colours
    ``clamp_min(sh + 0.5, 0)`` (``engine.py:508-512``)."""
    p = params[rows].to(dtype)
    xyz, logs, q, logit, sh = _split(p)
    f = types.SimpleNamespace(xyz=xyz, sh=sh)
    f.qnorm = torch.clamp(q.norm(dim=-1, keepdim=True), min=1e-12)
    f.qn = q / f.qnorm
    f.scales = torch.exp(logs)
    f.opac = torch.sigmoid(logit)
    f.vm, f.K = viewmat[None].to(dtype), K[None].to(dtype)
    f.radii, f.m2d, f.depths, f.conics, _ = G.project_fwd(xyz, f.qn, f.scales, f.vm, f.K, W, H,
                                                          dtype=dtype)
    campos = torch.linalg.inv(viewmat.to(torch.float64))[:3, 3].to(dtype)
    f.dirs = xyz - campos
    f.col_pre = G.sh_fwd(sh_degree, f.dirs, sh, dtype=dtype)
    f.colors = torch.clamp(f.col_pre + 0.5, min=0.0)
    return f


def _entry_backward(f, W, H, v_means2d, v_conics, v_colors, v_opacities, sh_degree, dtype):
    vm2 = torch.as_tensor(np.asarray(v_means2d)).to(dtype).reshape(-1, 2)
    vcon = torch.as_tensor(np.asarray(v_conics)).to(dtype).reshape(-1, 3)
    vcol = torch.as_tensor(np.asarray(v_colors)).to(dtype).reshape(-1, 3) * (f.col_pre + 0.5 >= 0)
    vop = torch.as_tensor(np.asarray(v_opacities)).to(dtype).reshape(-1)
    v_sh, v_dirs = G.sh_bwd(sh_degree, f.dirs, f.sh, vcol, dtype=dtype)
    v_xyz, v_qn, v_s, _, _ = G.project_bwd(f.xyz, f.qn, f.scales, f.vm, f.K, W, H, 0.3, f.radii,
                                           f.conics, vm2[None], None, vcon[None], dtype=dtype)
    g = torch.zeros((f.xyz.shape[0], 59), dtype=dtype)
    g[:, 0:3] = v_xyz + v_dirs
    g[:, 3:6] = v_s * f.scales
    g[:, 6:10] = (v_qn - (v_qn * f.qn).sum(-1, keepdim=True) * f.qn) / f.qnorm
    g[:, 10] = vop * f.opac * (1 - f.opac)
    g[:, 11:59] = v_sh.reshape(-1, 48)
    return g


def entry_backward(params, rows, viewmat, K, W, H, v_means2d, v_conics, v_colors, v_opacities,
                   sh_degree=3, dtype=torch.float64):
    """Row gradients [len(rows), 59] (table column order, w.r.t. the raw
    parameters) of one camera's entries from their splat gradients: the
    backward of the render projection (``fully_fused_projection_bwd.cu``), of
    the SH colours with their clamp (``compute_sh_bwd.cu``) and of TideGS's
    activations (``engine.py:2434-2469``)."""
    f = _render_entries(params, rows, viewmat, K, W, H, sh_degree, dtype)
    return _entry_backward(f, W, H, v_means2d, v_conics, v_colors, v_opacities, sh_degree, dtype)


def camera_step(params, rows, viewmat, K, gt, W, H, sh_degree=3, background=None, tile=16,
                lambda_dssim=0.2, proj_dtype=torch.float64, raster_dtype=np.float32,
                isect_inputs=None):
    """Forward + backward of one camera on the gathered rows.

    Returns (loss, image [H,W,3], grads [len(rows), 59]) with grads in the
    table's column order (w.r.t. the raw parameters, through the activations).

    ``isect_inputs`` = (means2d float32 [n,2], radii [n], depths float32 [n])
    replaces the projection's values in the intersection step only (tile
    rectangles and the depth-bit sort keys, ``isect_tiles.cu:55-92``), so that
    the index work runs on another implementation's float32 values: two
    float32 evaluations of a depth may differ in the last bit, and that
    reorders near-tied overlapping Gaussians.
    """
    f = _render_entries(params, rows, viewmat, K, W, H, sh_degree, proj_dtype)
    tw, th = -(-W // tile), -(-H // tile)
    if isect_inputs is None:
        i_m2d, i_radii, i_depths = (f.m2d.to(torch.float32).numpy(), f.radii.numpy(),
                                    f.depths.to(torch.float32).numpy())
    else:
        i_m2d, i_radii, i_depths = (np.asarray(x) for x in isect_inputs)
        i_m2d = i_m2d.astype(np.float32).reshape(1, -1, 2)
        i_radii = i_radii.astype(np.int32).reshape(1, -1)
        i_depths = i_depths.astype(np.float32).reshape(1, -1)
    _, ids, flat = R.isect_tiles(i_m2d, i_radii, i_depths, tile, tw, th)
    offs = R.isect_offset_encode(ids, 1, tw, th)
    bg = None if background is None else np.asarray(background, np.float64)[None]
    splat = (f.m2d.numpy().reshape(-1, 2), f.conics[0].numpy(), f.colors.numpy(),
             f.opac.numpy())
    img, alphas, last = R.rasterize_fwd(*splat, W, H, tile, offs, flat, backgrounds=bg,
                                        dtype=raster_dtype)
    loss, v_img = S.tide_loss(img[0].transpose(2, 0, 1), gt.numpy(), lambda_dssim=lambda_dssim,
                              dtype=np.float64)
    v_hwc = np.ascontiguousarray(v_img.transpose(1, 2, 0))[None]
    vm2, vcon, vcol, vop, _ = R.rasterize_bwd(*splat, W, H, tile, offs, flat, alphas, last,
                                              v_hwc, backgrounds=bg, dtype=raster_dtype)
    g = _entry_backward(f, W, H, vm2, vcon, vcol, vop, sh_degree, proj_dtype)
    return loss, img[0], g


def batch_grads(params, viewmats, Ks, gts, W, H, sh_degree=3, backgrounds=None,
                proj_dtype=torch.float64, raster_dtype=np.float32, lambda_dssim=0.2,
                filters=None, isect_inputs=None):
    """touched rows [T], compact grads [T,59], per-camera losses and images.

    ``filters`` (per-camera ascending row ids) replaces the packed-filter
    evaluation and ``isect_inputs`` (per camera, see camera_step) the values
    the intersection step sorts on, so that a caller can run the rest of the
    batch on exactly the index decisions another implementation made
    (identical inputs)."""
    if filters is None:
        filters = packed_filters(params, viewmats, Ks, W, H)
    filters = [torch.as_tensor(f, dtype=torch.long) for f in filters]
    touched = torch.unique(torch.cat(filters)) if filters else torch.empty(0, dtype=torch.long)
    grads = torch.zeros((touched.numel(), 59), dtype=proj_dtype)
    losses, images = [], []
    for c, rows in enumerate(filters):
        if rows.numel() == 0:
            losses.append(None)
            images.append(None)
            continue
        bg = None if backgrounds is None else backgrounds[c]
        loss, img, g = camera_step(params, rows, viewmats[c], Ks[c], gts[c], W, H, sh_degree,
                                   background=bg, lambda_dssim=lambda_dssim,
                                   proj_dtype=proj_dtype, raster_dtype=raster_dtype,
                                   isect_inputs=None if isect_inputs is None else isect_inputs[c])
        idx = torch.searchsorted(touched, rows)
        grads.index_add_(0, idx, g)
        losses.append(loss)
        images.append(img)
    return touched, grads, losses, images, filters


def batch_row_grads(params, viewmats, Ks, W, H, filters, splat_grads, sh_degree=3,
                    dtype=torch.float64):
    """touched rows [T] and compact row gradients [T,59] of a batch from given
    per-camera splat gradients ``splat_grads[c] = (v_means2d [n,2], v_conics
    [n,3], v_colors [n,3], v_opacities [n])`` over ``filters[c]``, summed in
    camera order as ``scatter_add_`` does (``engine.py:2434-2469``)."""
    filters = [torch.as_tensor(f, dtype=torch.long) for f in filters]
    touched = torch.unique(torch.cat(filters)) if filters else torch.empty(0, dtype=torch.long)
    grads = torch.zeros((touched.numel(), 59), dtype=dtype)
    for c, rows in enumerate(filters):
        if rows.numel():
            g = entry_backward(params, rows, viewmats[c], Ks[c], W, H, *splat_grads[c],
                               sh_degree=sh_degree, dtype=dtype)
            grads.index_add_(0, torch.searchsorted(touched, rows), g)
    return touched, grads
