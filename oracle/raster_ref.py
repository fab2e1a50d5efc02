"""CPU restatement of gsplat's tile intersection and tile rasterizer.

Test oracle only (see ``oracle/__init__.py``).

* ``isect_tiles`` / ``isect_offset_encode``: numpy restatement of
  ``gsplat/cuda/csrc/isect_tiles.cu:14-98`` (tile rect, key layout), ``:150-227``
  (count, cumsum, emit, stable radix sort on bits [0, 32+tile_bits+cam_bits))
  and ``:234-301`` (offset encode).  The sort is ``np.argsort(kind="stable")``
  on the masked key.  Pinned by a brute-force per-tile enumeration in
  tests/test_oracle_raster.py.
* ``rasterize_fwd`` / ``rasterize_bwd``: ctypes wrappers of ``raster_ref.c``
  (restating ``rasterize_to_pixels_fwd.cu:14-160`` / ``_bwd.cu:14-249``).
  Pinned by a tile-free brute-force compositor and by finite differences of
  the float64 forward.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np

_LIB = None


def _lib():
    global _LIB
    if _LIB is None:
        path = Path(__file__).resolve().parent / "_build" / "liboracle.so"
        if not path.exists():
            from . import build as _b
            _b.build()
        lib = ctypes.CDLL(str(path))
        _LIB = lib
    return _LIB


def bit_width(v: int) -> int:
    return int(v).bit_length()


def tile_rect(means2d: np.ndarray, radii: np.ndarray, tile_size: int, tw: int, th: int):
    """Per-entry [x0, x1) x [y0, y1) tile ranges in float32 arithmetic (isect_tiles.cu:55-64)."""
    ts = np.float32(tile_size)
    r = radii.astype(np.float32) / ts
    tx = means2d[..., 0].astype(np.float32) / ts
    ty = means2d[..., 1].astype(np.float32) / ts

    def clamp(v, lim):
        v = np.where(np.isnan(v), 0, v)
        return np.clip(v, 0, lim).astype(np.int64)

    x0 = clamp(np.floor(tx - r), tw)
    y0 = clamp(np.floor(ty - r), th)
    x1 = clamp(np.ceil(tx + r), tw)
    y1 = clamp(np.ceil(ty + r), th)
    return x0, y0, x1, y1


def isect_tiles(means2d, radii, depths, tile_size, tw, th, sort=True, camera_ids=None):
    """Returns (tiles_per_gauss i32, isect_ids i64, flatten_ids i32).

    Non-packed inputs are [C,N,*]; packed inputs are [nnz,*] with ``camera_ids``.
    """
    means2d = np.asarray(means2d, dtype=np.float32)
    radii = np.asarray(radii, dtype=np.int32)
    depths = np.asarray(depths, dtype=np.float32)
    if camera_ids is None:
        C, N = radii.shape
        cams = np.repeat(np.arange(C, dtype=np.int64), N)
    else:
        cams = np.asarray(camera_ids, dtype=np.int64)
        C = int(cams.max()) + 1 if cams.size else 1
    flat_m = means2d.reshape(-1, 2)
    flat_r = radii.reshape(-1)
    flat_d = depths.reshape(-1)
    x0, y0, x1, y1 = tile_rect(flat_m, flat_r, tile_size, tw, th)
    live = flat_r > 0
    nx = np.where(live, np.maximum(x1 - x0, 0), 0)
    ny = np.where(live, np.maximum(y1 - y0, 0), 0)
    tiles = (nx * ny).astype(np.int32)
    n_tiles = tw * th
    tile_bits = bit_width(n_tiles)
    cam_bits = bit_width(C if camera_ids is None else max(C, 1))
    total = int(tiles.astype(np.int64).sum())
    depth_bits = flat_d.view(np.int32).astype(np.int64)  # sign-extended, as the reference
    # Emission in entry order, row-major over each entry's tile rectangle.
    live_idx = np.nonzero(tiles)[0]
    cnt = tiles[live_idx].astype(np.int64)
    owner = np.repeat(live_idx, cnt)
    start = np.repeat(np.cumsum(cnt) - cnt, cnt)
    local = np.arange(total, dtype=np.int64) - start
    width = nx[owner].astype(np.int64)
    ty_ = y0[owner] + local // np.maximum(width, 1)
    tx_ = x0[owner] + local % np.maximum(width, 1)
    tid = ty_ * tw + tx_
    isect_ids = (cams[owner] << (32 + tile_bits)) | (tid << 32) | depth_bits[owner]
    flatten_ids = owner.astype(np.int32)
    if sort and total:
        end_bit = 32 + tile_bits + cam_bits
        mask = np.int64(-1) if end_bit >= 64 else np.int64((1 << end_bit) - 1)
        order = np.argsort(isect_ids & mask, kind="stable")
        isect_ids = isect_ids[order]
        flatten_ids = flatten_ids[order]
    return tiles.reshape(radii.shape), isect_ids, flatten_ids


def isect_offset_encode(isect_ids, C, tw, th):
    """offsets[c, tile] = first index of the (c, tile) run; empty tiles take the
    next run start; trailing tiles take n (isect_tiles.cu:234-301)."""
    n_tiles = tw * th
    tile_bits = bit_width(n_tiles)
    isect_ids = np.asarray(isect_ids, dtype=np.int64)
    hi = isect_ids >> 32
    ids = (hi >> tile_bits) * n_tiles + (hi & ((1 << tile_bits) - 1))
    total = C * n_tiles
    # offsets[b] = number of intersections whose bucket id < b
    offsets = np.searchsorted(ids, np.arange(total), side="left").astype(np.int32)
    return offsets.reshape(C, th, tw)


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p) if a is not None else None


def rasterize_fwd(means2d, conics, colors, opac, W, H, tile_size, offsets, flatten_ids,
                  backgrounds=None, dtype=np.float32):
    """Returns (colors [C,H,W,D], alphas [C,H,W], last_ids [C,H,W])."""
    suffix = "f32" if dtype == np.float32 else "f64"
    cvt = lambda a: None if a is None else np.ascontiguousarray(a, dtype=dtype)  # noqa: E731
    means2d, conics, colors, opac, backgrounds = map(cvt, (means2d, conics, colors, opac, backgrounds))
    offsets = np.ascontiguousarray(offsets, dtype=np.int32)
    flatten_ids = np.ascontiguousarray(flatten_ids, dtype=np.int32)
    C, th, tw = offsets.shape
    D = colors.shape[-1]
    assert D <= 513
    out_c = np.zeros((C, H, W, D), dtype=dtype)
    out_a = np.zeros((C, H, W), dtype=dtype)
    last = np.zeros((C, H, W), dtype=np.int32)
    fn = getattr(_lib(), f"oracle_raster_fwd_{suffix}")
    fn.restype = None
    fn(ctypes.c_int(C), ctypes.c_int(D), _p(means2d), _p(conics), _p(colors), _p(opac),
       _p(backgrounds), ctypes.c_int(W), ctypes.c_int(H), ctypes.c_int(tile_size), ctypes.c_int(tw),
       ctypes.c_int(th), _p(offsets), _p(flatten_ids), ctypes.c_int(flatten_ids.size), _p(out_c),
       _p(out_a), _p(last))
    return out_c, out_a, last


def rasterize_bwd(means2d, conics, colors, opac, W, H, tile_size, offsets, flatten_ids,
                  alphas, last_ids, v_colors, v_alphas=None, backgrounds=None, absgrad=False,
                  dtype=np.float32):
    """Returns float64 (v_means2d, v_conics, v_colors, v_opac, v_abs|None)."""
    suffix = "f32" if dtype == np.float32 else "f64"
    cvt = lambda a: None if a is None else np.ascontiguousarray(a, dtype=dtype)  # noqa: E731
    means2d, conics, colors, opac, backgrounds, alphas, v_colors, v_alphas = map(
        cvt, (means2d, conics, colors, opac, backgrounds, alphas, v_colors, v_alphas))
    offsets = np.ascontiguousarray(offsets, dtype=np.int32)
    flatten_ids = np.ascontiguousarray(flatten_ids, dtype=np.int32)
    last_ids = np.ascontiguousarray(last_ids, dtype=np.int32)
    C, th, tw = offsets.shape
    D = colors.shape[-1]
    vm = np.zeros(means2d.shape, dtype=np.float64)
    vc = np.zeros(conics.shape, dtype=np.float64)
    vcol = np.zeros(colors.shape, dtype=np.float64)
    vo = np.zeros(opac.shape, dtype=np.float64)
    va = np.zeros(means2d.shape, dtype=np.float64) if absgrad else None
    fn = getattr(_lib(), f"oracle_raster_bwd_{suffix}")
    fn.restype = None
    fn(ctypes.c_int(C), ctypes.c_int(D), _p(means2d), _p(conics), _p(colors), _p(opac),
       _p(backgrounds), ctypes.c_int(W), ctypes.c_int(H), ctypes.c_int(tile_size), ctypes.c_int(tw),
       ctypes.c_int(th), _p(offsets), _p(flatten_ids), ctypes.c_int(flatten_ids.size), _p(alphas),
       _p(last_ids), _p(v_colors), _p(v_alphas), _p(vm), _p(vc), _p(vcol), _p(vo), _p(va))
    return vm, vc, vcol, vo, va


def decision_flips(splats_a, splats_b, W, H, tile_size, offsets, flatten_ids,
                   dtype=np.float32, mark=None):
    """Compositing decisions (alpha >= 1/255, the T <= 1e-4 stop) that differ
    between two parameter sets of the same entries over the same intersection
    lists.  ``splats_*`` = (means2d [*,2], conics [*,3], opacities [*]).
    Returns (flipped pixels [C,H,W] bool, entries composited under either set
    at a flipped pixel or at a pixel of ``mark`` [C,H,W] bool)."""
    suffix = "f32" if dtype == np.float32 else "f64"
    cvt = lambda a: np.ascontiguousarray(a, dtype=dtype)  # noqa: E731
    ma, ca, oa = map(cvt, splats_a)
    mb, cb, ob = map(cvt, splats_b)
    assert ma.shape == mb.shape and ca.shape == cb.shape and oa.shape == ob.shape
    offsets = np.ascontiguousarray(offsets, dtype=np.int32)
    flatten_ids = np.ascontiguousarray(flatten_ids, dtype=np.int32)
    C, th, tw = offsets.shape
    flip = np.zeros((C, H, W), dtype=np.uint8)
    flag = np.zeros(oa.shape[0], dtype=np.uint8)
    mark = None if mark is None else np.ascontiguousarray(mark, dtype=np.uint8)
    assert mark is None or mark.shape == (C, H, W)
    fn = getattr(_lib(), f"oracle_raster_decision_flips_{suffix}")
    fn.restype = None
    fn(ctypes.c_int(C), _p(ma), _p(ca), _p(oa), _p(mb), _p(cb), _p(ob), ctypes.c_int(W),
       ctypes.c_int(H), ctypes.c_int(tile_size), ctypes.c_int(tw), ctypes.c_int(th),
       _p(offsets), _p(flatten_ids), ctypes.c_int(flatten_ids.size), _p(mark), _p(flip),
       _p(flag))
    return flip.astype(bool), flag.astype(bool)
