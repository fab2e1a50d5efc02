"""CPU restatement of TideGS's streaming PLY -> base-file initializer.

Test oracle only (see ``oracle/__init__.py``).

Follows ``storage/streaming_ply_init.py`` pass by pass, with the bucket files
kept as in-memory record lists (same append order, same names-sorted bucket
order):

* ``morton_codes``        - ``_morton_codes_np`` (:154-168)
* ``rgb_to_sh``           - ``_rgb_to_sh`` (:202-231), per chunk
* ``pack_rows``           - ``_pack_gaussian_rows`` (:234-248)
* ``estimate_log_scale`` / ``bucket_log_scale`` (:171-192)
* ``update_block_bounds`` (:299-316)
* ``build_base``          - passes 1-3 of ``streaming_ply_to_ssd_base`` (:541-651)
  with the recursion of ``_sort_bucket_to_base`` / ``_sort_large_bucket_to_base``
  / ``_stream_equal_key_bucket_to_base`` (:319-538)

Pinned by tests/test_oracle_streaming_init.py: ``spread_bits`` against a
bit-by-bit interleave of all 1024 values, corner codes in closed form, the
base order against ``np.argsort(codes, kind="stable")`` under sort-memory
limits that force every branch of the recursion, every row's scale against
the formula over its bucket found by an independent grouping, and block
bounds against ``np.min``/``np.max``.
"""
from __future__ import annotations

import math
from typing import Dict, List

import numpy as np

RECORD_BYTES = 8 + 59 * 4
C0 = 0.28209479177387814


def spread_bits(v: np.ndarray) -> np.ndarray:
    v = np.asarray(v, np.uint32)
    v = (v | (v << np.uint32(16))) & np.uint32(0x030000FF)
    v = (v | (v << np.uint32(8))) & np.uint32(0x0300F00F)
    v = (v | (v << np.uint32(4))) & np.uint32(0x030C30C3)
    v = (v | (v << np.uint32(2))) & np.uint32(0x09249249)
    return v


def morton_codes(xyz, scene_min, scene_max) -> np.ndarray:
    xyz = np.asarray(xyz, np.float32)
    smin = np.asarray(scene_min, np.float32)
    smax = np.asarray(scene_max, np.float32)
    normalized = (xyz - smin[None, :]) / (smax[None, :] - smin[None, :] + np.float32(1e-8))
    quantized = np.clip((normalized * np.float32(1023.0)).astype(np.uint32), 0, 1023)
    xx, yy, zz = (spread_bits(quantized[:, d]) for d in range(3))
    return (xx | (yy << np.uint32(1)) | (zz << np.uint32(2))).astype(np.uint64)


def rgb_to_sh(chunk: np.ndarray, rows: int) -> np.ndarray:
    names = set(chunk.dtype.names or ())
    if {"f_dc_0", "f_dc_1", "f_dc_2"} <= names:
        return np.stack([chunk[f"f_dc_{i}"].astype(np.float32) for i in range(3)], axis=1)

    def first(cands):
        for c in cands:
            if c in names:
                return c
        return None

    r, g, b = (first(("red", "r", "diffuse_red")), first(("green", "g", "diffuse_green")),
               first(("blue", "b", "diffuse_blue")))
    if r is not None and g is not None and b is not None:
        rgb = np.stack([chunk[n].astype(np.float32) for n in (r, g, b)], axis=1)
        if rgb.max(initial=0.0) > 1.0:
            rgb *= 1.0 / 255.0
    else:
        rgb = np.full((rows, 3), 0.5, dtype=np.float32)
    return (rgb - 0.5) / np.float32(C0)


def pack_rows(chunk: np.ndarray, log_scale: float, opacity_logit: float) -> np.ndarray:
    rows = int(chunk.shape[0])
    out = np.zeros((rows, 59), dtype=np.float32)
    for d, name in enumerate("xyz"):
        out[:, d] = chunk[name].astype(np.float32, copy=False)
    out[:, 3:6] = np.float32(log_scale)
    out[:, 6] = 1.0
    out[:, 10] = np.float32(opacity_logit)
    out[:, 11:14] = rgb_to_sh(chunk, rows)
    return out


def estimate_log_scale(scene_min, scene_max, n_points) -> float:
    extent = np.maximum(np.asarray(scene_max, np.float32) - np.asarray(scene_min, np.float32),
                        np.float32(1e-6))
    volume = float(np.prod(extent))
    density_side = (volume / max(int(n_points), 1)) ** (1.0 / 3.0)
    return float(math.log(max(density_side, 1e-4)))


def bucket_log_scale(xyz, n_points, global_log_scale, clamp_delta) -> float:
    if int(n_points) <= 1 or xyz.size == 0:
        return float(global_log_scale)
    local = estimate_log_scale(xyz.min(axis=0), xyz.max(axis=0), int(n_points))
    return float(np.clip(local, global_log_scale - clamp_delta, global_log_scale + clamp_delta))


def update_block_bounds(block_bounds, start_row, xyz, block_size) -> None:
    local, rows = 0, int(xyz.shape[0])
    while local < rows:
        g = start_row + local
        block_id, within = g // block_size, g % block_size
        take = min(rows - local, block_size - within)
        part = xyz[local:local + take]
        bmin, bmax = part.min(axis=0), part.max(axis=0)
        if within == 0:
            block_bounds[block_id, :3] = bmin
            block_bounds[block_id, 3:] = bmax
        else:
            block_bounds[block_id, :3] = np.minimum(block_bounds[block_id, :3], bmin)
            block_bounds[block_id, 3:] = np.maximum(block_bounds[block_id, 3:], bmax)
        local += take


def _bucket_for_codes(codes, bucket_bits, level):
    shift = max(0, 30 - bucket_bits * (level + 1))
    mask = (1 << bucket_bits) - 1
    return ((codes >> np.uint64(shift)) & np.uint64(mask)).astype(np.int32)


class _Writer:
    def __init__(self, n, block_size):
        self.parts: List[np.ndarray] = []
        self.row = 0
        self.block_size = block_size
        self.bounds = np.zeros(((n + block_size - 1) // block_size, 6), np.float32)

    def write(self, params):
        self.parts.append(params)
        update_block_bounds(self.bounds, self.row, params[:, 0:3], self.block_size)
        self.row += int(params.shape[0])


def _sort_bucket(records, writer, g_scale, delta, bucket_bits, level, max_bytes, stats):
    """_sort_bucket_to_base (:319-372) on a record array."""
    nbytes = int(records.shape[0]) * RECORD_BYTES
    stats["max_bucket_bytes"] = max(stats["max_bucket_bytes"], nbytes)
    if nbytes > max_bytes:
        max_level = max(0, int(math.ceil(30 / bucket_bits)) - 1)
        if level >= max_level:  # _stream_equal_key_bucket_to_base (:427-466)
            stats["streamed_equal_key_buckets"] += 1
            if records.shape[0] == 0:
                return
            xyz = records["params"][:, 0:3]
            scale = bucket_log_scale(np.stack([xyz.min(axis=0), xyz.max(axis=0)]),
                                     records.shape[0], g_scale, delta)
            params = np.ascontiguousarray(records["params"])
            params[:, 3:6] = np.float32(scale)
            writer.write(params)
            return
        child = level + 1  # _split_bucket_file (:379-405), children in id order
        ids = _bucket_for_codes(records["morton"], bucket_bits, child)
        kids = sorted(int(k) for k in np.unique(ids))
        stats["recursive_splits"] += 1
        stats["split_child_buckets"] += len(kids)
        for k in kids:
            _sort_bucket(records[ids == k], writer, g_scale, delta, bucket_bits, child, max_bytes,
                         stats)
        return
    if records.shape[0] == 0:
        return
    stats["in_memory_buckets"] += 1
    order = np.argsort(records["morton"], kind="stable")
    params = np.ascontiguousarray(records["params"][order])
    scale = bucket_log_scale(params[:, 0:3], params.shape[0], g_scale, delta)
    params[:, 3:6] = np.float32(scale)
    writer.write(params)


def build_base(vertices: np.ndarray, block_size: int, chunk_vertices: int = 1_000_000,
               bucket_bits: int = 10, scale_clamp_delta: float = 2.0,
               max_sort_memory_mb: float = 512.0) -> Dict:
    """Passes 1-3 of streaming_ply_to_ssd_base on a structured vertex array."""
    n = int(vertices.shape[0])
    chunks = [vertices[i:i + chunk_vertices] for i in range(0, n, chunk_vertices)]
    smin = np.full(3, np.inf, np.float32)
    smax = np.full(3, -np.inf, np.float32)
    for ch in chunks:
        xyz = np.stack([ch[c].astype(np.float32, copy=False) for c in "xyz"], axis=1)
        smin = np.minimum(smin, xyz.min(axis=0))
        smax = np.maximum(smax, xyz.max(axis=0))
    g_scale = estimate_log_scale(smin, smax, n)
    opacity_logit = float(math.log(0.1 / 0.9))
    dtype = np.dtype([("morton", "<u8"), ("params", "<f4", (59,))])
    buckets: Dict[int, List[np.ndarray]] = {}
    for ch in chunks:
        xyz = np.stack([ch[c].astype(np.float32, copy=False) for c in "xyz"], axis=1)
        codes = morton_codes(xyz, smin, smax)
        params = pack_rows(ch, g_scale, opacity_logit)
        ids = _bucket_for_codes(codes, bucket_bits, 0)
        for b in np.unique(ids):
            m = ids == b
            rec = np.empty(int(m.sum()), dtype=dtype)
            rec["morton"] = codes[m]
            rec["params"] = params[m]
            buckets.setdefault(int(b), []).append(rec)
    max_bytes = max(int(float(max_sort_memory_mb) * 1024 * 1024), RECORD_BYTES)
    stats = {"max_sort_memory_mb": float(max_sort_memory_mb), "recursive_splits": 0,
             "split_child_buckets": 0, "in_memory_buckets": 0, "streamed_equal_key_buckets": 0,
             "max_bucket_bytes": 0}
    writer = _Writer(n, block_size)
    for b in sorted(buckets, key=lambda k: f"bucket_{k:04d}.bin"):
        _sort_bucket(np.concatenate(buckets[b]), writer, g_scale, scale_clamp_delta, bucket_bits,
                     0, max_bytes, stats)
    base = np.concatenate(writer.parts) if writer.parts else np.zeros((0, 59), np.float32)
    return {"base": base, "block_bounds": writer.bounds, "scene_min": smin, "scene_max": smax,
            "global_log_scale": g_scale, "external_sort": stats}
