"""Morton-sorted base file from a PLY, built on the GPU (drop-in for
``storage/streaming_ply_init.py:streaming_ply_to_ssd_base``).

The reference streams the PLY three times on the CPU: bounding box, records
``(morton <u8, params <f4[59])`` appended to 1024 bucket files by the top 10
code bits, then every bucket sorted in memory (split again by the next 10
bits when it exceeds ``max_sort_memory_mb``, down to whole codes), each
sorted bucket getting its own clamped log-scale, and per-block xyz bounds.
The rows it writes are the vertices in stable Morton order.

Here the vertices are read once (host), uploaded, and the GPU computes the
bounds, the codes, one stable radix sort, the bucket ("leaf") boundaries the
reference's recursion would produce (from the 10- and 20-bit bucket sizes),
per-leaf bounds and the packed rows; the log-scale formula of each leaf runs
on the host with the reference's own float arithmetic.  Output files are the
same: ``base_file.bin``, ``block_bounds.npy``, ``streaming_init_manifest.json``.
The scene's ``[N, 59]`` table must fit in HBM (about 1.2 billion rows on one
MI355X); ``bucket_bits`` is the reference default, 10.
"""
from __future__ import annotations

import ctypes
import json
import math
import os
from dataclasses import dataclass
from pathlib import Path
from typing import List, Tuple

import numpy as np
import torch

from . import _native as N

RECORD_DTYPE = np.dtype([("morton", "<u8"), ("params", "<f4", (59,))])
MORTON_BITS = 30
C0 = 0.28209479177387814  # real SH band 0: 1 / (2 sqrt(pi))

PLY_DTYPE_MAP = {
    "char": "i1", "int8": "i1", "uchar": "u1", "uint8": "u1", "short": "<i2", "int16": "<i2",
    "ushort": "<u2", "uint16": "<u2", "int": "<i4", "int32": "<i4", "uint": "<u4",
    "uint32": "<u4", "float": "<f4", "float32": "<f4", "double": "<f8", "float64": "<f8",
}


@dataclass(frozen=True)
class PlyHeader:
    path: str
    fmt: str
    vertex_count: int
    vertex_properties: Tuple[Tuple[str, str], ...]
    data_offset: int

    @property
    def vertex_dtype(self) -> np.dtype:
        """Packed little-endian record of one vertex, in header order."""
        bad = [f"{name} ({kind})" for name, kind in self.vertex_properties
               if kind not in PLY_DTYPE_MAP]
        if bad:
            raise ValueError("PLY vertex properties of unsupported type: " + ", ".join(bad))
        return np.dtype({"names": [name for name, _ in self.vertex_properties],
                         "formats": [PLY_DTYPE_MAP[kind] for _, kind in self.vertex_properties]})


def read_binary_ply_header(path) -> PlyHeader:
    """Vertex layout of a binary little-endian PLY (streaming_ply_init.py:80-135)."""
    path = os.fspath(path)
    fmt, count, props, element = None, None, [], None
    with open(path, "rb") as f:
        if f.readline().strip() != b"ply":
            raise ValueError(f"{path} is not a PLY file")
        while True:
            raw = f.readline()
            if not raw:
                raise ValueError(f"{path} ended before end_header")
            line = raw.decode("ascii", errors="replace").strip()
            if line == "end_header":
                offset = f.tell()
                break
            if not line or line.startswith("comment"):
                continue
            tok = line.split()
            if tok[0] == "format":
                fmt = tok[1]
            elif tok[0] == "element":
                element = tok[1]
                if element == "vertex":
                    count = int(tok[2])
            elif tok[0] == "property" and element == "vertex":
                if tok[1] == "list":
                    raise ValueError("Streaming PLY init supports only scalar vertex properties")
                props.append((tok[2], tok[1]))
    if fmt != "binary_little_endian":
        raise ValueError(f"Streaming PLY init supports binary_little_endian only, got {fmt!r}")
    if count is None:
        raise ValueError(f"{path} has no vertex element")
    missing = {"x", "y", "z"} - {n for n, _ in props}
    if missing:
        raise ValueError(f"{path} missing required vertex properties: {sorted(missing)}")
    return PlyHeader(path, fmt, int(count), tuple(props), int(offset))


def _first_name(names, candidates):
    for c in candidates:
        if c in names:
            return c
    return None


def rgb_to_sh(chunk: np.ndarray, rows: int) -> np.ndarray:
    """SH band-0 colour of a vertex chunk (streaming_ply_init.py:202-231):
    f_dc_* as stored, else (rgb - 0.5) / C0 with 8-bit colours scaled to [0,1]
    when the chunk's maximum exceeds 1, else zero colour."""
    names = set(chunk.dtype.names or ())
    if {"f_dc_0", "f_dc_1", "f_dc_2"} <= names:
        return np.stack([chunk[f"f_dc_{i}"].astype(np.float32) for i in range(3)], axis=1)
    r = _first_name(names, ("red", "r", "diffuse_red"))
    g = _first_name(names, ("green", "g", "diffuse_green"))
    b = _first_name(names, ("blue", "b", "diffuse_blue"))
    if r is not None and g is not None and b is not None:
        rgb = np.stack([chunk[n].astype(np.float32) for n in (r, g, b)], axis=1)
        if rgb.max(initial=0.0) > 1.0:
            rgb *= 1.0 / 255.0
    else:
        rgb = np.full((rows, 3), 0.5, dtype=np.float32)
    return (rgb - 0.5) / np.float32(C0)


def estimate_log_scale(scene_min: np.ndarray, scene_max: np.ndarray, n_points: int) -> float:
    """streaming_ply_init.py:171-175 (float32 extent and product, float64 rest)."""
    extent = np.maximum(np.asarray(scene_max, np.float32) - np.asarray(scene_min, np.float32),
                        np.float32(1e-6))
    volume = float(np.prod(extent))
    density_side = (volume / max(int(n_points), 1)) ** (1.0 / 3.0)
    return float(math.log(max(density_side, 1e-4)))


def bucket_log_scale(lo: np.ndarray, hi: np.ndarray, n_points: int, global_log_scale: float,
                     clamp_delta: float) -> float:
    """streaming_ply_init.py:178-192 from a bucket's xyz min/max."""
    if int(n_points) <= 1:
        return float(global_log_scale)
    local = estimate_log_scale(lo, hi, int(n_points))
    return float(np.clip(local, global_log_scale - clamp_delta, global_log_scale + clamp_delta))


def _read_vertices(header: PlyHeader, chunk_vertices: int):
    """xyz and SH dc as fp32 [N,3] (pinned), chunk by chunk as the reference."""
    n = header.vertex_count
    xyz = torch.empty((n, 3), dtype=torch.float32, pin_memory=True)
    dc = torch.empty((n, 3), dtype=torch.float32, pin_memory=True)
    xn, dn = xyz.numpy(), dc.numpy()
    dtype = header.vertex_dtype
    with open(header.path, "rb") as f:
        f.seek(header.data_offset)
        done = 0
        while done < n:
            count = min(int(chunk_vertices), n - done)
            chunk = np.fromfile(f, dtype=dtype, count=count)
            if chunk.size != count:
                raise IOError(f"Expected {count} PLY vertices, read {chunk.size}; "
                              "file may be truncated")
            for d, name in enumerate("xyz"):
                xn[done:done + count, d] = chunk[name].astype(np.float32, copy=False)
            dn[done:done + count] = rgb_to_sh(chunk, count)
            done += count
    return xyz, dc


def _sort_stats(counts0, counts1, leaf_codes, leaf_rows, big0, big1, max_bytes):
    """The external-sort counters the reference's recursion reports
    (streaming_ply_init.py:319-538) for the same buckets."""
    rec = RECORD_DTYPE.itemsize
    stats = {"in_memory_buckets": 0, "recursive_splits": 0, "split_child_buckets": 0,
             "streamed_equal_key_buckets": 0,
             "max_bucket_bytes": int(counts0.max(initial=0)) * rec}
    stats["in_memory_buckets"] += int(((counts0 > 0) & ~big0).sum())
    for p0 in np.nonzero(big0)[0]:
        stats["recursive_splits"] += 1
        kids = counts1[p0 << 10:(p0 + 1) << 10]
        stats["split_child_buckets"] += int((kids > 0).sum())
        stats["in_memory_buckets"] += int(((kids > 0) & ~big1[p0 << 10:(p0 + 1) << 10]).sum())
    lvl2 = big1[leaf_codes >> 10] & big0[leaf_codes >> 20]
    stats["recursive_splits"] += int(np.count_nonzero(big1 & (counts1 > 0)
                                                      & np.repeat(big0, 1 << 10)))
    stats["split_child_buckets"] += int(lvl2.sum())
    eq = lvl2 & (leaf_rows.astype(np.int64) * rec > max_bytes)
    stats["streamed_equal_key_buckets"] += int(eq.sum())
    stats["in_memory_buckets"] += int((lvl2 & ~eq).sum())
    return stats


def streaming_ply_to_ssd_base(ply_path, output_dir, block_size: int, debug_fast_init_scales: bool,
                              chunk_vertices: int = 1_000_000, bucket_bits: int = 10,
                              scale_clamp_delta: float = 2.0, max_sort_memory_mb: float = 512.0,
                              keep_temp: bool = False, device="cuda",
                              timings: dict | None = None) -> dict:
    """Write ``base_file.bin``, ``block_bounds.npy`` and
    ``streaming_init_manifest.json`` for a binary PLY (streaming_ply_init.py:541-696).
    ``timings``, if given, receives the wall-clock seconds of the host read,
    the GPU passes and the file writes (the GPU is synchronized between them)."""
    import time

    clock = {"t": time.perf_counter()}

    def lap(name):
        if timings is not None:
            torch.cuda.synchronize(device)
            now = time.perf_counter()
            timings[name] = now - clock["t"]
            clock["t"] = now

    if not debug_fast_init_scales:
        raise RuntimeError("streaming PLY init requires --debug_fast_init_scales; "
                           "full distCUDA2 is not out-of-core")
    if int(bucket_bits) != 10:
        raise ValueError("the GPU initializer implements bucket_bits=10 (the reference default)")
    dev = torch.device(device)
    out_dir = Path(output_dir)
    out_dir.mkdir(parents=True, exist_ok=True)
    header = read_binary_ply_header(ply_path)
    n = header.vertex_count
    if n <= 0:
        raise ValueError(f"{ply_path} has no vertices")
    stream = N.stream_handle(dev)
    xyz_h, dc_h = _read_vertices(header, chunk_vertices)
    lap("read_ply")
    xyz = xyz_h.to(dev, non_blocking=True)
    dc = dc_h.to(dev, non_blocking=True)

    scratch = torch.empty(8, dtype=torch.int32, device=dev)
    bounds = torch.empty(6, dtype=torch.float32, device=dev)
    N.call("tgs_init_scene_bounds", N.ptr(xyz), n, N.ptr(scratch), N.ptr(bounds), stream)
    b = bounds.cpu().numpy()
    scene_min, scene_max = b[:3].copy(), b[3:].copy()
    log_scale = estimate_log_scale(scene_min, scene_max, n)

    codes = torch.empty(n, dtype=torch.int32, device=dev)
    N.call("tgs_init_morton_codes", N.ptr(xyz), n, N.ptr(bounds), N.ptr(codes), stream)
    # stable sort of (code, vertex id): rows in the order of the reference's base file
    vals = torch.arange(n, dtype=torch.int32, device=dev)
    codes_alt = torch.empty_like(codes)
    vals_alt = torch.empty_like(vals)
    ws_bytes = N.load().tgs_segmented_sort_workspace_size(n, 1)
    work = torch.empty(max(int(ws_bytes), 1), dtype=torch.uint8, device=dev)
    seg = (ctypes.c_uint32 * 2)(0, n)
    sel = ctypes.c_int(0)
    N.call("tgs_segmented_sort_pairs_u32", N.ptr(codes), N.ptr(vals), N.ptr(codes_alt),
           N.ptr(vals_alt), 4, n, 1, seg, 0, MORTON_BITS, N.ptr(work), int(ws_bytes),
           ctypes.byref(sel), stream)
    sorted_codes, perm = (codes_alt, vals_alt) if sel.value else (codes, vals)

    counts0 = torch.empty(1024, dtype=torch.int32, device=dev)
    counts1 = torch.empty(1 << 20, dtype=torch.int32, device=dev)
    N.call("tgs_init_prefix_counts", N.ptr(sorted_codes), n, N.ptr(counts0), N.ptr(counts1),
           stream)
    c0 = counts0.cpu().numpy().view(np.uint32).astype(np.int64)
    c1 = counts1.cpu().numpy().view(np.uint32).astype(np.int64)
    max_bytes = max(int(float(max_sort_memory_mb) * 1024 * 1024), RECORD_DTYPE.itemsize)
    big0 = c0 * RECORD_DTYPE.itemsize > max_bytes
    big1 = (c1 * RECORD_DTYPE.itemsize > max_bytes) & np.repeat(big0, 1 << 10)
    big0_d = torch.from_numpy(big0.astype(np.uint8)).to(dev)
    big1_d = torch.from_numpy(big1.astype(np.uint8)).to(dev)
    flags = torch.empty(n, dtype=torch.int32, device=dev)
    N.call("tgs_init_leaf_flags", N.ptr(sorted_codes), n, N.ptr(big0_d), N.ptr(big1_d),
           N.ptr(flags), stream)
    leaf_incl = torch.empty(n, dtype=torch.int64, device=dev)
    scan_bytes = N.load().tgs_scan_workspace_size(n)
    scan_work = torch.empty(max(int(scan_bytes), 1), dtype=torch.uint8, device=dev)
    N.call("tgs_inclusive_scan_i32_i64", N.ptr(flags), N.ptr(leaf_incl), n, N.ptr(scan_work),
           int(scan_bytes), stream)
    n_leaves = int(leaf_incl[-1].item())
    stats = torch.empty((n_leaves, 8), dtype=torch.int32, device=dev)
    N.call("tgs_init_leaf_stats", N.ptr(leaf_incl), N.ptr(sorted_codes), N.ptr(perm), N.ptr(xyz),
           n, n_leaves, N.ptr(stats), stream)
    st = stats.cpu().numpy()
    lo = st[:, 0:3].view(np.float32)
    hi = st[:, 3:6].view(np.float32)
    rows = st[:, 6].view(np.uint32).astype(np.int64)
    leaf_codes = st[:, 7].view(np.uint32).astype(np.int64)
    if int(rows.sum()) != n:
        raise RuntimeError(f"leaf rows {int(rows.sum())} != vertices {n}")
    scales = np.array([bucket_log_scale(lo[i], hi[i], int(rows[i]), log_scale, scale_clamp_delta)
                       for i in range(n_leaves)], dtype=np.float64).astype(np.float32)
    scales_d = torch.from_numpy(scales).to(dev)

    table = torch.empty((n, 59), dtype=torch.float32, device=dev)
    opacity_logit = float(np.float32(math.log(0.1 / 0.9)))
    N.call("tgs_init_pack_rows", N.ptr(perm), N.ptr(leaf_incl), N.ptr(xyz), N.ptr(dc),
           N.ptr(scales_d), opacity_logit, n, N.ptr(table), stream)
    num_blocks = (n + int(block_size) - 1) // int(block_size)
    starts = torch.arange(num_blocks, dtype=torch.int64) * int(block_size)
    lengths = torch.clamp(n - starts, max=int(block_size))
    starts_d, lengths_d = starts.to(dev), lengths.to(dev)
    block_bounds = torch.empty((num_blocks, 6), dtype=torch.float32, device=dev)
    N.call("tgs_ws_block_bounds", N.ptr(table), 59, N.ptr(starts_d), N.ptr(lengths_d), num_blocks,
           int(block_size), N.ptr(block_bounds), stream)

    lap("gpu")
    base_file = out_dir / "base_file.bin"
    chunk_rows = 1 << 20
    host = torch.empty((min(chunk_rows, n), 59), dtype=torch.float32, pin_memory=True)
    with open(base_file, "wb") as f:
        for r0 in range(0, n, chunk_rows):
            r1 = min(n, r0 + chunk_rows)
            part = host[:r1 - r0]
            part.copy_(table[r0:r1])
            part.numpy().tofile(f)
    bounds_path = out_dir / "block_bounds.npy"
    np.save(bounds_path, block_bounds.cpu().numpy())
    actual = base_file.stat().st_size
    if actual != n * 59 * 4:
        raise RuntimeError(f"base_file.bin size mismatch: actual={actual}, expected={n * 59 * 4}")

    sort_stats = {"max_sort_memory_mb": float(max_sort_memory_mb)}
    sort_stats.update(_sort_stats(c0, c1, leaf_codes, rows, big0, big1, max_bytes))
    manifest = {
        "version": 1,
        "source": "streaming_ply_to_ssd_base",
        "ply_path": os.fspath(ply_path),
        "base_file": str(base_file),
        "block_bounds": str(bounds_path),
        "total_points": int(n),
        "num_blocks": int(num_blocks),
        "block_size": int(block_size),
        "param_dim": 59,
        "dtype": "float32",
        "layout": "cache: xyz|scaling|rotation|opacity|features_dc|features_rest",
        "scene_min": scene_min.astype(float).tolist(),
        "scene_max": scene_max.astype(float).tolist(),
        "scale_mode": "morton_bucket_density_clamped",
        "global_log_scale": float(log_scale),
        "scale_clamp_delta": float(scale_clamp_delta),
        "external_sort": sort_stats,
        "morton": {"type": "standard_10bit", "bucket_bits": int(bucket_bits)},
    }
    manifest_path = out_dir / "streaming_init_manifest.json"
    with open(manifest_path, "w") as f:
        json.dump(manifest, f, indent=2, sort_keys=True)
    manifest["manifest_path"] = str(manifest_path)
    lap("write")
    return manifest


def write_binary_ply(path, xyz: np.ndarray, extra: dict | None = None) -> None:
    """A binary little-endian PLY with float x,y,z plus ``extra`` scalar
    vertex properties ({name: array}); for tests and tools."""
    extra = extra or {}
    kinds = {np.dtype("float32"): "float", np.dtype("float64"): "double",
             np.dtype("uint8"): "uchar", np.dtype("int32"): "int"}
    fields = [("x", "<f4"), ("y", "<f4"), ("z", "<f4")]
    fields += [(k, np.asarray(v).dtype.newbyteorder("<").str) for k, v in extra.items()]
    rec = np.empty(len(xyz), dtype=np.dtype(fields))
    for d, name in enumerate("xyz"):
        rec[name] = xyz[:, d]
    for k, v in extra.items():
        rec[k] = v
    lines = ["ply", "format binary_little_endian 1.0", f"element vertex {len(xyz)}"]
    lines += [f"property float {c}" for c in "xyz"]
    lines += [f"property {kinds[np.asarray(v).dtype]} {k}" for k, v in extra.items()]
    lines += ["end_header"]
    with open(path, "wb") as f:
        f.write(("\n".join(lines) + "\n").encode("ascii"))
        rec.tofile(f)
