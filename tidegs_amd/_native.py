"""ctypes binding of ``libtidegs_amd.so`` (the C ABI in ``include/tidegs_amd.h``).

The library is loaded after ``torch`` so that both share one HIP runtime
(``libamdhip64.so.7``).  There is no fallback: if the library is missing or a
call fails, a ``RuntimeError`` is raised.
"""
from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

import torch

_LIB_PATH = Path(__file__).resolve().parent / "libtidegs_amd.so"
_lock = threading.Lock()
_lib = None

P = ctypes.c_void_p
I32 = ctypes.c_int32
U32 = ctypes.c_uint32
I64 = ctypes.c_int64
U64 = ctypes.c_uint64
F32 = ctypes.c_float
SZ = ctypes.c_size_t

# name -> (restype, argtypes); mirrors include/tidegs_amd.h one to one.
SIGNATURES = {
    "tgs_abi_version": (ctypes.c_int, []),
    "tgs_last_error": (ctypes.c_char_p, []),
    "tgs_fill_u32": (ctypes.c_int, [P, U64, U32, P]),
    "tgs_fully_fused_projection_fwd": (
        ctypes.c_int,
        [U32, U32, P, P, P, P, P, P, I32, I32, F32, F32, F32, F32, P, P, P, P, P, P],
    ),
    "tgs_fully_fused_projection_bwd": (
        ctypes.c_int,
        [U32, U32, P, P, P, P, P, P, I32, I32, F32, P, P, P, P, P, P, P, P, P, P, P, P, P],
    ),
    "tgs_fully_fused_projection_packed_blocks": (U32, [U32]),
    "tgs_fully_fused_projection_packed_count": (
        ctypes.c_int, [U32, U32, P, P, P, P, P, P, I32, I32, F32, F32, F32, F32, P, P]),
    "tgs_fully_fused_projection_packed_fwd": (
        ctypes.c_int,
        [U32, U32, P, P, P, P, P, P, I32, I32, F32, F32, F32, F32, P, U32, P, P, P, P, P, P, P,
         P, P]),
    "tgs_fully_fused_projection_packed_bwd": (
        ctypes.c_int,
        [U32, U32, U32, P, P, P, P, P, P, I32, I32, F32, P, P, P, P, P, P, P, P, ctypes.c_int,
         P, P, P, P, P, P]),
    "tgs_compute_sh_fwd": (ctypes.c_int, [U32, U32, I32, P, P, P, P, P]),
    "tgs_compute_sh_bwd": (ctypes.c_int, [U32, U32, I32, P, P, P, P, P, P, P]),
    "tgs_bit_width": (U32, [U32]),
    "tgs_isect_tiles_count": (ctypes.c_int, [U64, P, P, U32, U32, U32, P, P]),
    "tgs_scan_workspace_size": (SZ, [U64]),
    "tgs_inclusive_scan_i32_i64": (ctypes.c_int, [P, P, U64, P, SZ, P]),
    "tgs_exclusive_scan_u32": (ctypes.c_int, [P, P, U64, P, SZ, P]),
    "tgs_isect_tiles_emit": (
        ctypes.c_int,
        [U64, U32, P, P, P, P, P, U32, U32, U32, U32, P, P, P],
    ),
    "tgs_radix_sort_workspace_size": (SZ, [U64]),
    "tgs_radix_sort_pairs": (
        ctypes.c_int,
        [P, P, P, P, U64, ctypes.c_int, ctypes.c_int, P, SZ, ctypes.POINTER(ctypes.c_int), P],
    ),
    "tgs_radix_sort_pairs_noalloc": (
        ctypes.c_int,
        [P, P, P, P, U64, ctypes.c_int, ctypes.c_int, ctypes.POINTER(ctypes.c_int), P],
    ),
    "tgs_segmented_sort_workspace_size": (SZ, [U64, U32]),
    "tgs_segmented_sort_pairs_u32": (
        ctypes.c_int,
        [P, P, P, P, U32, U64, U32, P, ctypes.c_int, ctypes.c_int, P, SZ,
         ctypes.POINTER(ctypes.c_int), P],
    ),
    "tgs_segmented_sort_pairs_u32_range": (
        ctypes.c_int,
        [P, P, P, P, U32, U64, U32, P, U32, ctypes.c_int, P, SZ, ctypes.POINTER(ctypes.c_int), P],
    ),
    "tgs_isect_offset_encode": (ctypes.c_int, [U64, P, U32, U32, U32, P, P]),
    "tgs_rasterize_supported_channels": (ctypes.c_int, [ctypes.POINTER(I32), I32]),
    "tgs_rasterize_to_pixels_fwd": (
        ctypes.c_int,
        [U32, U32, P, P, P, P, P, U32, U32, U32, U32, U32, P, P, U32, P, P, P, P],
    ),
    "tgs_rasterize_to_pixels_bwd": (
        ctypes.c_int,
        [U32, U32, P, P, P, P, P, U32, U32, U32, U32, U32, P, P, U32, P, P, P, P,
         P, P, P, P, P, P],
    ),
    "tgs_fused_ssim_fwd": (ctypes.c_int, [I32, I32, I32, I32, F32, F32, P, P, P, P, P, P, P]),
    "tgs_fused_ssim_bwd": (
        ctypes.c_int, [I32, I32, I32, I32, F32, F32, P, P, P, P, P, P, P, P]
    ),
    "tgs_tide_loss": (ctypes.c_int, [I32, I32, I32, P, P, F32, F32, P, P, P]),
    "tgs_tide_camera_centers": (ctypes.c_int, [U32, P, P, P]),
    "tgs_tide_row_blocks": (U32, [U64]),
    "tgs_tide_visibility": (
        ctypes.c_int, [U64, P, U32, U32, P, P, P, I32, I32, F32, F32, F32, F32, P, P, P, P]),
    "tgs_tide_compact": (ctypes.c_int, [U64, U32, P, P, P, P, P, P, P, P, P, P]),
    "tgs_tide_project_fwd": (
        ctypes.c_int,
        [U32, P, P, P, P, P, U32, P, U32, P, P, P, I32, I32, F32, F32, F32, F32, I32, U32, U32,
         U32, P, P, P, P, P, P]),
    "tgs_tide_isect_totals": (ctypes.c_int, [U32, P, P, P, U32, P, P]),
    "tgs_tide_isect_count": (ctypes.c_int, [U32, P, P, P]),
    "tgs_tide_isect_segments": (ctypes.c_int, [U32, P, P, P, P]),
    "tgs_tide_isect_emit": (ctypes.c_int, [U32, P, U32, P, P, U32, U32, P, P, P]),
    "tgs_tide_isect_emit_blocks": (U32, [U32]),
    "tgs_tide_isect_block_sums": (ctypes.c_int, [U32, P, P, P]),
    "tgs_tide_isect_emit_blocked": (ctypes.c_int, [U32, P, U32, P, P, U32, U32, P, P, P]),
    "tgs_tide_isect_emit_blocked_hist": (
        ctypes.c_int, [U32, P, U32, P, P, U32, U32, P, P, P, P, U64, P]),
    "tgs_segmented_sort_pairs_u32_hist0": (
        ctypes.c_int,
        [P, P, P, P, U64, U32, P, ctypes.c_int, ctypes.c_int, P, SZ, ctypes.POINTER(ctypes.c_int),
         P]),
    "tgs_tide_isect_fused_digit_bits": (U32, [U32]),
    "tgs_tide_isect_fused_hist_words": (U64, [U32, P, U32]),
    "tgs_tide_isect_fused_count": (ctypes.c_int, [U32, P, P, U32, U32, P, U64, P]),
    "tgs_tide_isect_fused_scatter": (
        ctypes.c_int, [U32, P, P, U32, U32, P, U64, U32, P, P, P]),
    "tgs_tide_offset_encode": (ctypes.c_int, [U32, P, U32, U32, U32, U32, P, P]),
    "tgs_tide_isect_ids": (ctypes.c_int, [U32, P, P, P, P, P]),
    "tgs_tide_rasterize_fwd": (
        ctypes.c_int, [U32, P, P, U32, U32, U32, U32, P, P, U32, P, P, P, P, P, U64, P]),
    "tgs_tide_rasterize_bwd": (
        ctypes.c_int, [U32, P, P, U32, U32, U32, U32, P, P, U32, P, P, P, P, P, P]),
    "tgs_pack_splats": (ctypes.c_int, [U64, P, P, P, P, P, P]),
    "tgs_unpack_splat_grads": (ctypes.c_int, [U64, P, P, P, P, P, P]),
    "tgs_tide_project_bwd": (
        ctypes.c_int,
        [U32, P, P, P, P, U32, P, U32, P, P, P, I32, I32, F32, F32, F32, F32, I32, P, P, U32, P]),
    "tgs_tide_project_bwd_update": (
        ctypes.c_int,
        [U32, P, P, P, P, U32, P, U32, P, P, P, I32, I32, F32, F32, F32, F32, I32, P,
         P, P, P, I64, I64, P, P, P, P, U32, P, I32, F32, F32, F32, F32, F32, I32, P, P]),
    "tgs_resident_adam_step": (
        ctypes.c_int,
        [I64, P, ctypes.c_int, P, P, P, I64, I64, P, P, ctypes.c_int, P, P, P, P, P, P, P,
         F32, F32, F32, F32, P, P],
    ),
    "tgs_resident_sophia_step": (
        ctypes.c_int,
        [I64, P, ctypes.c_int, P, P, P, I64, I64, ctypes.c_int, P, P, P, P, P, P, P,
         F32, F32, F32, F32, F32, ctypes.c_int, P, P],
    ),
    "tgs_block_touch_counts": (ctypes.c_int, [I64, P, ctypes.c_int, P, P, I64, P, P]),
    "tgs_ws_copy_rows": (ctypes.c_int, [P, U32, P, P, P, U32, I64, U32, P, U32, P, P]),
    "tgs_ws_fill_global_ids": (ctypes.c_int, [P, U32, P, I64, I64, U32, P]),
    "tgs_ws_unpack_rows": (ctypes.c_int, [P, ctypes.c_int, I64, P, U32, I64, P, U32, U32, P, P]),
    "tgs_ws_pack_rows": (ctypes.c_int, [P, U32, P, P, P, U32, U32, P, P]),
    "tgs_ws_block_bounds": (ctypes.c_int, [P, U32, P, P, U32, U32, P, P]),
    "tgs_ws_build_block_starts": (ctypes.c_int, [P, P, U32, P, U32, P]),
    "tgs_ws_global_to_local": (ctypes.c_int, [P, U64, P, U32, U32, P, P]),
    "tgs_io_read_blocks": (ctypes.c_int, [U32, P, P, P, P, P, U32]),
    "tgs_init_scene_bounds": (ctypes.c_int, [P, U64, P, P, P]),
    "tgs_init_morton_codes": (ctypes.c_int, [P, U64, P, P, P]),
    "tgs_init_prefix_counts": (ctypes.c_int, [P, U64, P, P, P]),
    "tgs_init_leaf_flags": (ctypes.c_int, [P, U64, P, P, P, P]),
    "tgs_init_leaf_stats": (ctypes.c_int, [P, P, P, P, U64, U64, P, P]),
    "tgs_init_pack_rows": (ctypes.c_int, [P, P, P, P, P, F32, U64, P, P]),
    "tgs_cull_block_spheres": (ctypes.c_int, [P, U32, P, P, P]),
    "tgs_cull_blocks": (ctypes.c_int, [P, P, P, U32, P, U32, P, P]),
    "tgs_cull_blocks_cone": (ctypes.c_int, [P, U32] + [ctypes.c_double] * 7 + [P, P]),
}


def library_path() -> Path:
    return _LIB_PATH


def load() -> ctypes.CDLL:
    """Load the native library (once) and bind every declared signature."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not _LIB_PATH.exists():
            raise RuntimeError(
                f"{_LIB_PATH} is missing: build it with `python -m tidegs_amd.build` "
                "(or __graft_entry__.build()); there is no CPU fallback"
            )
        lib = ctypes.CDLL(str(_LIB_PATH), mode=os.RTLD_LOCAL | getattr(os, "RTLD_NOW", 2))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def last_error() -> str:
    msg = load().tgs_last_error()
    return msg.decode() if msg else ""


def call(name: str, *args) -> int:
    """Call an int-returning entry point and raise RuntimeError on failure."""
    fn = getattr(load(), name)
    rc = fn(*args)
    if rc != 0:
        raise RuntimeError(f"{name} failed (code {rc}): {last_error()}")
    return rc


def ptr(t) -> int | None:
    """Device pointer of a tensor (None for None)."""
    if t is None:
        return None
    return t.data_ptr()


def stream_handle(device=None) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def require_cuda(*tensors, names=None) -> None:
    for i, t in enumerate(tensors):
        if t is None:
            continue
        name = names[i] if names else f"arg{i}"
        if not t.is_cuda:
            raise RuntimeError(f"{name} must be a GPU tensor (the TideGS HIP kernels have no CPU path)")
        if not t.is_contiguous():
            raise RuntimeError(f"{name} must be contiguous")
