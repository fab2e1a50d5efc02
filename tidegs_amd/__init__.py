"""TideGS per-iteration GPU hot path, native to MI355X (gfx950 / CDNA4).

Drop-in surfaces (same names and call conventions as the reference):

* gsplat ops used by TideGS: ``fully_fused_projection``, ``spherical_harmonics``,
  ``isect_tiles``, ``isect_offset_encode``, ``rasterize_to_pixels``
* ``fused_ssim`` (clm_kernels)
* ``GPUResidentAdam`` (+ ``GPUResidentSophia``)
* ``TideStep``: the fused per-batch render/backward/optimizer step over a
  resident ``[N,59]`` Gaussian table
* ``ResidentWorkingSet``: GPU materialization and writeback of the resident
  block set (the Triton movers of TideGS's double-buffered working set)

All compute runs in hand-written HIP kernels in ``libtidegs_amd.so`` behind a
plain C ABI (``include/tidegs_amd.h``); PyTorch only provides device memory and
streams.
"""
from .gsplat_ops import (
    fully_fused_projection,
    isect_offset_encode,
    isect_tiles,
    radix_sort_pairs,
    rasterize_to_pixels,
    spherical_harmonics,
)
from .clm_ops import FusedSSIMMap, fused_ssim
from .resident_optim import GPUResidentAdam, GPUResidentSophia
from .working_set import BlockLayout, ResidentBuffer, ResidentWorkingSet

__all__ = [
    "fully_fused_projection",
    "spherical_harmonics",
    "isect_tiles",
    "isect_offset_encode",
    "rasterize_to_pixels",
    "radix_sort_pairs",
    "fused_ssim",
    "FusedSSIMMap",
    "GPUResidentAdam",
    "GPUResidentSophia",
    "ResidentWorkingSet",
    "ResidentBuffer",
    "BlockLayout",
]
