"""CPU oracle for the TideGS hot path — TEST INFRASTRUCTURE ONLY.

This package restates the reference algorithms (gsplat 1.0 CUDA sources,
clm_kernels' fused SSIM and TideGS's GPUResidentAdam) on the CPU so that the
HIP kernels can be checked against them.  Only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import
it, and only as the checker or the timed CPU baseline: the product path
(``tidegs_amd``) never imports, calls or falls back to anything here.

Each function cites the reference file:line it restates.  How each one is
pinned (golden vectors, closed forms, autograd, brute force) is listed in the
module docstrings and exercised by ``tests/test_oracle_*.py``.
"""
