"""The C ABI library loads and exports exactly what include/*.h declares.

Runs without a GPU: it only loads the shared object and inspects symbols
(no kernel is launched).
"""
import ctypes
import re
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


def _declarations():
    decls = {}
    for header in sorted((ROOT / "include").glob("*.h")):
        text = header.read_text()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        for m in re.finditer(r"\b(?:int|size_t|uint32_t|uint64_t|const char\*)\s+(tgs_\w+)\s*\(([^;]*?)\)\s*;",
                             text, flags=re.S):
            args = m.group(2).strip()
            n_args = 0 if args in ("", "void") else args.count(",") + 1
            decls[m.group(1)] = n_args
    return decls


def test_header_declares_entry_points():
    decls = _declarations()
    assert len(decls) >= 20
    for name in ("tgs_fully_fused_projection_fwd", "tgs_rasterize_to_pixels_bwd",
                 "tgs_radix_sort_pairs", "tgs_resident_adam_step", "tgs_fused_ssim_bwd"):
        assert name in decls


def test_library_exports_every_declared_symbol():
    from tidegs_amd import _native

    lib = _native.library_path()
    assert lib.exists(), "run __graft_entry__.build() first"
    out = subprocess.run(["nm", "-D", "--defined-only", str(lib)], capture_output=True, text=True,
                         check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    missing = sorted(set(_declarations()) - exported)
    assert not missing, missing


def test_bindings_match_header():
    from tidegs_amd import _native

    decls = _declarations()
    assert set(_native.SIGNATURES) == set(decls)
    for name, n_args in decls.items():
        assert len(_native.SIGNATURES[name][1]) == n_args, name


def test_library_loads_and_reports_version():
    # dlopen + a host-only call; no device work.
    import torch  # noqa: F401  (shares the HIP runtime, as in production)
    from tidegs_amd import _native

    lib = _native.load()
    assert lib.tgs_abi_version() == 1
    assert lib.tgs_bit_width(8160) == 13 and lib.tgs_bit_width(1) == 1
    assert lib.tgs_radix_sort_workspace_size(1 << 20) > 0
    buf = (ctypes.c_int32 * 16)()
    n = lib.tgs_rasterize_supported_channels(buf, 16)
    assert list(buf[:n]) == [1, 2, 3, 4, 8, 16, 32]


def test_argument_errors_are_reported_without_a_gpu():
    from tidegs_amd import _native

    lib = _native.load()
    rc = lib.tgs_fully_fused_projection_fwd(1, 4, None, None, None, None, None, None, 8, 8, 0.3,
                                            0.01, 1e10, 0.0, None, None, None, None, None, None)
    assert rc == -1
    assert "null pointer" in _native.last_error()
    with pytest.raises(RuntimeError, match="null pointer"):
        _native.call("tgs_compute_sh_fwd", 4, 16, 3, None, None, None, None, None)


def test_working_set_argument_checks_without_a_gpu():
    # Host-side validation only: every call below returns before any launch.
    from tidegs_amd import _native

    lib = _native.load()
    fake = ctypes.c_void_p(0x1000)  # never dereferenced: the checks fail first
    assert lib.tgs_ws_copy_rows(None, 59, None, None, None, 0, 0, 4096, None, 59, None, None) == 0
    assert lib.tgs_ws_copy_rows(None, 59, None, None, None, 1, 10, 4096, None, 59, None, None) == -1
    assert "null pointer" in _native.last_error()
    assert lib.tgs_ws_copy_rows(fake, 60, None, fake, fake, 1, 10, 4096, fake, 59, None, None) == -1
    assert "pitch" in _native.last_error()
    # 9000 rows of 4096-row blocks need 3 starts
    assert lib.tgs_ws_copy_rows(fake, 64, None, fake, fake, 2, 9000, 4096, fake, 64, None, None) == -1
    assert "3 blocks" in _native.last_error()
    assert lib.tgs_ws_copy_rows(fake, 64, fake, fake, fake, 3, 9000, 4096, fake, 64, None, None) == -1
    assert "id arrays" in _native.last_error()
    assert lib.tgs_ws_unpack_rows(fake, 2, 10, fake, 64, 0, None, 0, 4096, None, None) == -1
    assert "source_layout" in _native.last_error()
    assert lib.tgs_ws_unpack_rows(fake, 1, 10, fake, 64, 0, fake, 0, 4096, fake, None) == -1
    assert lib.tgs_ws_fill_global_ids(fake, 1, fake, 0, 5000, 4096, None) == -1
    assert lib.tgs_ws_pack_rows(fake, 59, fake, fake, fake, 0, 4096, fake, None) == 0
    assert lib.tgs_ws_block_bounds(fake, 60, fake, fake, 1, 4096, fake, None) == -1
    assert lib.tgs_ws_global_to_local(fake, 5, fake, 0, 4096, fake, None) == -1


def test_fused_update_argument_checks_without_a_gpu():
    # tgs_tide_project_bwd_update validates its arguments before any launch
    from tidegs_amd import _native

    _native.load()
    fake = ctypes.c_void_p(0x1000)  # never dereferenced: the checks fail first
    lrs = (ctypes.c_float * 6)()

    def call(n, optimizer=0, row_stride=64, block_size=4096, ptr=fake, bias=fake):
        return _native.load().tgs_tide_project_bwd_update(
            n, ptr, ptr, ptr, ptr, 2, ptr, row_stride, ptr, ptr, ptr, 64, 48, 0.3, 0.01, 1e10, 0.0,
            3, ptr, ptr, ptr, ptr, 4, block_size, bias, bias, ptr, ptr, 64, lrs, optimizer,
            0.9, 0.999, 1e-15, 2.0, 0.04, 1, ptr, None)

    assert call(0) == 0
    assert call(0, optimizer=2) == -1
    assert "optimizer must be" in _native.last_error()
    assert call(5, ptr=None) == -1 and "null" in _native.last_error()
    assert call(5, bias=None) == -1 and "bias table" in _native.last_error()
    assert call(5, optimizer=1, bias=None, row_stride=65) == -1  # Sophia needs no bias tables
    assert "row_stride" in _native.last_error()
    assert call(5, block_size=1 << 23) == -1 and "block_size" in _native.last_error()
