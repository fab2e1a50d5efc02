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
        for m in re.finditer(r"\b(?:int|size_t|uint32_t|const char\*)\s+(tgs_\w+)\s*\(([^;]*?)\)\s*;",
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
