"""GPU build of the Morton-sorted base file (tidegs_amd.streaming_init) against
the CPU restatement of TideGS's bucketed external sort
(oracle/streaming_init_ref.py): base_file.bin byte for byte, block bounds and
the manifest's numbers identical, under sort-memory limits that take every
branch of the reference's recursion."""
import json

import numpy as np
import pytest

from oracle import streaming_init_ref as S
from tests.gpu_util import announce
from tidegs_amd.streaming_init import read_binary_ply_header, streaming_ply_to_ssd_base, \
    write_binary_ply

pytestmark = pytest.mark.gpu


def _ply(path, seed, n, colour):
    rng = np.random.default_rng(seed)
    k1, k2 = n // 2, n // 8
    xyz = np.concatenate([rng.uniform(0.0, 0.02, (k1, 3)),
                          np.repeat(rng.uniform(0, 1, (1, 3)), k2, axis=0),
                          rng.uniform(-50.0, 50.0, (n - k1 - k2, 3))]).astype(np.float32)
    rng.shuffle(xyz)
    if colour == "uchar":
        extra = {c: rng.integers(0, 256, n).astype(np.uint8) for c in ("red", "green", "blue")}
    elif colour == "f_dc":
        extra = {f"f_dc_{i}": rng.standard_normal(n).astype(np.float32) for i in range(3)}
        extra["opacity"] = rng.standard_normal(n).astype(np.float32)  # ignored by the init
    else:
        extra = {}
    write_binary_ply(path, xyz, extra)


@pytest.mark.parametrize("n,mb,colour,chunk", [(20000, 512.0, "uchar", 7000),
                                                (60000, 0.5, "f_dc", 1_000_000),
                                                (60000, 0.0, "none", 25000),
                                                (2_000_000, 64.0, "uchar", 1_000_000)])
def test_streaming_init_matches_oracle(gpu, tmp_path, n, mb, colour, chunk):
    announce(f"streaming init n={n} sort_mb={mb} colour={colour}")
    ply = tmp_path / "scene.ply"
    _ply(ply, n % 97, n, colour)
    man = streaming_ply_to_ssd_base(ply, tmp_path / "out", block_size=4096,
                                    debug_fast_init_scales=True, chunk_vertices=chunk,
                                    max_sort_memory_mb=mb, device=gpu)
    h = read_binary_ply_header(ply)
    with open(ply, "rb") as f:
        f.seek(h.data_offset)
        verts = np.fromfile(f, dtype=h.vertex_dtype, count=h.vertex_count)
    ref = S.build_base(verts, block_size=4096, chunk_vertices=chunk, max_sort_memory_mb=mb)
    got = np.fromfile(tmp_path / "out" / "base_file.bin", dtype=np.float32).reshape(-1, 59)
    assert got.shape == ref["base"].shape
    assert got.tobytes() == ref["base"].tobytes()
    np.testing.assert_array_equal(np.load(tmp_path / "out" / "block_bounds.npy"),
                                  ref["block_bounds"])
    disk = json.loads((tmp_path / "out" / "streaming_init_manifest.json").read_text())
    assert disk["external_sort"] == ref["external_sort"]
    assert disk["global_log_scale"] == ref["global_log_scale"]
    assert disk["scene_min"] == ref["scene_min"].astype(float).tolist()
    assert disk["scene_max"] == ref["scene_max"].astype(float).tolist()
    assert disk["total_points"] == n and disk["num_blocks"] == -(-n // 4096)
    assert man["base_file"] == disk["base_file"]


def test_streaming_init_rejects_what_the_reference_rejects(gpu, tmp_path):
    announce("streaming init argument errors")
    ply = tmp_path / "s.ply"
    _ply(ply, 0, 100, "none")
    with pytest.raises(RuntimeError, match="debug_fast_init_scales"):
        streaming_ply_to_ssd_base(ply, tmp_path / "o", 64, debug_fast_init_scales=False)
    ascii_ply = tmp_path / "a.ply"
    ascii_ply.write_bytes(b"ply\nformat ascii 1.0\nelement vertex 1\nproperty float x\n"
                          b"property float y\nproperty float z\nend_header\n0 0 0\n")
    with pytest.raises(ValueError, match="binary_little_endian"):
        streaming_ply_to_ssd_base(ascii_ply, tmp_path / "o", 64, debug_fast_init_scales=True)
