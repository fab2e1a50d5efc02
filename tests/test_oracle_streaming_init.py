"""Pins of the streaming-initializer oracle (oracle/streaming_init_ref.py).

Closed forms and library routines that a wrong shift, a dropped axis, an
unstable sort or a mis-chosen bucket would break: bit-by-bit interleaving,
corner codes, np.argsort(kind="stable") of the codes, the scale formula over
buckets found by independent counting, and np.min/np.max block bounds."""
import math

import numpy as np
import pytest

from oracle import streaming_init_ref as S


def test_spread_bits_matches_bitwise_interleave():
    v = np.arange(1024, dtype=np.uint32)
    want = np.zeros(1024, np.uint32)
    for bit in range(10):
        want |= ((v >> bit) & 1) << (3 * bit)
    np.testing.assert_array_equal(S.spread_bits(v), want)


def test_corner_codes():
    lo, hi = np.float32([-3, 0.5, 10]), np.float32([5, 2.5, 30])
    pts = np.stack([lo, hi, np.float32([5, 0.5, 10]), np.float32([-3, 0.5, 30])])
    codes = S.morton_codes(pts, lo, hi)
    assert codes.tolist() == [0, (1 << 30) - 1, int(S.spread_bits(np.uint32([1023]))[0]),
                              int(S.spread_bits(np.uint32([1023]))[0]) << 2]


def scene(seed, n):
    """Clustered vertices: a dense cube (big buckets), duplicated points
    (equal codes) and a uniform background; uchar colours."""
    rng = np.random.default_rng(seed)
    k1, k2 = n // 2, n // 8
    xyz = np.concatenate([
        rng.uniform(0.0, 0.02, (k1, 3)),
        np.repeat(rng.uniform(0, 1, (1, 3)), k2, axis=0),
        rng.uniform(-5.0, 5.0, (n - k1 - k2, 3))]).astype(np.float32)
    v = np.empty(n, dtype=[("x", "<f4"), ("y", "<f4"), ("z", "<f4"), ("red", "u1"),
                           ("green", "u1"), ("blue", "u1")])
    for d, c in enumerate("xyz"):
        v[c] = xyz[:, d]
    for c in ("red", "green", "blue"):
        v[c] = rng.integers(0, 256, n)
    return v


def leaf_of_rows(codes_sorted, max_bytes):
    """Independent bucket choice from prefix counts (np.unique)."""
    rec = S.RECORD_BYTES
    p0, p1 = codes_sorted >> 20, codes_sorted >> 10
    u0, c0 = np.unique(p0, return_counts=True)
    u1, c1 = np.unique(p1, return_counts=True)
    n0 = dict(zip(u0.tolist(), c0.tolist()))
    n1 = dict(zip(u1.tolist(), c1.tolist()))
    keys = []
    for a, b, c in zip(p0.tolist(), p1.tolist(), codes_sorted.tolist()):
        if n0[a] * rec <= max_bytes:
            keys.append((0, a))
        elif n1[b] * rec <= max_bytes:
            keys.append((1, b))
        else:
            keys.append((2, c))
    return keys


@pytest.mark.parametrize("mb", [512.0, 0.5, 0.02, 0.0])
def test_base_order_scales_and_bounds(mb):
    v = scene(1, 20000)
    out = S.build_base(v, block_size=512, chunk_vertices=7000, max_sort_memory_mb=mb)
    base = out["base"]
    xyz = np.stack([v[c] for c in "xyz"], axis=1)
    codes = S.morton_codes(xyz, out["scene_min"], out["scene_max"])
    order = np.argsort(codes, kind="stable")
    np.testing.assert_array_equal(base[:, 0:3], xyz[order])
    assert (base[:, 6] == 1).all() and not base[:, 7:10].any() and not base[:, 14:].any()
    np.testing.assert_array_equal(base[:, 10], np.float32(math.log(0.1 / 0.9)))
    # scales: one value per bucket, from the formula over that bucket's rows
    max_bytes = max(int(mb * 1024 * 1024), S.RECORD_BYTES)
    keys = leaf_of_rows(codes[order], max_bytes)
    groups = {}
    for i, k in enumerate(keys):
        groups.setdefault(k, []).append(i)
    for k, rows in groups.items():
        want = S.bucket_log_scale(base[rows, 0:3], len(rows), out["global_log_scale"], 2.0)
        np.testing.assert_array_equal(base[rows, 3:6], np.float32(want))
    st = out["external_sort"]
    assert st["in_memory_buckets"] + st["streamed_equal_key_buckets"] == len(groups)
    if mb == 0.0:
        assert st["streamed_equal_key_buckets"] > 0 and st["recursive_splits"] > 0
    if mb == 512.0:
        assert st["recursive_splits"] == 0
    # block bounds
    for b in range(out["block_bounds"].shape[0]):
        part = base[b * 512:(b + 1) * 512, 0:3]
        np.testing.assert_array_equal(out["block_bounds"][b, :3], part.min(axis=0))
        np.testing.assert_array_equal(out["block_bounds"][b, 3:], part.max(axis=0))


def test_rgb_to_sh_cases():
    v = np.zeros(3, dtype=[("x", "<f4"), ("y", "<f4"), ("z", "<f4"), ("red", "u1"),
                           ("green", "u1"), ("blue", "u1")])
    v["red"], v["green"], v["blue"] = [0, 255, 51], [0, 0, 0], [255, 255, 255]
    got = S.rgb_to_sh(v, 3)
    want = (np.float32([[0, 0, 255], [255, 0, 255], [51, 0, 255]]) * np.float32(1 / 255)
            - np.float32(0.5)) / np.float32(S.C0)
    np.testing.assert_allclose(got, want, rtol=1e-6)
    assert abs(got[1, 0] - 0.5 / S.C0) < 1e-5
    f = np.zeros(2, dtype=[("x", "<f4"), ("y", "<f4"), ("z", "<f4"), ("f_dc_0", "<f4"),
                           ("f_dc_1", "<f4"), ("f_dc_2", "<f4")])
    f["f_dc_1"] = 3.5
    np.testing.assert_array_equal(S.rgb_to_sh(f, 2)[:, 1], [3.5, 3.5])
    none = np.zeros(2, dtype=[("x", "<f4"), ("y", "<f4"), ("z", "<f4")])
    np.testing.assert_array_equal(S.rgb_to_sh(none, 2), 0.0)
