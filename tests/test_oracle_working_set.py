"""Pins of the resident-set oracle (oracle/working_set_ref.py) on the CPU.

Known answers come from the reference's
tests/test_double_buffer_materialization.py (:85-160 CACHE/UNIFIED
materialization + resident refresh + global_to_local, :195-262 the
persistent-slot copy); the rest are library closed forms (np.concatenate,
np.min/np.max, a dictionary lookup) that a dropped row, a swapped column or
an off-by-one block index would break.
"""
import numpy as np
import pytest

from oracle import working_set_ref as W


def components(global_ids):
    """The reference test's closed-form rows (test_double_buffer_materialization.py:11-20):
    every value is the row's global id plus a per-column constant."""
    rows = np.asarray(global_ids, np.float32)[:, None]
    return {
        "xyz": rows + np.array([0.1, 0.2, 0.3], np.float32),
        "scaling": rows + np.array([1.1, 1.2, 1.3], np.float32),
        "rotation": rows + np.array([2.1, 2.2, 2.3, 2.4], np.float32),
        "opacity": rows + np.float32(3.1),
        "features_dc": rows + np.array([4.1, 4.2, 4.3], np.float32),
        "features_rest": rows + (np.arange(45, dtype=np.float32) * np.float32(0.01)
                                 + np.float32(5.0)),
    }


def pack_block(global_ids, layout):
    """test_double_buffer_materialization.py:23-29."""
    v = components(global_ids)
    order = (("xyz", "scaling", "rotation", "opacity", "features_dc", "features_rest")
             if layout == "cache" else
             ("xyz", "opacity", "scaling", "rotation", "features_dc", "features_rest"))
    return np.concatenate([v[n] for n in order], axis=1)


def assert_components(comp, expected):
    for name in W.NAMES:
        np.testing.assert_array_equal(comp[name], expected[name], err_msg=name)


@pytest.mark.parametrize("layout", ["cache", "unified"])
def test_reference_materialization_known_answers(layout):
    # test_double_buffer_materialization.py:85-160 (14 Gaussians, blocks of 4:
    # block 3 is partial)
    src = W.BufferRef()
    ids = np.array([4, 5, 6, 7, 12, 13], np.int64)
    src.comp = components(ids)
    src.gids = ids.copy()
    src.block_to_local_slice = {1: slice(0, 4), 3: slice(4, 6)}
    calls = []

    def read_blocks(block_ids):
        calls.append(list(block_ids))
        return {2: pack_block(np.array([8, 9, 10, 11]), layout)}

    tgt = W.materialize(src, [3, 2, 1], {1, 3}, {0}, True, read_blocks, layout, 14, 4)
    expected_ids = np.array([4, 5, 6, 7, 12, 13, 8, 9, 10, 11], np.int64)
    np.testing.assert_array_equal(tgt.gids, expected_ids)
    assert_components(tgt.comp, components(expected_ids))
    assert tgt.loaded_blocks == [1, 3, 2]
    assert tgt.resident_blocks == [1, 3] and tgt.streamed_blocks == [2]
    assert tgt.evicted_blocks == [0] and calls == [[2]]
    assert tgt.block_to_local_slice == {1: slice(0, 4), 3: slice(4, 6), 2: slice(6, 10)}
    assert tgt.block_starts[[1, 2, 3]].tolist() == [0, 6, 4]
    # resident refresh after the active buffer moved on (:146-155)
    for name in W.NAMES:
        src.comp[name] += np.float32(10.0)
    assert W.finalize_retained_blocks(src, tgt, [1, 3], 4) == 2
    refreshed = components(expected_ids)
    for name in W.NAMES:
        refreshed[name][:6] += np.float32(10.0)
    assert_components(tgt.comp, refreshed)
    # global_to_local after the swap (:157-159)
    assert W.global_ids_to_local([4, 12, 8], tgt.block_starts, 4).tolist() == [0, 4, 6]


def test_reference_persistent_slot_known_answer():
    # test_double_buffer_materialization.py:195-262: block 2 (streamed into the
    # loading buffer) replaces evicted block 0 in place; block 1 stays.
    active = W.BufferRef()
    ids = np.arange(8, dtype=np.int64)
    active.comp = components(ids)
    active.gids = ids.copy()
    active.block_to_local_slice = {0: slice(0, 4), 1: slice(4, 8)}
    for name in W.NAMES:
        active.comp[name][4:8] += np.float32(10.0)
    loading = W.BufferRef()
    loading.comp = W.empty_components(4)
    loading.gids = np.zeros(4, np.int64)
    loading.block_to_local_slice = {2: slice(0, 4)}
    W.unpack_streamed_rows(pack_block(np.array([8, 9, 10, 11]), "cache"), loading.comp, 0, 4, False)
    W.fill_cold_global_ids([2], loading.gids, 0, 4, 4)
    W.copy_resident_blocks(loading, active, [2], {2: slice(0, 4)}, 4)
    expected_ids = np.array([8, 9, 10, 11, 4, 5, 6, 7], np.int64)
    np.testing.assert_array_equal(active.gids, expected_ids)
    expected = components(expected_ids)
    for name in W.NAMES:
        expected[name][4:8] += np.float32(10.0)
    assert_components(active.comp, expected)


def test_unified_columns_are_a_permutation_of_cache():
    cu, cc = W.component_columns("unified"), W.component_columns("cache")
    assert sorted(cu) == sorted(cc)
    for name in cu:
        assert cu[name].stop - cu[name].start == cc[name].stop - cc[name].start == W.WIDTHS[name]
    with pytest.raises(ValueError):
        W.component_columns("other")


@pytest.mark.parametrize("layout", ["cache", "unified"])
def test_pack_unpack_round_trip(layout):
    rng = np.random.default_rng(3)
    rows = 37
    comp = {n: rng.standard_normal((rows, W.WIDTHS[n])).astype(np.float32) for n in W.NAMES}
    order = W.component_columns(layout)
    packed = np.zeros((rows, 59), np.float32)
    for n in W.NAMES:
        packed[:, order[n]] = comp[n]
    out = W.empty_components(rows + 5)
    W.unpack_streamed_rows(packed, out, 5, rows, layout == "unified")
    for n in W.NAMES:
        np.testing.assert_array_equal(out[n][5:], comp[n])
        assert not out[n][:5].any()
    # pack the unpacked rows back: always CACHE order = concatenation
    back = np.zeros((rows, 59), np.float32)
    W.pack_resident_rows(out, [5, 5 + 16], [16, rows - 16], [0, 16], back, 32)
    np.testing.assert_array_equal(back, np.concatenate([comp[n] for n in W.NAMES], axis=1))


def test_pack_clips_each_block_at_its_count_and_block_rows():
    comp = components(np.arange(20))
    out = np.full((7, 59), -1.0, np.float32)
    # block 0: 3 rows from local 10; block 1: 4 rows from local 2
    W.pack_resident_rows(comp, [10, 2], [3, 4], [0, 3], out, 4)
    np.testing.assert_array_equal(out[:3], pack_block(np.arange(10, 13), "cache"))
    np.testing.assert_array_equal(out[3:], pack_block(np.arange(2, 6), "cache"))


def test_copy_rows_block_rule_and_partial_last_block():
    src = components(np.arange(30))
    src_g = np.arange(30, dtype=np.int64) + 100
    dst = W.empty_components(20)
    dst_g = np.full(20, -7, np.int64)
    # 2 full blocks of 5 rows and a partial one of 3: 13 rows
    W.copy_resident_rows(src, src_g, [20, 0, 10], [0, 10, 5], 13, 5, dst, dst_g)
    exp_rows = np.full(20, -1)
    exp_rows[0:5] = np.arange(20, 25)
    exp_rows[10:15] = np.arange(0, 5)
    exp_rows[5:8] = np.arange(10, 13)
    for n in W.NAMES:
        for r in range(20):
            if exp_rows[r] >= 0:
                np.testing.assert_array_equal(dst[n][r], src[n][exp_rows[r]])
            else:
                assert not dst[n][r].any()
    np.testing.assert_array_equal(dst_g[exp_rows >= 0], src_g[exp_rows[exp_rows >= 0]])
    assert (dst_g[exp_rows < 0] == -7).all()


def test_fill_cold_ids_closed_form():
    g = np.full(12, -1, np.int64)
    W.fill_cold_global_ids([7, 2, 9], g, 2, 10, 4)
    assert g.tolist() == [-1, -1, 28, 29, 30, 31, 8, 9, 10, 11, 36, 37]


def test_bounds_match_numpy_min_max():
    rng = np.random.default_rng(5)
    xyz = rng.standard_normal((300, 3)).astype(np.float32) * 50
    starts, lengths = [0, 64, 200, 7], [64, 100, 1, 0]
    out = W.resident_block_bounds(xyz, starts, lengths, 128)
    for b, (s, n) in enumerate(zip(starts, lengths)):
        if n == 0:
            np.testing.assert_array_equal(out[b], np.float32([1e20] * 3 + [-1e20] * 3))
            continue
        np.testing.assert_array_equal(out[b, :3], xyz[s:s + n].min(axis=0))
        np.testing.assert_array_equal(out[b, 3:], xyz[s:s + n].max(axis=0))
    # lengths beyond block_rows are clipped to block_rows
    out2 = W.resident_block_bounds(xyz, [0], [300], 16)
    np.testing.assert_array_equal(out2[0, :3], xyz[:16].min(axis=0))


def test_global_to_local_matches_dictionary_lookup():
    rng = np.random.default_rng(9)
    bs, nb = 16, 40
    loaded = rng.choice(nb, 15, replace=False)
    slices, off = {}, 0
    for b in loaded:
        slices[int(b)] = slice(off, off + bs)
        off += bs
    starts = W.build_block_starts(slices, nb)
    assert (starts >= 0).sum() == 15
    g = rng.integers(-40, nb * bs + 40, 5000)
    got = W.global_ids_to_local(g, starts, bs)
    for gi, li in zip(g.tolist(), got.tolist()):
        b = gi // bs
        want = slices[b].start + gi - b * bs if (0 <= b < nb and b in slices) else -1
        assert li == want, (gi, li, want)
