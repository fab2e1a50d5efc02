"""GPU parity of the resident-set movers (tidegs_amd.working_set, tgs_ws_*)
with the CPU oracle (oracle/working_set_ref.py), which restates TideGS's
Triton materialization/writeback kernels.  Row moves, ids and bounds are
bit-exact; the reference's own known answers
(tests/test_double_buffer_materialization.py) run through the host mirror;
at full size the closed-form rows (value = global id + column constant) make
every row self-checking."""
import numpy as np
import pytest
import torch

from oracle import working_set_ref as W
from tests.gpu_util import announce, to_np
from tidegs_amd import _native as N
from tidegs_amd.working_set import (BlockLayout, ResidentBuffer, ResidentWorkingSet,
                                    allocate_table)

pytestmark = pytest.mark.gpu

CONST = np.concatenate([[0.1, 0.2, 0.3], [1.1, 1.2, 1.3], [2.1, 2.2, 2.3, 2.4], [3.1],
                        [4.1, 4.2, 4.3]]).astype(np.float32)


def _const_row(device=None):
    rest = torch.arange(45, dtype=torch.float32) * 0.01 + 5.0
    return torch.cat([torch.from_numpy(CONST), rest]).to(device)


def closed_form_rows(gids, device=None, layout="cache"):
    """[n,59] rows of the reference test's closed form
    (test_double_buffer_materialization.py:11-29) in CACHE or UNIFIED order."""
    g = torch.as_tensor(gids, dtype=torch.float32, device=device)[:, None]
    rows = g + _const_row(device)[None]
    if layout == "unified":
        cols = W.component_columns("cache")
        rows = torch.cat([rows[:, cols[n]] for n in
                          ("xyz", "opacity", "scaling", "rotation", "features_dc",
                           "features_rest")], dim=1)
    return rows


def make_table(rows59, pitch, device):
    t = allocate_table(rows59.shape[0], device, pitch)
    if pitch == 64:
        t.as_strided((t.shape[0], 64), (64, 1))[:, 59:].zero_()
    t.copy_(rows59)
    return t


def padding(t):
    return t.as_strided((t.shape[0], 64), (64, 1))[:, 59:]


class Reader:
    def __init__(self, layout, block_size, num_total, batch=False):
        self.layout = layout
        self.bs = block_size
        self.num_total = num_total
        self.calls = []
        if batch:
            self.read_batch = self._read_batch

    def read_blocks(self, block_ids):
        self.calls.append(list(block_ids))
        out = {}
        for b in block_ids:
            g = torch.arange(b * self.bs, min((b + 1) * self.bs, self.num_total))
            out[b] = closed_form_rows(g, layout=self.layout.value)
        return out

    def _read_batch(self, block_ids, out=None):
        from types import SimpleNamespace

        blocks = self.read_blocks(block_ids)
        slices, off = {}, 0
        for b in block_ids:
            n = blocks[b].shape[0]
            out[off:off + n].copy_(blocks[b])
            slices[b] = slice(off, off + n)
            off += n
        return SimpleNamespace(tensor=out[:off], block_ids=tuple(block_ids), block_slices=slices,
                               layout=self.layout)


@pytest.mark.parametrize("layout,pitch,batch", [("cache", 64, False), ("unified", 64, True),
                                               ("cache", 59, True), ("unified", 59, False)])
def test_reference_materialization_known_answers(gpu, layout, pitch, batch):
    announce(f"working set known answers layout={layout} pitch={pitch} read_batch={batch}")
    ws = ResidentWorkingSet(14, block_size=4, device=gpu, row_pitch=pitch)
    src = ResidentBuffer()
    ids = torch.tensor([4, 5, 6, 7, 12, 13], device=gpu)
    src.table = make_table(closed_form_rows(ids, gpu), pitch, gpu)
    src.local_to_global_idx = ids.clone()
    src.loaded_blocks = [1, 3]
    src.block_to_local_slice = {1: slice(0, 4), 3: slice(4, 6)}
    src.num_gaussians = 6
    reader = Reader(BlockLayout(layout), 4, 14, batch=batch)
    tgt = ws.materialize(src, [3, 2, 1], {1, 3}, {0}, True, reader)
    torch.cuda.synchronize()
    expected_ids = torch.tensor([4, 5, 6, 7, 12, 13, 8, 9, 10, 11], device=gpu)
    assert torch.equal(tgt.local_to_global_idx, expected_ids)
    assert torch.equal(tgt.table, closed_form_rows(expected_ids, gpu))
    if pitch == 64:
        assert not bool(padding(tgt.table).any())
    assert tgt.loaded_blocks == [1, 3, 2] and tgt.resident_blocks == [1, 3]
    assert tgt.streamed_blocks == [2] and tgt.evicted_blocks == [0]
    assert reader.calls == [[2]]
    assert tgt.block_to_local_slice == {1: slice(0, 4), 3: slice(4, 6), 2: slice(6, 10)}
    assert tgt._block_starts[[1, 2, 3]].cpu().tolist() == [0, 6, 4]
    # the component views read like the reference's six tensors
    assert torch.equal(tgt.opacity[:, 0], expected_ids.float() + np.float32(3.1))
    # resident refresh after the active buffer moved on (:146-155)
    src.table.add_(10.0)
    h = ws.finalize_retained_blocks(src, tgt, [1, 3])
    assert (h.ready_blocks, h.copied_blocks) == (2, 2)
    want = closed_form_rows(expected_ids, gpu)
    want[:6] += 10.0
    assert torch.equal(tgt.table, want)
    q = ws.global_to_local(tgt, torch.tensor([4, 12, 8], device=gpu))
    assert q.cpu().tolist() == [0, 4, 6]
    st = ws.get_stats()
    assert st["batched_materializations"] == 1 and st["batched_h2d_calls"] == 1
    assert st["batched_resident_blocks"] == 2 and st["batched_streamed_blocks"] == 1


@pytest.mark.parametrize("pitch", [59, 64])
def test_reference_persistent_slot_known_answer(gpu, pitch):
    announce(f"working set persistent slot pitch={pitch}")
    ws = ResidentWorkingSet(16, block_size=4, device=gpu, row_pitch=pitch)
    active = ResidentBuffer()
    ids = torch.arange(8, device=gpu)
    active.table = make_table(closed_form_rows(ids, gpu), pitch, gpu)
    active.local_to_global_idx = ids.clone()
    active.block_to_local_slice = {0: slice(0, 4), 1: slice(4, 8)}
    active.table[4:8] += 10.0
    loading = ws.materialize(None, [2], set(), {0}, True, Reader(BlockLayout.CACHE, 4, 16))
    ws.copy_resident_blocks(loading, active, [2], {2: slice(0, 4)})
    torch.cuda.synchronize()
    expected_ids = torch.tensor([8, 9, 10, 11, 4, 5, 6, 7], device=gpu)
    assert torch.equal(active.local_to_global_idx, expected_ids)
    want = closed_form_rows(expected_ids, gpu)
    want[4:8] += 10.0
    assert torch.equal(active.table, want)


def _random_table(rng, rows, pitch, device):
    data = torch.from_numpy(rng.standard_normal((rows, 59)).astype(np.float32))
    return make_table(data.to(device), pitch, device)


@pytest.mark.parametrize("sp,dp,block_rows", [(59, 59, 4096), (64, 64, 4096), (59, 64, 100),
                                              (64, 59, 64), (64, 64, 37)])
def test_copy_rows_matches_oracle(gpu, sp, dp, block_rows):
    announce(f"ws copy rows sp={sp} dp={dp} block_rows={block_rows}")
    rng = np.random.default_rng(sp + dp + block_rows)
    nb = 9
    src_rows = nb * block_rows + 11
    src = _random_table(rng, src_rows, sp, gpu)
    src_g = torch.from_numpy(rng.integers(0, 1 << 40, src_rows)).to(gpu)
    n_copy = 5
    num_rows = (n_copy - 1) * block_rows + block_rows // 2 + 1  # partial last block
    src_blocks = rng.choice(nb, n_copy, replace=False)
    dst_rows = (n_copy + 2) * block_rows
    dst_slots = rng.choice(n_copy + 2, n_copy, replace=False)
    src_starts = src_blocks * block_rows + 3
    dst_starts = dst_slots * block_rows
    dst = make_table(torch.full((dst_rows, 59), -9.0, device=gpu), dp, gpu)
    dst_g = torch.full((dst_rows,), -7, dtype=torch.int64, device=gpu)
    ss = torch.from_numpy(src_starts.astype(np.int64)).to(gpu)
    ds = torch.from_numpy(dst_starts.astype(np.int64)).to(gpu)
    N.call("tgs_ws_copy_rows", N.ptr(src), sp, N.ptr(src_g), N.ptr(ss), N.ptr(ds), n_copy,
           num_rows, block_rows, N.ptr(dst), dp, N.ptr(dst_g), N.stream_handle())
    torch.cuda.synchronize()
    o_dst = W.components_of_table(np.full((dst_rows, 59), -9.0, np.float32))
    o_g = np.full(dst_rows, -7, np.int64)
    W.copy_resident_rows(W.components_of_table(to_np(src)), to_np(src_g), src_starts, dst_starts,
                         num_rows, block_rows, o_dst, o_g)
    np.testing.assert_array_equal(to_np(dst), W.table_of_components(o_dst))
    np.testing.assert_array_equal(to_np(dst_g), o_g)
    if dp == 64:
        moved = o_g != -7
        pad = to_np(padding(dst))
        assert not pad[moved].any()


@pytest.mark.parametrize("layout,dp,fused", [("cache", 64, True), ("unified", 64, True),
                                             ("cache", 59, False), ("unified", 59, True)])
def test_unpack_rows_matches_oracle(gpu, layout, dp, fused):
    announce(f"ws unpack layout={layout} dp={dp} fused_ids={fused}")
    rng = np.random.default_rng(11)
    block_rows, n_blocks = 256, 6
    rows = (n_blocks - 1) * block_rows + 77
    off = 130
    packed = torch.from_numpy(rng.standard_normal((rows, 59)).astype(np.float32)).to(gpu)
    dst = make_table(torch.full((off + rows + 5, 59), -3.0, device=gpu), dp, gpu)
    gids = torch.full((off + rows + 5,), -1, dtype=torch.int64, device=gpu)
    block_ids = rng.choice(10000, n_blocks, replace=False).astype(np.int64)
    bid = torch.from_numpy(block_ids).to(gpu)
    N.call("tgs_ws_unpack_rows", N.ptr(packed), 1 if layout == "unified" else 0, rows,
           N.ptr(dst), dp, off, N.ptr(bid) if fused else None, n_blocks if fused else 0,
           block_rows, N.ptr(gids) if fused else None, N.stream_handle())
    if not fused:
        N.call("tgs_ws_fill_global_ids", N.ptr(bid), n_blocks, N.ptr(gids), off, rows,
               block_rows, N.stream_handle())
    torch.cuda.synchronize()
    o = W.components_of_table(np.full((off + rows + 5, 59), -3.0, np.float32))
    W.unpack_streamed_rows(to_np(packed), o, off, rows, layout == "unified")
    og = np.full(off + rows + 5, -1, np.int64)
    W.fill_cold_global_ids(block_ids, og, off, rows, block_rows)
    np.testing.assert_array_equal(to_np(dst), W.table_of_components(o))
    np.testing.assert_array_equal(to_np(gids), og)
    if dp == 64:
        assert not to_np(padding(dst))[off:off + rows].any()


@pytest.mark.parametrize("sp", [59, 64])
def test_pack_rows_matches_oracle(gpu, sp):
    announce(f"ws pack sp={sp}")
    rng = np.random.default_rng(13)
    block_rows = 512
    table = _random_table(rng, 20 * block_rows, sp, gpu)
    starts = rng.choice(19, 7, replace=False) * block_rows + rng.integers(0, 64, 7)
    counts = rng.integers(1, block_rows + 1, 7)
    counts[2] = block_rows
    counts[4] = 0  # an empty plan packs nothing
    out_starts = np.concatenate([[0], np.cumsum(counts)[:-1]])
    total = int(counts.sum())
    out = torch.full((total + 3, 59), -5.0, device=gpu)
    t = lambda a: torch.from_numpy(np.asarray(a, np.int64)).to(gpu)  # noqa: E731
    s_, c_, o_ = t(starts), t(counts), t(out_starts)
    N.call("tgs_ws_pack_rows", N.ptr(table), sp, N.ptr(s_), N.ptr(c_), N.ptr(o_), 7, block_rows,
           N.ptr(out), N.stream_handle())
    torch.cuda.synchronize()
    o = np.full((total + 3, 59), -5.0, np.float32)
    W.pack_resident_rows(W.components_of_table(to_np(table)), starts, counts, out_starts, o,
                         block_rows)
    np.testing.assert_array_equal(to_np(out), o)


@pytest.mark.parametrize("pitch", [3, 59, 64])
def test_block_bounds_match_oracle(gpu, pitch):
    announce(f"ws bounds pitch={pitch}")
    rng = np.random.default_rng(17)
    block_rows = 4096
    rows = 12 * block_rows
    data = rng.standard_normal((rows, 59)).astype(np.float32) * 100
    if pitch == 3:
        table = torch.from_numpy(np.ascontiguousarray(data[:, :3])).to(gpu)
    else:
        table = make_table(torch.from_numpy(data).to(gpu), pitch, gpu)
    starts = np.array([0, 4096, 8192 + 5, 3 * 4096, 7 * 4096, 11 * 4096], np.int64)
    lengths = np.array([4096, 1, 4000, 0, 2048, 4096], np.int64)
    bounds = torch.empty((6, 6), device=gpu)
    t = lambda a: torch.from_numpy(a).to(gpu)  # noqa: E731
    s_, l_ = t(starts), t(lengths)
    N.call("tgs_ws_block_bounds", N.ptr(table), pitch, N.ptr(s_), N.ptr(l_), 6, block_rows,
           N.ptr(bounds), N.stream_handle())
    torch.cuda.synchronize()
    ref = W.resident_block_bounds(data[:, :3], starts, lengths, block_rows)
    np.testing.assert_array_equal(to_np(bounds), ref)


def test_block_starts_and_global_to_local_match_oracle(gpu):
    announce("ws block starts + global_to_local")
    rng = np.random.default_rng(19)
    bs, nb = 4096, 3000
    loaded = rng.choice(nb, 900, replace=False)
    slices, off = {}, 0
    for b in loaded:
        n = bs if b != nb - 1 else 1234
        slices[int(b)] = slice(off, off + n)
        off += n
    ws = ResidentWorkingSet(nb * bs - bs + 1234, block_size=bs, device=gpu)
    starts = ws.build_block_starts(slices)
    o_starts = W.build_block_starts(slices, nb)
    np.testing.assert_array_equal(to_np(starts), o_starts)
    g = rng.integers(-10 * bs, (nb + 10) * bs, 1_000_003).astype(np.int64)
    buf = ResidentBuffer(_block_starts=starts)
    got = ws.global_to_local(buf, torch.from_numpy(g).to(gpu))
    np.testing.assert_array_equal(to_np(got), W.global_ids_to_local(g, o_starts, bs))


def test_empty_calls_launch_nothing(gpu):
    announce("ws empty inputs")
    ws = ResidentWorkingSet(100, block_size=16, device=gpu)
    src = ResidentBuffer()
    assert ws.copy_resident_blocks(src, src, [], {}) == 0
    assert ws.stage_updated_blocks(src, [1]) is None
    assert ws.stage_block_bounds(src, []) is None
    assert N.call("tgs_ws_copy_rows", None, 59, None, None, None, 0, 0, 16, None, 59, None,
                  N.stream_handle()) == 0
    tgt = ws.materialize(None, [], set(), set(), True, None)
    assert tgt.num_gaussians == 0 and tgt.loaded_blocks == []
    with pytest.raises(ValueError, match="Invalid block IDs"):
        ws.materialize(None, [7], set(), set(), True, Reader(BlockLayout.CACHE, 16, 100))


def test_full_size_materialize_writeback_bounds(gpu):
    """4M-row working set (1000 blocks of 4096, the last partial) from a 6M
    scene: half the blocks kept from the previous buffer, half streamed in
    UNIFIED order; every row checked against the closed form, then all blocks
    packed for writeback and bounded."""
    announce("ws full size 4M rows")
    bs = 4096
    num_total = 1500 * bs - 1000
    ws = ResidentWorkingSet(num_total, block_size=bs, device=gpu, row_pitch=64)
    rng = np.random.default_rng(23)
    prev_blocks = sorted(rng.choice(1500, 800, replace=False).tolist())
    if 1499 not in prev_blocks:
        prev_blocks[-1] = 1499
    prev = ResidentBuffer()
    prev_g = torch.cat([torch.arange(b * bs, min((b + 1) * bs, num_total)) for b in prev_blocks])
    prev.table = make_table(closed_form_rows(prev_g.to(gpu), gpu), 64, gpu)
    prev.local_to_global_idx = prev_g.to(gpu)
    off = 0
    for b in prev_blocks:
        n = ws.block_length(b)
        prev.block_to_local_slice[b] = slice(off, off + n)
        off += n
    visible = sorted(set(rng.choice(prev_blocks, 500, replace=False).tolist())
                     | set(rng.choice(1500, 520, replace=False).tolist()))
    reader = Reader(BlockLayout.UNIFIED, bs, num_total, batch=True)
    tgt = ws.materialize(prev, visible, set(prev_blocks), set(), True, reader)
    torch.cuda.synchronize()
    gids = tgt.local_to_global_idx
    assert tgt.num_gaussians == gids.numel() == sum(ws.block_length(b) for b in visible)
    assert torch.equal(tgt.table, closed_form_rows(gids, gpu))
    assert not bool(padding(tgt.table).any())
    for b in (tgt.loaded_blocks[0], tgt.loaded_blocks[-1], 1499):
        if b in tgt.block_to_local_slice:
            sl = tgt.block_to_local_slice[b]
            assert gids[sl.start].item() == b * bs and gids[sl.stop - 1].item() == b * bs + (sl.stop - sl.start) - 1
    # writeback of every loaded block: CACHE-order rows grouped by ascending block id
    pend = ws.stage_updated_blocks(tgt, tgt.loaded_blocks)
    plans, packed_cpu = pend.wait()
    order = [b for b, _ in plans]
    assert order == sorted(tgt.loaded_blocks)
    want_g = torch.cat([torch.arange(b * bs, b * bs + c) for b, c in plans])
    assert torch.equal(packed_cpu, closed_form_rows(want_g))
    # bounds of every loaded block: closed form (xyz = gid + 0.1/0.2/0.3)
    pb = ws.stage_block_bounds(tgt, tgt.loaded_blocks)
    ids, cpu = pb.wait()
    lo = torch.tensor([float(b * bs) for b in ids])[:, None] + torch.tensor([0.1, 0.2, 0.3])
    hi = torch.tensor([float(b * bs + ws.block_length(b) - 1) for b in ids])[:, None] \
        + torch.tensor([0.1, 0.2, 0.3])
    assert torch.equal(cpu[:, :3], lo) and torch.equal(cpu[:, 3:], hi)


def test_materialize_from_block_store(gpu, tmp_path):
    """Stream blocks of an on-disk store (base file + two patches) into the
    resident table through the native reader, the pinned upload and the GPU
    unpack; every row equals the oracle's per-block file read."""
    from oracle import block_store_ref as B
    from tidegs_amd.block_store import BlockStore, BlockStoreReader

    announce("ws materialize from block store")
    rng = np.random.default_rng(29)
    bs, n_rows = 1024, 1024 * 300 - 77
    nb = -(-n_rows // bs)
    store = BlockStore(tmp_path, block_size=bs, num_blocks=nb)
    store.write_base(rng.standard_normal((n_rows, 59)).astype(np.float32))
    for _ in range(2):
        store.write_patch({int(b): torch.from_numpy(
            rng.standard_normal((min(bs, n_rows - b * bs), 59)).astype(np.float32))
            for b in rng.choice(nb, 40, replace=False)})
    visible = sorted(set(rng.choice(nb, 120, replace=False).tolist()) | {nb - 1})
    ws = ResidentWorkingSet(n_rows, block_size=bs, device=gpu)
    tgt = ws.materialize(None, visible, set(), set(), True, BlockStoreReader(store, n_rows))
    torch.cuda.synchronize()
    paths = {f: str(p) for f, p in store.file_paths.items()}
    table = to_np(tgt.table)
    gids = to_np(tgt.local_to_global_idx)
    for b in visible:
        loc = store.index[b]
        want = B.read_block(paths, (loc.file_id, loc.offset, loc.size), b, bs, 59)
        sl = tgt.block_to_local_slice[b]
        np.testing.assert_array_equal(table[sl], want)
        np.testing.assert_array_equal(gids[sl], np.arange(b * bs, b * bs + want.shape[0]))
    assert not bool(padding(tgt.table).any())
    store.close()
