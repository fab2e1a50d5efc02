"""The on-disk block store (tidegs_amd.block_store) against the reference's
known answers and the CPU oracle (oracle/block_store_ref.py).  Host code
only: the native parallel reader runs without a GPU."""
import ctypes
import json
import os

import numpy as np
import pytest
import torch

from oracle import block_store_ref as B
from tidegs_amd import _native as N
from tidegs_amd.block_store import BlockStore, BlockStoreReader


def _block(value, rows=2, dim=3):
    return torch.full((rows, dim), float(value), dtype=torch.float32)


def _kat_store(path):
    # tests/test_log_storage_lifecycle.py:16-31
    store = BlockStore(path, block_size=2, num_blocks=4, point_dim=3)
    store.write_base(torch.arange(24, dtype=torch.float32).reshape(8, 3))
    return store


def test_reference_lifecycle_known_answers(tmp_path):
    # tests/test_log_storage_lifecycle.py:41-62 (reads and versions after two
    # patches) and :64-100 (manifest export + load into a fresh store)
    store = _kat_store(tmp_path / "cache")
    base_bytes = store.file_paths[0].read_bytes()
    first = store.write_patch({0: _block(10), 1: _block(11)})
    second = store.write_patch({0: _block(20), 2: _block(12)})
    assert (first, second) == (1, 2)
    got = store.read_blocks([0, 1, 2, 3])
    assert torch.equal(got[0], _block(20))
    assert torch.equal(got[1], _block(11))
    assert torch.equal(got[2], _block(12))
    assert torch.equal(got[3], torch.arange(18, 24, dtype=torch.float32).reshape(2, 3))
    assert {b: loc.version for b, loc in store.index.items()} == {0: 2, 1: 1, 2: 1, 3: 0}
    assert store.file_paths[0].read_bytes() == base_bytes
    # patch files hold the blocks in ascending id order
    data, layout = B.patch_bytes({0: _block(20).numpy(), 2: _block(12).numpy()})
    assert store.file_paths[second].read_bytes() == data
    assert {b: (store.index[b].offset, store.index[b].size) for b in (0, 2)} == layout
    assert store.file_paths[second].name.startswith("patch_000002_")

    manifest_path = tmp_path / "checkpoint" / "storage_index.json"
    manifest = store.export_index_manifest(manifest_path, tmp_path / "checkpoint" / "patches",
                                           patch_file_mode="hardlink")
    assert manifest["copied_patch_bytes"] == 0 and manifest["linked_patch_files"] == 2
    assert manifest["storage_type"] == "log_structured_blocks" and manifest["next_patch_id"] == 3
    assert json.loads(manifest_path.read_text())["index"]["0"] == {
        "file_id": 2, "offset": 0, "size": 24, "version": 2}
    resume = BlockStore(tmp_path / "resume", block_size=2, num_blocks=4, point_dim=3)
    resume.load_index_manifest(manifest_path)
    assert torch.equal(resume.read_blocks([0])[0], _block(20))
    assert torch.equal(resume.read_blocks([1])[1], _block(11))
    assert resume.next_patch_id == 3
    copy = store.export_index_manifest(tmp_path / "c2" / "m.json", tmp_path / "c2" / "p",
                                       patch_file_mode="copy")
    assert copy["copied_patch_files"] == 2 and copy["linked_patch_files"] == 0
    with pytest.raises(ValueError, match="block_size mismatch"):
        BlockStore(tmp_path / "bad", block_size=4, num_blocks=4, point_dim=3).load_index_manifest(
            manifest_path)
    store.close()
    resume.close()


@pytest.mark.parametrize("threads", [1, 8])
def test_read_batch_matches_oracle(tmp_path, threads):
    rng = np.random.default_rng(threads)
    bs, n_rows = 64, 64 * 37 + 19  # partial last block
    nb = -(-n_rows // bs)
    table = rng.standard_normal((n_rows, 59)).astype(np.float32)
    store = BlockStore(tmp_path, block_size=bs, num_blocks=nb, io_threads=threads)
    store.write_base(table)
    for _ in range(3):
        upd = {int(b): rng.standard_normal((min(bs, n_rows - b * bs), 59)).astype(np.float32)
               for b in rng.choice(nb, 9, replace=False)}
        store.write_patch({b: torch.from_numpy(v) for b, v in upd.items()})
    ids = [int(b) for b in rng.permutation(nb)[:25]] + [nb - 1]
    reader = BlockStoreReader(store, n_rows)
    rows = sum(min(bs, n_rows - b * bs) for b in ids)
    out = torch.empty((rows, 59), dtype=torch.float32)
    batch = reader.read_batch(ids, out=out)
    assert batch.tensor.data_ptr() == out.data_ptr() and batch.block_ids == tuple(ids)
    paths = {f: str(p) for f, p in store.file_paths.items()}
    for b in ids:
        loc = store.index[b]
        want = B.read_block(paths, (loc.file_id, loc.offset, loc.size), b, bs, 59)
        sl = batch.block_slices[b]
        np.testing.assert_array_equal(out[sl].numpy(), want)
    blocks = reader.read_blocks(ids[:5])
    for b in ids[:5]:
        np.testing.assert_array_equal(blocks[b].numpy(), out[batch.block_slices[b]].numpy())
    assert reader.read_blocks([nb, -1]) == {}
    with pytest.raises(ValueError, match="must be CPU"):
        reader.read_batch(ids, out=torch.empty((rows + 1, 59)))
    store.close()


def test_native_reader_rejects_reads_past_the_end(tmp_path):
    path = tmp_path / "f.bin"
    path.write_bytes(np.arange(10, dtype=np.float32).tobytes())
    fd = os.open(path, os.O_RDONLY)
    try:
        dst = np.zeros(16, np.float32)
        fds = np.array([fd], np.int32)
        sizes = np.array([48], np.int64)  # 40 bytes exist
        zero = np.zeros(1, np.int64)
        rc = N.load().tgs_io_read_blocks(1, fds.ctypes.data, zero.ctypes.data, sizes.ctypes.data,
                                         ctypes.c_void_p(dst.ctypes.data), zero.ctypes.data, 2)
        assert rc == -1 and "past the end" in N.last_error()
        sizes[0] = 40
        N.call("tgs_io_read_blocks", 1, fds.ctypes.data, zero.ctypes.data, sizes.ctypes.data,
               ctypes.c_void_p(dst.ctypes.data), zero.ctypes.data, 2)
        np.testing.assert_array_equal(dst[:10], np.arange(10, dtype=np.float32))
    finally:
        os.close(fd)


def test_empty_and_invalid_requests(tmp_path):
    store = _kat_store(tmp_path)
    assert store.read_blocks([]) == {}
    assert store.write_patch({}) == -1 and store.write_patch({1: torch.empty(0, 3)}) == -1
    with pytest.raises(ValueError, match="not in index"):
        store.read_blocks([7])
    with pytest.raises(ValueError, match="at most 2"):
        store.write_patch({0: _block(1, rows=3)})
    store.close()
