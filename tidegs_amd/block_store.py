"""On-disk Gaussian block store: base file, append-only patch logs, index manifest.

The format is TideGS's log-structured block store
(``storage/log_storage_manager.py``):

* ``base_file.bin``: raw little-endian fp32 rows of ``point_dim`` (59) columns in
  CACHE order (xyz | scaling | rotation | opacity | dc | rest); block ``b``
  starts at byte ``b * block_size * point_dim * 4`` (``:169-202``).
* ``patch_{id:06d}_{timestamp_us}.bin``: updated blocks appended in ascending
  block id order, each as raw fp32 rows (``:311-394``).
* the index: block id -> (file id, byte offset, byte size, version); file id 0
  is the base file.  ``export_index_manifest`` / ``load_index_manifest`` persist
  it as the same JSON document (``:397-600``).

Reads go through one native call (``tgs_io_read_blocks``) that preads every
requested block straight into its place in a pinned ``[rows, 59]`` staging
tensor with a pool of threads, instead of one seek/read/copy per block; that
tensor is what ``ResidentWorkingSet.materialize`` uploads and unpacks on the
GPU.  ``BlockStoreReader`` serves the ``storage/block_reader.py`` protocol
over a store.

Not rebuilt (storage engine, outside the GPU path): patch compaction, the
free-space reserve, the RAM block cache and the maintenance locks of
``LogStorageManager``.
"""
from __future__ import annotations

import ctypes
import json
import os
import shutil
import threading
import time
from dataclasses import dataclass
from pathlib import Path
from typing import Dict, List, Optional, Sequence

import numpy as np
import torch

from . import _native as N
from .working_set import BlockLayout


@dataclass
class BlockLocation:
    """Where a block lives (log_storage_manager.py:23-29)."""

    file_id: int  # 0 = base file, 1+ = patch files
    offset: int   # byte offset in the file
    size: int     # size in bytes
    version: int  # bumped by every patch that rewrites the block


@dataclass(frozen=True)
class BlockBatch:
    """Rows of several blocks packed in request order (block_reader.py:47-52)."""

    tensor: torch.Tensor
    block_ids: tuple
    block_slices: Dict[int, slice]
    layout: BlockLayout


def _as_rows(tensor, point_dim: int) -> np.ndarray:
    if torch.is_tensor(tensor):
        tensor = tensor.detach()
        if tensor.is_cuda:
            tensor = tensor.cpu()
        tensor = tensor.numpy()
    arr = np.ascontiguousarray(np.asarray(tensor, dtype=np.float32))
    if arr.ndim != 2 or arr.shape[1] != point_dim:
        raise ValueError(f"expected (*, {point_dim}) rows, got {arr.shape}")
    return arr


class BlockStore:
    """Base file + patch logs + index of ``num_blocks`` blocks of ``block_size``
    rows of ``point_dim`` fp32 values."""

    def __init__(self, storage_dir, block_size: int, num_blocks: int, point_dim: int = 59,
                 io_threads: int = 8):
        self.storage_dir = Path(storage_dir)
        self.storage_dir.mkdir(parents=True, exist_ok=True)
        self.block_size = int(block_size)
        self.num_blocks = int(num_blocks)
        self.point_dim = int(point_dim)
        self.bytes_per_point = self.point_dim * 4
        self.bytes_per_block = self.block_size * self.bytes_per_point
        self.io_threads = int(io_threads)
        self.index: Dict[int, BlockLocation] = {}
        self.index_lock = threading.Lock()
        self.file_paths: Dict[int, Path] = {0: self.storage_dir / "base_file.bin"}
        self.next_patch_id = 1
        self.patch_counter_lock = threading.Lock()
        self._fds: Dict[int, int] = {}
        self._fd_lock = threading.Lock()
        self.stats = {"reads": 0, "writes": 0, "patches_created": 0, "read_bytes": 0}
        base = self.file_paths[0]
        if not base.exists():
            # a sparse file of the full size, as log_storage_manager.py:186-196
            with open(base, "wb") as f:
                if self.num_blocks > 0:
                    f.seek(self.num_blocks * self.bytes_per_block - 1)
                    f.write(b"\0")
        for b in range(self.num_blocks):
            self.index[b] = BlockLocation(0, b * self.bytes_per_block, self.bytes_per_block, 0)

    # ------------------------------------------------------------------ base
    def write_base(self, rows) -> None:
        """Write ``[N, point_dim]`` rows as the base file (block b at
        b * bytes_per_block; the last block may be partial)."""
        arr = _as_rows(rows, self.point_dim)
        if arr.shape[0] > self.num_blocks * self.block_size:
            raise ValueError("more rows than the store's blocks hold")
        self._close_fds()
        with open(self.file_paths[0], "wb") as f:
            arr.tofile(f)
            f.flush()
            os.fsync(f.fileno())

    # ------------------------------------------------------------------ reads
    def _fd(self, file_id: int) -> int:
        with self._fd_lock:
            fd = self._fds.get(file_id)
            if fd is None:
                fd = os.open(self.file_paths[file_id], os.O_RDONLY)
                self._fds[file_id] = fd
            return fd

    def _plan(self, block_ids: Sequence[int]):
        """(fd, offset, nbytes) per block: the stored size, cut at the end of
        the file like a short read (log_storage_manager.py:244-276)."""
        fds, offs, sizes = [], [], []
        with self.index_lock:
            locs = []
            for b in block_ids:
                if b not in self.index:
                    raise ValueError(f"Block {b} not in index")
                locs.append(self.index[b])
        for b, loc in zip(block_ids, locs):
            file_id, offset, size = loc.file_id, loc.offset, loc.size
            if size <= 0:  # empty patch record: fall back to the base file (:253-259)
                file_id, offset, size = 0, int(b) * self.bytes_per_block, self.bytes_per_block
            fd = self._fd(file_id)
            end = os.fstat(fd).st_size
            nbytes = max(0, min(size, end - offset))
            nbytes -= nbytes % self.bytes_per_point
            if nbytes <= 0:
                raise RuntimeError(f"block {b} read as empty from {self.file_paths[file_id]}")
            fds.append(fd)
            offs.append(offset)
            sizes.append(nbytes)
        return fds, offs, sizes

    def _read_into(self, fds, offs, sizes, out: torch.Tensor, dst_offsets) -> None:
        n = len(fds)
        if n == 0:
            return
        order = sorted(range(n), key=lambda i: (fds[i], offs[i]))  # forward through each file
        a_fd = np.array([fds[i] for i in order], np.int32)
        a_off = np.array([offs[i] for i in order], np.int64)
        a_sz = np.array([sizes[i] for i in order], np.int64)
        a_dst = np.array([dst_offsets[i] for i in order], np.int64)
        N.call("tgs_io_read_blocks", n, a_fd.ctypes.data, a_off.ctypes.data, a_sz.ctypes.data,
               ctypes.c_void_p(out.data_ptr()), a_dst.ctypes.data, self.io_threads)
        self.stats["reads"] += n
        self.stats["read_bytes"] += int(a_sz.sum())

    def read_blocks(self, block_ids: List[int]) -> Dict[int, torch.Tensor]:
        """{block id: CPU [rows, point_dim] tensor} (log_storage_manager.py:204-278)."""
        ids = [int(b) for b in block_ids]
        if not ids:
            return {}
        fds, offs, sizes = self._plan(ids)
        total = sum(sizes)
        buf = torch.empty(total // 4, dtype=torch.float32)
        dst, acc = [], 0
        for s in sizes:
            dst.append(acc)
            acc += s
        self._read_into(fds, offs, sizes, buf, dst)
        out = {}
        for b, d, s in zip(ids, dst, sizes):
            out[b] = buf[d // 4:(d + s) // 4].view(-1, self.point_dim)
        return out

    def read_batch(self, block_ids: List[int], out: Optional[torch.Tensor] = None) -> BlockBatch:
        """The requested blocks' rows packed in request order into ``out``
        (a CPU ``[rows, point_dim]`` tensor, normally pinned), one native call."""
        ids = [int(b) for b in block_ids]
        fds, offs, sizes = self._plan(ids)
        rows = sum(sizes) // self.bytes_per_point
        if out is None:
            out = torch.empty((rows, self.point_dim), dtype=torch.float32)
        elif (out.device.type != "cpu" or out.dim() != 2 or tuple(out.shape) != (rows, self.point_dim)
              or not out.is_contiguous() or out.dtype != torch.float32):
            raise ValueError(f"BlockBatch output must be CPU fp32 ({rows}, {self.point_dim}); got "
                             f"{tuple(out.shape)} on {out.device}")
        dst, slices, acc = [], {}, 0
        for b, s in zip(ids, sizes):
            dst.append(acc * self.bytes_per_point)
            n = s // self.bytes_per_point
            slices[b] = slice(acc, acc + n)
            acc += n
        self._read_into(fds, offs, sizes, out, dst)
        return BlockBatch(out, tuple(ids), slices, BlockLayout.CACHE)

    # ---------------------------------------------------------------- patches
    def write_patch(self, block_dict: Dict[int, torch.Tensor]) -> int:
        """Append updated blocks to a new patch file and point the index at them
        (log_storage_manager.py:311-394); returns the patch id, -1 if empty."""
        if not block_dict:
            return -1
        valid = {}
        for b, t in block_dict.items():
            if t is None or t.numel() == 0:
                continue
            arr = _as_rows(t, self.point_dim)
            if arr.shape[0] > self.block_size:
                raise ValueError(f"Invalid dirty block {b} rows {arr.shape[0]}; "
                                 f"expected at most {self.block_size}")
            valid[int(b)] = arr
        if not valid:
            return -1
        with self.patch_counter_lock:
            patch_id = self.next_patch_id
            self.next_patch_id += 1
        stamp = int(time.time() * 1_000_000)
        path = self.storage_dir / f"patch_{patch_id:06d}_{stamp}.bin"
        locations, offset = {}, 0
        try:
            with open(path, "wb") as f:
                for b in sorted(valid):
                    data = valid[b].tobytes()
                    f.write(data)
                    with self.index_lock:
                        old = self.index[b].version if b in self.index else 0
                    locations[b] = BlockLocation(patch_id, offset, len(data), old + 1)
                    offset += len(data)
                f.flush()
                os.fsync(f.fileno())
        except Exception:
            path.unlink(missing_ok=True)
            raise
        with self.index_lock:
            self.file_paths[patch_id] = path
            self.index.update(locations)
        self.stats["writes"] += len(valid)
        self.stats["patches_created"] += 1
        return patch_id

    # --------------------------------------------------------------- manifest
    def export_index_manifest(self, manifest_path, patches_dir,
                              patch_file_mode: str = "hardlink") -> Dict:
        """Persist the index; patch files are hard-linked (or copied) into
        ``patches_dir``, the base file is referenced by absolute path
        (log_storage_manager.py:413-542)."""
        mode = str(patch_file_mode).lower()
        if mode not in {"hardlink", "copy"}:
            raise ValueError(f"Invalid patch_file_mode={patch_file_mode!r}; expected hardlink or copy")
        manifest_path, patches_dir = Path(manifest_path), Path(patches_dir)
        manifest_path.parent.mkdir(parents=True, exist_ok=True)
        patches_dir.mkdir(parents=True, exist_ok=True)
        with self.index_lock:
            index = dict(self.index)
            paths = dict(self.file_paths)
        with self.patch_counter_lock:
            next_patch_id = int(self.next_patch_id)
        referenced = {0} | {int(loc.file_id) for loc in index.values()}
        files = {}
        counters = dict(patch_files=0, patch_bytes=0, copied_patch_files=0, copied_patch_bytes=0,
                        linked_patch_files=0, linked_patch_bytes=0)
        for file_id, src in sorted(paths.items()):
            if file_id not in referenced:
                continue
            src = Path(src)
            if not src.exists():
                raise FileNotFoundError(f"Log storage file missing for file_id={file_id}: {src}")
            linked = copied = False
            if file_id == 0:
                dst = src.resolve()
            else:
                dst = patches_dir / src.name
                if src.resolve() != dst.resolve():
                    if dst.exists():
                        if os.path.samefile(src, dst) and mode == "hardlink":
                            linked = True
                        else:
                            dst.unlink()
                    if not dst.exists():
                        if mode == "hardlink":
                            try:
                                os.link(src, dst)
                                linked = True
                            except OSError:
                                shutil.copy2(src, dst)
                                copied = True
                        else:
                            shutil.copy2(src, dst)
                            copied = True
                dst = dst.resolve()
            size = int(dst.stat().st_size)
            if file_id != 0:
                counters["patch_files"] += 1
                counters["patch_bytes"] += size
                if copied:
                    counters["copied_patch_files"] += 1
                    counters["copied_patch_bytes"] += size
                if linked:
                    counters["linked_patch_files"] += 1
                    counters["linked_patch_bytes"] += size
            files[str(file_id)] = {"path": str(dst), "role": "base" if file_id == 0 else "patch",
                                   "copied": bool(copied), "linked": bool(linked), "size": size}
        manifest = {
            "version": 1,
            "storage_type": "log_structured_blocks",
            "block_size": self.block_size,
            "num_blocks": self.num_blocks,
            "point_dim": self.point_dim,
            "dtype": "float32",
            "bytes_per_block": self.bytes_per_block,
            "next_patch_id": next_patch_id,
            "files": files,
            "index": {str(b): {"file_id": int(loc.file_id), "offset": int(loc.offset),
                               "size": int(loc.size), "version": int(loc.version)}
                      for b, loc in sorted(index.items())},
            "patch_file_mode": mode,
            **counters,
        }
        tmp = manifest_path.with_name(f".{manifest_path.name}.tmp")
        with open(tmp, "w", encoding="utf-8") as handle:
            json.dump(manifest, handle, indent=2, sort_keys=True)
            handle.flush()
            os.fsync(handle.fileno())
        os.replace(tmp, manifest_path)
        return manifest

    def load_index_manifest(self, manifest_path) -> Dict:
        """Adopt a persisted index (log_storage_manager.py:544-600)."""
        with open(manifest_path, "r", encoding="utf-8") as handle:
            manifest = json.load(handle)
        for key, mine in (("block_size", self.block_size), ("num_blocks", self.num_blocks),
                          ("point_dim", self.point_dim)):
            if int(manifest.get(key, -1)) != int(mine):
                raise ValueError(f"Index {key} mismatch: manifest={manifest.get(key)} runtime={mine}")
        paths = {}
        for fid, info in manifest.get("files", {}).items():
            p = Path(info["path"])
            if not p.exists():
                raise FileNotFoundError(f"Index file_id={fid} path does not exist: {p}")
            paths[int(fid)] = p
        index = {}
        for bid, loc in manifest.get("index", {}).items():
            if int(loc["file_id"]) not in paths:
                raise KeyError(f"Block {bid} references missing file_id={loc['file_id']}")
            index[int(bid)] = BlockLocation(int(loc["file_id"]), int(loc["offset"]),
                                            int(loc["size"]), int(loc["version"]))
        if len(index) != self.num_blocks:
            raise ValueError(f"Index block count mismatch: manifest={len(index)} "
                             f"runtime={self.num_blocks}")
        self._close_fds()
        with self.index_lock:
            self.file_paths = paths
            self.index = index
        with self.patch_counter_lock:
            self.next_patch_id = max(int(manifest.get("next_patch_id", 1)), max(paths, default=0) + 1)
        return manifest

    # ------------------------------------------------------------------ misc
    def get_stats(self) -> Dict:
        out = dict(self.stats)
        out["num_patches"] = len([f for f in self.file_paths if f != 0])
        return out

    def _close_fds(self) -> None:
        with self._fd_lock:
            for fd in self._fds.values():
                os.close(fd)
            self._fds = {}

    def close(self) -> None:
        self._close_fds()

    def __del__(self):
        try:
            self._close_fds()
        except Exception:
            pass


class BlockStoreReader:
    """``storage/block_reader.py`` protocol over a ``BlockStore`` holding
    ``total_gaussians`` rows (CACHE layout); what ``ResidentWorkingSet.materialize``
    takes as ``block_reader``."""

    layout = BlockLayout.CACHE

    def __init__(self, store: BlockStore, total_gaussians: int):
        self.store = store
        self.total_gaussians = int(total_gaussians)
        self.block_size = store.block_size
        self.num_blocks = (self.total_gaussians + self.block_size - 1) // self.block_size

    def _valid(self, block_ids):
        return [int(b) for b in block_ids if 0 <= int(b) < self.num_blocks]

    def read_blocks(self, block_ids: List[int]) -> Dict[int, torch.Tensor]:
        return self.store.read_blocks(self._valid(block_ids))

    def read_batch(self, block_ids: List[int], out: Optional[torch.Tensor] = None) -> BlockBatch:
        return self.store.read_batch(self._valid(block_ids), out=out)

    def hint_future(self, block_ids: List[int]) -> int:
        return 0

    def contains_block(self, block_id: int) -> bool:
        return 0 <= int(block_id) < self.num_blocks
