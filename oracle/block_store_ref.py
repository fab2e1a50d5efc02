"""CPU restatement of TideGS's on-disk block store reads and patch layout.

Test oracle only (see ``oracle/__init__.py``).

* ``read_block``   - one seek + read per block, short reads at the end of a
  file, empty patch records fall back to the base file
  (``storage/log_storage_manager.py:244-291``).
* ``patch_bytes``  - the bytes of a patch file: blocks in ascending id order,
  raw fp32 rows (``:311-394``), and the (offset, size) each block gets.
* ``base_offset``  - block b of the base file at b * block_size * point_dim * 4
  (``:169-202``).

Pinned by tests/test_block_store.py: the reference's own known answers in
``tests/test_log_storage_lifecycle.py`` (block_size 2, four blocks of three
floats, the arange base, two patches; the manifest round trip) and a
byte-for-byte comparison of patch files with ``np.concatenate``.
"""
from __future__ import annotations

from typing import Dict, Tuple

import numpy as np


def base_offset(block_id: int, block_size: int, point_dim: int) -> int:
    return int(block_id) * int(block_size) * int(point_dim) * 4


def read_block(paths: Dict[int, str], location: Tuple[int, int, int], block_id: int,
               block_size: int, point_dim: int) -> np.ndarray:
    """location = (file_id, offset, size)."""
    file_id, offset, size = location
    if size <= 0:
        file_id, offset, size = 0, base_offset(block_id, block_size, point_dim), \
            block_size * point_dim * 4
    with open(paths[file_id], "rb") as f:
        f.seek(offset)
        data = f.read(size)
    arr = np.frombuffer(data, dtype=np.float32).copy()
    rows = arr.size // point_dim
    return arr[:rows * point_dim].reshape(rows, point_dim)


def patch_bytes(blocks: Dict[int, np.ndarray]):
    """(file bytes, {block id: (offset, size)}) of one patch."""
    chunks, layout, offset = [], {}, 0
    for b in sorted(blocks):
        data = np.ascontiguousarray(blocks[b], dtype=np.float32).tobytes()
        layout[b] = (offset, len(data))
        chunks.append(data)
        offset += len(data)
    return b"".join(chunks), layout
