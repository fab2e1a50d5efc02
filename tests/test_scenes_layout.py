"""The benchmark's resident row order (scenes.block_layout) on the CPU.

Morton codes are checked against the oracle's restatement of the streaming
initializer's code (storage/streaming_ply_init.py:154-168) and against closed
forms (one set bit per axis lands at bit 3k + axis); the layout is a
permutation whose 4096-row blocks are consecutive runs of the stable Morton
order, placed in a seeded random block order."""
import numpy as np
import torch

from oracle import streaming_init_ref as SR
from tidegs_amd import scenes


def test_morton_codes_match_streaming_init():
    g = torch.Generator().manual_seed(11)
    xyz = torch.rand((50_000, 3), generator=g) * torch.tensor([100.0, 100.0, 20.0]) - 50.0
    got = scenes.morton_codes(xyz).numpy().astype(np.uint64)
    x = xyz.numpy()
    np.testing.assert_array_equal(got, SR.morton_codes(x, x.min(0), x.max(0)))


def test_morton_codes_closed_form():
    # corners of the unit cube quantize to 0 and 1023 per axis; a point at the
    # lower corner in two axes isolates the third axis' bits
    pts = torch.tensor([[0.0, 0.0, 0.0], [1.0, 0.0, 0.0], [0.0, 1.0, 0.0], [0.0, 0.0, 1.0],
                        [1.0, 1.0, 1.0]])
    c = scenes.morton_codes(pts).tolist()
    x_bits = sum(1 << (3 * k) for k in range(10))
    assert c[0] == 0
    assert c[1] == x_bits and c[2] == x_bits << 1 and c[3] == x_bits << 2
    assert c[4] == (1 << 30) - 1


def test_block_layout_is_blocked_morton_order():
    n, B = 10_000, 1024
    g = torch.Generator().manual_seed(5)
    p = torch.cat([torch.rand((n, 3), generator=g), torch.zeros((n, 56))], 1)
    perm = scenes.block_layout(p, block_rows=B, seed=3)
    assert torch.equal(torch.sort(perm).values, torch.arange(n))
    order = torch.argsort(scenes.morton_codes(p[:, :3]), stable=True)
    chunks = [order[i:i + B] for i in range(0, n, B)]
    got, pos, used = [], 0, set()
    while pos < n:
        # each placed block is one whole chunk of the sorted order
        k = next(i for i, ch in enumerate(chunks) if int(ch[0]) == int(perm[pos]))
        assert k not in used
        used.add(k)
        assert torch.equal(perm[pos:pos + len(chunks[k])], chunks[k])
        got.append(k)
        pos += len(chunks[k])
    assert len(used) == len(chunks)
    assert got != sorted(got)  # the blocks are not left in Morton order
    assert torch.equal(perm, scenes.block_layout(p, block_rows=B, seed=3))
