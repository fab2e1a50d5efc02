"""Host-side guards, checked without a GPU: the fused step's index widths
(tidegs_amd.tide_step: a batch whose 32-bit entry/visit counts or int32
intersection ranges would wrap is refused before any launch, on synthetic
totals) and the drop-in rasterizer's launch plan and refusals."""
import pytest

from tidegs_amd.tide_step import MAX_ISECTS, check_batch_capacity, check_isect_count


def test_batch_capacity():
    check_batch_capacity(4_000_000, 16)
    check_batch_capacity(65_000_000, 32)
    with pytest.raises(ValueError, match="32-bit"):
        check_batch_capacity(67_000_000, 32)
    with pytest.raises(ValueError, match="32-bit"):
        check_batch_capacity((1 << 32) // 3 + 1, 1)


def test_isect_count():
    check_isect_count(0)
    check_isect_count(122_056_264)
    check_isect_count(MAX_ISECTS)
    for bad in (MAX_ISECTS + 1, 1 << 32, -1):
        with pytest.raises(RuntimeError, match="int32"):
            check_isect_count(bad)


def test_rasterize_absgrad_above_32_channels_refused():
    """|dL/dmean2d| needs every channel's share of dL/dalpha in one launch, so
    the drop-in refuses absgrad above 32 channels before touching the GPU."""
    import torch
    from tidegs_amd import gsplat_ops as ops
    C, n, D = 1, 4, 40
    with pytest.raises(NotImplementedError, match="absgrad"):
        ops.rasterize_to_pixels(torch.zeros(C, n, 2), torch.zeros(C, n, 3), torch.zeros(C, n, D),
                                torch.zeros(C, n), 32, 32, 16,
                                torch.zeros(C, 2, 2, dtype=torch.int32),
                                torch.zeros(0, dtype=torch.int32), absgrad=True)


def test_channel_chunks():
    """Launch plan of the drop-in rasterizer: one launch (padded to an
    instantiated count) up to 32 channels, runs of 32 above."""
    from tidegs_amd.gsplat_ops import _channel_chunks
    assert _channel_chunks(3) == [(0, 3, 3)]
    assert _channel_chunks(5) == [(0, 5, 8)]
    assert _channel_chunks(32) == [(0, 32, 32)]
    assert _channel_chunks(33) == [(0, 32, 32), (32, 1, 1)]
    assert _channel_chunks(45) == [(0, 32, 32), (32, 13, 16)]
    assert _channel_chunks(513)[-1] == (512, 1, 1) and len(_channel_chunks(513)) == 17


def test_depth_key_range():
    """Key range of the depth sort: the visible keys and the slack map below
    2^bits - 1 (where the culled sentinel ties), bits as few as that allows;
    nothing visible ({~0, 0} from the device) sorts on all 32 bits."""
    from tidegs_amd.tide_step import DEPTH_KEY_SLACK, depth_key_range
    import numpy as np
    lo, hi = int(np.float32(24.0).view(np.uint32)), int(np.float32(146.0).view(np.uint32))
    base, bits = depth_key_range(lo, hi)
    assert base == lo - DEPTH_KEY_SLACK
    assert (hi + DEPTH_KEY_SLACK) - base < (1 << bits) - 1
    assert (hi + DEPTH_KEY_SLACK) - base >= (1 << (bits - 1)) - 1
    assert bits == 25
    assert depth_key_range(-1, 0) == (0, 32)  # int32 views of {~0, 0}
    assert depth_key_range(5, 5)[1] == ((5 + DEPTH_KEY_SLACK) - 0 + 1).bit_length()
    base, bits = depth_key_range(0x7F000000, 0x7F7FFFFF)
    assert bits <= 32 and 0x7F7FFFFF + DEPTH_KEY_SLACK - base < (1 << bits) - 1


def test_depth_range_holds():
    """The projection's own depth-key range against the ranked sort's
    [key_base, key_base + 2^bits - 1): keys at the base and just under the cap
    hold; one key below the base or at the cap (where it would tie with the
    culled sentinel) does not; slots with nothing written ({~0, 0}) are
    ignored."""
    from tidegs_amd.tide_step import RANGE_SLOTS, depth_range_holds
    empty = [0xFFFFFFFF, 0] * RANGE_SLOTS
    base, bits = 1000, 10
    cap = (1 << bits) - 1

    def slots(lo, hi):
        s = list(empty)
        s[6], s[7] = lo, hi
        s[40], s[41] = (lo + hi) // 2, (lo + hi) // 2
        return s

    assert depth_range_holds(empty, base, bits)
    assert depth_range_holds(slots(base, base + cap - 1), base, bits)
    assert not depth_range_holds(slots(base - 1, base + 5), base, bits)
    assert not depth_range_holds(slots(base, base + cap), base, bits)
    assert depth_range_holds(slots(0, 0xFFFFFFFE), 0, 32)


def test_hist0_sort_refuses_offset_first_pass():
    """tgs_segmented_sort_pairs_u32_hist0 trusts a first-pass histogram counted
    from bit 0, so it refuses any other begin_bit before launching anything."""
    import ctypes
    from tidegs_amd import _native as N
    lib = N.load()
    sel = ctypes.c_int(0)
    segs = (ctypes.c_uint32 * 2)(0, 16)
    rc = lib.tgs_segmented_sort_pairs_u32_hist0(None, None, None, None, 16, 1, segs, 1, 13,
                                                None, 0, ctypes.byref(sel), None)
    assert rc != 0 and "bit 0" in N.last_error()
