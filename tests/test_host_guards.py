"""Host-side index-width guards of the fused step (tidegs_amd.tide_step): a
batch whose 32-bit entry/visit counts or int32 intersection ranges would wrap
is refused before any launch (checked on synthetic totals; no GPU)."""
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
