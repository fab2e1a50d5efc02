"""Host bookkeeping of the resident optimizer (tidegs_amd.resident_optim.SlotTable
and the learning-rate table), on the CPU.

The sequence restates the known answers of the reference's
tests/test_gpu_resident_optimizer.py:155-214 (retention, eviction and
re-admission of blocks 10/20/30 with 4-row blocks): per-step cold rows, and
the aggregate cold restarts (4), evictions of initialised state (3) and live
state blocks (1).  The residency streaks follow gpu_resident_optimizer.py:
219-264 (a block's streak counts the consecutive resident sets holding it;
the mean runs over finished and current streaks).
"""
import numpy as np
import pytest

from tidegs_amd.resident_optim import GPUResidentAdam, SlotTable, component_learning_rates


def _grow(table, capacity_blocks=2):
    """GPUResidentAdam's growth rule: max(required, capacity_blocks, 2x)."""
    def reserve(required):
        have = table.capacity
        if required > have:
            table.add_slots(max(required, capacity_blocks, 2 * have, 1) - have)
    return reserve


def _step(table, layout, rows):
    """Per-block touch counts of ``rows`` over ``layout`` [(block, start,
    stop)], then SlotTable.advance of the touched blocks' slots."""
    blocks = np.array([b for b, _, _ in layout])
    starts = np.array([a for _, a, _ in layout])
    stops = np.array([z for _, _, z in layout])
    counts = np.array([np.count_nonzero((rows >= a) & (rows < z)) for a, z in zip(starts, stops)])
    hit = np.flatnonzero(counts)
    slots = table.slots_of(blocks[hit])
    assert np.all(slots >= 0)
    return table.advance(slots, (stops - starts)[hit], counts[hit])


def test_reference_residency_sequence():
    t = SlotTable()
    grow = _grow(t)
    first = t.retarget([10, 20], grow)
    assert t.capacity == 2 and sorted(first.tolist()) == [0, 1]
    assert _step(t, [(10, 0, 4), (20, 4, 7)], np.array([0, 2, 4, 6])) == (2, 4)
    assert _step(t, [(10, 0, 4), (20, 4, 7)], np.array([1, 4, 5])) == (0, 0)
    slot20 = int(t.slots_of(np.array([20]))[0])
    # block 20 stays (its slot and warm state kept), 10 leaves, 30 arrives cold
    arriving = t.retarget([20, 30], grow)
    assert int(t.slots_of(np.array([20]))[0]) == slot20
    assert arriving.tolist() == [int(t.slots_of(np.array([30]))[0])]
    assert t.evicted_warm == 1 and t.steps[slot20] == 2
    assert _step(t, [(20, 0, 3), (30, 3, 7)], np.array([0, 2, 3, 6])) == (1, 2)
    # re-admitting 10 does not recover its discarded state
    t.retarget([10], grow)
    assert _step(t, [(10, 0, 4)], np.array([0, 3])) == (1, 2)
    assert t.evicted_warm == 3
    live_blocks, live_bytes = t.live_state()
    assert live_blocks == 1 and live_bytes == 4 * 59 * 2 * 4
    cold_restarts = 2 + 0 + 1 + 1
    assert cold_restarts == 4
    # streaks: 10 ended at 1; 20 ended at 2, 30 at 1; 10 runs at 1
    assert t.mean_streak() == pytest.approx((1 + 2 + 1 + 1) / 4)
    assert int(t.steps[t.slots_of(np.array([10]))[0]]) == 1


def test_slots_lowest_free_first_and_growth():
    t = SlotTable()
    grow = _grow(t, capacity_blocks=0)
    t.retarget(range(5), grow)
    assert t.capacity == 5 and t.slots_of(np.arange(5)).tolist() == [0, 1, 2, 3, 4]
    t.retarget([3, 4], grow)              # frees 0, 1, 2
    t.retarget([0, 1, 3, 4, 7, 9], grow)  # arrivals 0, 1, 7, 9 -> slots 0, 1, 2, then growth
    assert t.capacity == 10               # doubled
    assert t.slots_of(np.array([0, 1, 7, 9, 3, 4, 8])).tolist() == [0, 1, 2, 5, 3, 4, -1]
    assert sorted(t.owner[t.owner >= 0].tolist()) == [0, 1, 3, 4, 7, 9]
    # an empty set releases everything
    t.retarget([], grow)
    assert t.blocks.size == 0 and np.all(t.owner == -1)


def test_component_learning_rates():
    specs = GPUResidentAdam.COMPONENT_SPECS
    six = [0.1, 0.2, 0.3, 0.4, 0.5, 0.6]
    lrs = component_learning_rates(six, specs)
    assert lrs == {name: pytest.approx(six[g]) for name, _, _, g in specs}
    # 59 per-column values in the unified order: each group's first column
    widths = [w for _, _, w, _ in specs]
    cols = np.concatenate([np.full(w, 10.0 * (g + 1)) + np.arange(w) for w, g in
                           zip(widths, range(6))])
    lrs = component_learning_rates(cols, specs)
    assert [lrs[name] for name, _, _, _ in specs] == [10.0, 20.0, 30.0, 40.0, 50.0, 60.0]
    with pytest.raises(RuntimeError, match="columns_lr"):
        component_learning_rates(None, specs)
    with pytest.raises(RuntimeError, match="12 values"):
        component_learning_rates(np.ones(12), specs)
