"""Resident-set policies (tidegs_amd.resident_policy) on hand-worked cases.
Host logic only (no GPU)."""
import pytest

from tidegs_amd.resident_policy import (compute_passthrough_resident_transition,
                                        compute_topc_resident_transition)


def test_passthrough_sets_and_recency():
    t = compute_passthrough_resident_transition([3, 1, 1, 2], [2, 4],
                                                previous_recency_scores={7: 0.5, 8: 1e-6},
                                                next_camera_ids=[5],
                                                next_camera_blocks={5: [4, 9], 6: [9]})
    assert t.current_resident_blocks == [1, 2, 3]
    assert t.current_resident_source == "current_active_fallback"
    assert t.next_resident_blocks == [2, 4] and t.keep_resident_blocks == [2]
    assert t.stream_in_blocks == [4] and t.evict_blocks == [1, 3]
    assert (t.active_overlap_blocks, t.active_delta_plus_blocks, t.active_delta_minus_blocks) \
        == ([2], [4], [1, 3])
    assert t.updated_recency_scores == {7: 0.475, 1: 1.0, 2: 1.0, 3: 1.0}
    assert (t.next_camera_coverage, t.next_camera_total) == (1, 1)  # camera 6 sees no next block
    assert t.topc_cutoff_score == 1.0 and t.next_active_coverage == 2
    d = t.to_dict()
    assert d["omega_blocks"] == [2] and d["current_blocks"] == [1, 2, 3]
    assert d["resident_selection_policy"] == "passthrough_active_set"
    # a resident list equal to the active set is the expected state
    t2 = compute_passthrough_resident_transition([1, 2], [2], current_resident_blocks=[2, 1])
    assert t2.current_resident_source == "expected_resident_match"
    t3 = compute_passthrough_resident_transition([1, 2], [2], current_resident_blocks=[5])
    assert t3.current_resident_source == "current_active_fallback"
    assert t3.current_resident_blocks == [1, 2]


def test_topc_scores_ranking_and_capacity():
    # recency after decay: 1 -> 1.0 (used now), 2 -> 1.0, 3 -> 1.0, 9 -> 0.19
    t = compute_topc_resident_transition([1, 2, 3], [3, 4, 5],
                                         previous_recency_scores={1: 1.0, 2: 0.5, 9: 0.2},
                                         lambda_weight=0.7, recency_decay=0.95,
                                         resident_capacity_blocks=4)
    # scores: 3 -> 1.0; 4, 5 -> 0.7; 1, 2 -> 0.3 (tie broken by id)
    assert t.candidate_blocks == [1, 2, 3, 4, 5]
    assert t.next_resident_blocks == [1, 3, 4, 5]
    assert t.keep_resident_blocks == [1, 3] and t.stream_in_blocks == [4, 5]
    assert t.evict_blocks == [2] and t.optional_selected_blocks == [1]
    assert t.topc_cutoff_score == pytest.approx(0.3)
    assert t.resident_capacity_blocks == 4 and t.requested_resident_capacity_blocks == 4
    assert t.next_active_coverage == 3 and t.resident_selection_policy == "topc_strict"
    assert t.updated_recency_scores[9] == pytest.approx(0.19)
    # unlimited capacity keeps every candidate; zero keeps none
    assert compute_topc_resident_transition([1, 2], [2, 3]).next_resident_blocks == [1, 2, 3]
    z = compute_topc_resident_transition([1, 2], [2, 3], resident_capacity_blocks=0)
    assert z.next_resident_blocks == [] and z.topc_cutoff_score == 0.0
    assert z.evict_blocks == [1, 2]


def test_topc_prefers_resident_blocks_on_equal_score_and_recency():
    # loaded resident state differs from the active set: blocks 7 and 8 are
    # resident, neither is active next and both have recency 0 -> score 0;
    # block 6 is not resident and also scores 0: residents first, then by id
    t = compute_topc_resident_transition([1], [2], current_resident_blocks=[7, 8],
                                         lambda_weight=1.0, resident_capacity_blocks=2)
    assert t.current_resident_source == "loaded_resident_state"
    assert t.candidate_blocks == [2, 7, 8]
    assert t.next_resident_blocks == [2, 7]


def test_topc_balanced_camera_seeds():
    cams = {0: [4], 1: [5, 3]}
    t = compute_topc_resident_transition([1, 2, 3], [3, 4, 5], next_camera_blocks=cams,
                                         lambda_weight=0.7, resident_capacity_blocks=2,
                                         balanced_camera_seeds=True)
    # round robin: camera 0 takes 4, camera 1 its best (3, score 1.0)
    assert t.camera_seed_blocks == [4, 3]
    assert t.next_resident_blocks == [3, 4]
    assert (t.next_camera_coverage, t.next_camera_total) == (2, 2)
    assert t.resident_selection_policy == "topc_balanced" and t.balanced_seed_fraction == 1.0
    # half the capacity as seeds, at least one per camera: 2 seeds, then global TopC
    h = compute_topc_resident_transition([1, 2, 3], [3, 4, 5], next_camera_blocks=cams,
                                         lambda_weight=0.7, resident_capacity_blocks=3,
                                         balanced_camera_seeds=True, balanced_seed_fraction=0.5)
    assert h.camera_seed_blocks == [4, 3]
    assert h.next_resident_blocks == [3, 4, 5]
