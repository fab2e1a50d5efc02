"""Resident-set policy: which blocks stay in HBM for the next batch.

Host logic over block-id sets, as in TideGS
(``strategies/tide_engine/resident_policy.py``), called once per batch from
the runtime (``runtime.py:358-372, :524``).  Two policies:

* passthrough (``compute_passthrough_resident_transition``): the next active
  set is the next resident set;
* TopC (``compute_topc_resident_transition``): rank the union of the current
  resident set and the next active set by
  ``lambda * [block is active next] + (1 - lambda) * recency`` (recency decays
  by ``recency_decay`` per batch and is 1 for blocks used this batch), keep the
  best ``resident_capacity_blocks``; ties go to higher recency, then to blocks
  already resident, then to the lower id.  Optionally a share of the
  capacity is first dealt round-robin over the next batch's cameras, each
  camera taking its best remaining block, so every camera keeps some data.

The result, a ``ResidentTransition``, names the blocks to keep, stream in and
evict; ``ResidentWorkingSet.materialize`` consumes exactly that.  The field
names and ``to_dict`` keys are the reference's, so its logging and runtime
code read them unchanged.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Dict, Iterable, List, Optional, Set, Tuple


def _ids(blocks: Optional[Iterable[int]]) -> List[int]:
    return sorted({int(b) for b in blocks}) if blocks else []


@dataclass
class ResidentTransition:
    current_active_blocks: List[int]
    next_active_blocks: List[int]
    current_resident_blocks: List[int]
    candidate_blocks: List[int]
    next_resident_blocks: List[int]
    keep_resident_blocks: List[int]
    stream_in_blocks: List[int]
    evict_blocks: List[int]
    active_overlap_blocks: List[int]
    active_delta_plus_blocks: List[int]
    active_delta_minus_blocks: List[int]
    next_camera_ids: List[int]
    resident_selection_policy: str = "passthrough_active_set"
    resident_capacity_blocks: int = -1
    requested_resident_capacity_blocks: int = -1
    resident_capacity_bytes: int = -1
    current_resident_source: str = "current_active_fallback"
    resident_lambda_weight: float = 1.0
    resident_recency_decay: float = 1.0
    balanced_seed_fraction: float = 1.0
    topc_cutoff_score: float = 0.0
    next_active_coverage: int = 0
    next_camera_coverage: int = 0
    next_camera_total: int = 0
    enforce_next_active_coverage: bool = False
    updated_recency_scores: Dict[int, float] = field(default_factory=dict)
    optional_selected_blocks: List[int] = field(default_factory=list)
    camera_seed_blocks: List[int] = field(default_factory=list)

    def __post_init__(self):
        # None means "empty", as the reference's constructor accepts
        if self.updated_recency_scores is None:
            self.updated_recency_scores = {}
        if self.optional_selected_blocks is None:
            self.optional_selected_blocks = []
        if self.camera_seed_blocks is None:
            self.camera_seed_blocks = []

    _DICT_NAMES = (("current_blocks", "current_active_blocks"),
                   ("next_blocks", "next_active_blocks"),
                   ("omega_blocks", "active_overlap_blocks"),
                   ("delta_plus_blocks", "active_delta_plus_blocks"),
                   ("delta_minus_blocks", "active_delta_minus_blocks"))

    def to_dict(self) -> Dict[str, object]:
        """The reference's key names (resident_policy.py:46-75)."""
        out = {key: getattr(self, attr) for key, attr in self._DICT_NAMES}
        for attr in ("current_resident_blocks", "candidate_blocks", "next_resident_blocks",
                     "keep_resident_blocks", "stream_in_blocks", "evict_blocks", "next_camera_ids",
                     "resident_selection_policy", "resident_capacity_blocks",
                     "requested_resident_capacity_blocks", "resident_capacity_bytes",
                     "current_resident_source", "resident_lambda_weight",
                     "resident_recency_decay", "balanced_seed_fraction", "topc_cutoff_score",
                     "next_active_coverage", "next_camera_coverage", "next_camera_total",
                     "enforce_next_active_coverage", "updated_recency_scores",
                     "optional_selected_blocks", "camera_seed_blocks"):
            out[attr] = getattr(self, attr)
        return out


def _current_resident(active: List[int], resident, scored: bool) -> Tuple[List[int], str]:
    """Which set counts as resident now, and why (resident_policy.py:84-106):
    a given resident list equal to the active set is an "expected" match; a
    different one is used as loaded state by TopC only; else the active set."""
    if resident:
        given = _ids(resident)
        if set(given) == set(active):
            return given, "expected_resident_match"
        if scored:
            return given, "loaded_resident_state"
    return list(active), "current_active_fallback"


def _recency(previous: Optional[Dict[int, float]], accessed: List[int],
             decay: float) -> Dict[int, float]:
    """Decay every score, drop those at or below 1e-6, set used blocks to 1
    (resident_policy.py:109-123)."""
    out = {}
    for b, s in (previous or {}).items():
        v = float(s) * float(decay)
        if v > 1e-6:
            out[int(b)] = v
    for b in _ids(accessed):
        out[b] = 1.0
    return out


def _camera_lists(camera_blocks, allowed: Optional[Set[int]] = None):
    """(camera, sorted blocks) per camera with at least one allowed block,
    cameras ascending (resident_policy.py:126-140)."""
    out = []
    for cam in sorted(camera_blocks or {}):
        blocks = _ids((camera_blocks or {}).get(cam, []))
        if allowed is not None:
            blocks = [b for b in blocks if b in allowed]
        if blocks:
            out.append((int(cam), blocks))
    return out


def _coverage(camera_blocks, selected: Set[int], allowed: Optional[Set[int]] = None):
    """(cameras with a selected block, cameras considered) (resident_policy.py:143-156)."""
    lists = _camera_lists(camera_blocks, allowed)
    if not lists:
        return 0, 0
    return sum(1 for _, blocks in lists if not selected.isdisjoint(blocks)), len(lists)


def _seed_capacity(camera_blocks, candidates: Set[int], capacity: int, fraction: float) -> int:
    """Capacity share dealt per camera first (resident_policy.py:226-243)."""
    if capacity <= 0:
        return 0
    frac = min(1.0, max(0.0, float(fraction)))
    if frac >= 1.0:
        return int(capacity)
    if frac <= 0.0:
        return 0
    quota = max(1, int(capacity * frac))
    cams = len(_camera_lists(camera_blocks, candidates))
    if cams > 0:
        quota = max(quota, min(int(capacity), cams))
    return min(int(capacity), quota)


def _balanced_seeds(camera_blocks, candidates: Set[int], scores: Dict[int, float],
                    resident_now: Set[int], capacity: int) -> List[int]:
    """Round-robin over cameras, each taking its best block not yet taken, until
    ``capacity`` blocks or no camera has one left (resident_policy.py:159-223).
    A camera's order: score, then how many cameras see the block, then
    already resident, then id."""
    if capacity <= 0:
        return []
    lists = _camera_lists(camera_blocks, candidates)
    if not lists:
        return []
    seen_by: Dict[int, int] = {}
    for _, blocks in lists:
        for b in blocks:
            seen_by[b] = seen_by.get(b, 0) + 1
    queues = [sorted(blocks, key=lambda b: (-float(scores.get(b, 0.0)), -seen_by.get(b, 0),
                                            -(b in resident_now), b))
              for _, blocks in lists]
    heads = [0] * len(queues)
    taken: List[int] = []
    taken_set: Set[int] = set()
    while len(taken) < capacity:
        progressed = False
        for q, queue in enumerate(queues):
            while heads[q] < len(queue) and queue[heads[q]] in taken_set:
                heads[q] += 1
            if heads[q] == len(queue):
                continue
            b = queue[heads[q]]
            heads[q] += 1
            taken.append(b)
            taken_set.add(b)
            progressed = True
            if len(taken) >= capacity:
                break
        if not progressed:
            break
    return taken


def _set_deltas(current_resident, next_resident, current_active, next_active):
    cr, nr, ca, na = map(set, (current_resident, next_resident, current_active, next_active))
    return dict(candidate_blocks=sorted(cr | na), keep_resident_blocks=sorted(cr & nr),
                stream_in_blocks=sorted(nr - cr), evict_blocks=sorted(cr - nr),
                active_overlap_blocks=sorted(ca & na), active_delta_plus_blocks=sorted(na - ca),
                active_delta_minus_blocks=sorted(ca - na))


def compute_passthrough_resident_transition(
        current_active_blocks: List[int], next_active_blocks: List[int],
        current_resident_blocks: Optional[List[int]] = None,
        next_camera_ids: Optional[List[int]] = None,
        next_camera_blocks: Optional[Dict[int, List[int]]] = None,
        previous_recency_scores: Optional[Dict[int, float]] = None,
        recency_decay: float = 0.95) -> ResidentTransition:
    """The next active set becomes the resident set (resident_policy.py:246-310)."""
    active, nxt = _ids(current_active_blocks), _ids(next_active_blocks)
    resident, source = _current_resident(active, current_resident_blocks, scored=False)
    covered, total = _coverage(next_camera_blocks, set(nxt), set(nxt))
    return ResidentTransition(
        current_active_blocks=active, next_active_blocks=nxt, current_resident_blocks=resident,
        next_resident_blocks=list(nxt), next_camera_ids=list(next_camera_ids or []),
        current_resident_source=source, resident_lambda_weight=1.0,
        resident_recency_decay=recency_decay, topc_cutoff_score=1.0 if nxt else 0.0,
        next_active_coverage=len(nxt), next_camera_coverage=covered, next_camera_total=total,
        updated_recency_scores=_recency(previous_recency_scores, active, recency_decay),
        **_set_deltas(resident, nxt, active, nxt))


def compute_topc_resident_transition(
        current_active_blocks: List[int], next_active_blocks: List[int],
        current_resident_blocks: Optional[List[int]] = None,
        next_camera_ids: Optional[List[int]] = None,
        next_camera_blocks: Optional[Dict[int, List[int]]] = None,
        previous_recency_scores: Optional[Dict[int, float]] = None,
        lambda_weight: float = 0.7, recency_decay: float = 0.95,
        resident_capacity_blocks: int = -1, balanced_camera_seeds: bool = False,
        balanced_seed_fraction: float = 1.0) -> ResidentTransition:
    """TopC selection over current resident + next active blocks
    (resident_policy.py:313-442)."""
    active, nxt = _ids(current_active_blocks), _ids(next_active_blocks)
    resident, source = _current_resident(active, current_resident_blocks, scored=True)
    recency = _recency(previous_recency_scores, active, recency_decay)
    resident_now, nxt_set = set(resident), set(nxt)
    candidates = sorted(resident_now | nxt_set)
    requested = int(resident_capacity_blocks)
    capacity = len(candidates) if requested < 0 else max(0, requested)
    capacity = min(capacity, len(candidates))
    lam = float(lambda_weight)
    scores = {b: lam * (1.0 if b in nxt_set else 0.0) + (1.0 - lam) * float(recency.get(b, 0.0))
              for b in candidates}
    seeds: List[int] = []
    if balanced_camera_seeds and capacity > 0:
        seeds = _balanced_seeds(next_camera_blocks, nxt_set, scores, resident_now,
                                _seed_capacity(next_camera_blocks, nxt_set, capacity,
                                               balanced_seed_fraction))
    chosen = list(seeds)
    room = max(0, capacity - len(chosen))
    if room > 0:
        chosen_set = set(chosen)
        ranked = sorted(candidates, key=lambda b: (-scores[b], -float(recency.get(b, 0.0)),
                                                   -(b in resident_now), b))
        chosen.extend([b for b in ranked if b not in chosen_set][:room])
    chosen = chosen[:capacity]
    nxt_resident = sorted(set(chosen))
    covered, total = _coverage(next_camera_blocks, set(nxt_resident), nxt_set)
    return ResidentTransition(
        current_active_blocks=active, next_active_blocks=nxt, current_resident_blocks=resident,
        next_resident_blocks=nxt_resident, next_camera_ids=list(next_camera_ids or []),
        resident_selection_policy="topc_balanced" if balanced_camera_seeds else "topc_strict",
        resident_capacity_blocks=capacity, requested_resident_capacity_blocks=requested,
        current_resident_source=source, resident_lambda_weight=lam,
        resident_recency_decay=float(recency_decay),
        balanced_seed_fraction=float(balanced_seed_fraction) if balanced_camera_seeds else 0.0,
        topc_cutoff_score=float(min((scores[b] for b in nxt_resident), default=0.0)),
        next_active_coverage=len(nxt_set & set(nxt_resident)), next_camera_coverage=covered,
        next_camera_total=total, enforce_next_active_coverage=False,
        updated_recency_scores=recency,
        optional_selected_blocks=sorted(b for b in chosen if b not in nxt_set),
        camera_seed_blocks=seeds,
        **_set_deltas(resident, nxt_resident, active, nxt))
