"""CPU restatement of TideGS's resident-block Adam and of the Sophia-style step.

Test oracle only (see ``oracle/__init__.py``).

* ``ResidentAdamRef`` restates ``GPUResidentAdam`` semantics
  (``strategies/tide_engine/gpu_resident_optimizer.py:73-513``) in the closed
  per-block form of ``tests/test_gpu_resident_optimizer.py:59-106``: per-block
  step counters, ``g / batch_size``, bias correction ``1 - b1^t`` and
  ``sqrt(1 - b2^t)``, moments dropped on eviction.  It also reproduces the
  stats dictionaries.  Pinned by the reference test's known-answer stats
  sequence and by a hand-computed single-step value.
* ``sophia_update`` (no reference implementation): Liu et al. 2023 with the
  per-coordinate clip; pinned by closed-form special cases.
"""
from __future__ import annotations

import math
from typing import Dict, List, Tuple

import numpy as np

COMPONENT_SPECS = (
    ("xyz", "_xyz", 3, 0),
    ("opacity", "_opacity", 1, 1),
    ("scaling", "_scaling", 3, 2),
    ("rotation", "_rotation", 4, 3),
    ("features_dc", "_features_dc", 3, 4),
    ("features_rest", "_features_rest", 45, 5),
)


def adam_rows(p, g, m, v, lr, b1, b2, eps, bsz, bias1, denom_scale):
    """One Adam update of whole rows (gpu_resident_optimizer.py:46-70)."""
    g = g / bsz
    m = b1 * m + (1 - b1) * g
    v = b2 * v + (1 - b2) * g * g
    p = p - (lr / bias1) * m / (np.sqrt(v) / denom_scale + eps)
    return p, m, v


class ResidentAdamRef:
    """Per-block closed-form resident Adam (tests/test_gpu_resident_optimizer.py:59-106)."""

    def __init__(self, batch_size, betas=(0.9, 0.999), eps=1e-8, dtype=np.float64):
        self.batch_size = batch_size
        self.b1, self.b2 = betas
        self.eps = eps
        self.dtype = dtype
        self.state: Dict[int, dict] = {}

    def evict_missing(self, resident_blocks):
        for b in list(self.state):
            if b not in resident_blocks:
                self.state.pop(b)

    def step(self, params: Dict[str, np.ndarray], layout: List[Tuple[int, slice]],
             local_ids: np.ndarray, grads: Dict[str, np.ndarray], columns_lr) -> dict:
        updated, cold = [], 0
        for block_id, sl in sorted(layout, key=lambda it: it[1].start):
            sel = (local_ids >= sl.start) & (local_ids < sl.stop)
            pos = np.nonzero(sel)[0]
            if pos.size == 0:
                continue
            rows = local_ids[pos] - sl.start
            n_rows = sl.stop - sl.start
            st = self.state.get(block_id)
            if st is None:
                st = {"step": 0,
                      "m": {n: np.zeros((n_rows, w), self.dtype) for n, _, w, _ in COMPONENT_SPECS},
                      "v": {n: np.zeros((n_rows, w), self.dtype) for n, _, w, _ in COMPONENT_SPECS}}
                self.state[block_id] = st
                cold += pos.size
            st["step"] += 1
            t = st["step"]
            bias1 = 1.0 - self.b1 ** t
            denom = math.sqrt(1.0 - self.b2 ** t)
            for name, _, _, gi in COMPONENT_SPECS:
                p = params[name][local_ids[pos]].astype(self.dtype)
                g = grads[name][pos].astype(self.dtype)
                p2, m2, v2 = adam_rows(p, g, st["m"][name][rows], st["v"][name][rows],
                                       columns_lr[gi], self.b1, self.b2, self.eps,
                                       float(self.batch_size), bias1, denom)
                st["m"][name][rows] = m2
                st["v"][name][rows] = v2
                params[name][local_ids[pos]] = p2
            updated.append(block_id)
        return {"updated_blocks": len(updated), "updated_block_ids": updated,
                "touched_rows": int(local_ids.size), "cold_rows": int(cold)}


def sophia_update(p, g, m, h, lr, b1, b2, eps, rho, bsz, update_h=True):
    """m = b1 m + (1-b1) g; h = b2 h + (1-b2) g^2 (refresh steps);
    p -= lr clip(m / max(h, eps), -rho, rho), with g = grad / bsz."""
    g = g / bsz
    m = b1 * m + (1 - b1) * g
    if update_h:
        h = b2 * h + (1 - b2) * g * g
    r = np.clip(m / np.maximum(h, eps), -rho, rho)
    return p - lr * r, m, h
