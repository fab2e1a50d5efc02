"""GPU parity of GPUResidentAdam / GPUResidentSophia against the oracle.

test_matches_reference_across_retention_eviction_and_readmission restates
tests/test_gpu_resident_optimizer.py:155-210 of the reference (same layouts,
same expected stats, same tolerance rtol 2e-5 / atol 2e-6) with the oracle's
closed-form per-block Adam as the expected values.
"""
import types

import numpy as np
import pytest
import torch

from oracle import optim_ref as O
from tests.gpu_util import announce, rel_l2, to_np
from tidegs_amd.resident_optim import GPUResidentAdam, GPUResidentSophia

pytestmark = pytest.mark.gpu
SPECS = GPUResidentAdam.COMPONENT_SPECS


class _Manager:
    def __init__(self, layout, device):
        self.device = device
        self.set_layout(layout)

    def set_layout(self, layout):
        self.loaded_blocks = [b for b, _ in layout]
        self.block_to_gpu_slice = {b: s for b, s in layout}
        rows = max(s.stop for _, s in layout)
        self.local_to_global_idx = torch.arange(rows, device=self.device)


class _Gaussians:
    def __init__(self, manager, params, columns_lr, betas=(0.9, 0.999), eps=1e-8):
        self.gpu_working_set_manager = manager
        for name, attr, _, _ in SPECS:
            setattr(self, attr, torch.nn.Parameter(params[name].clone()))
        self.optimizer = types.SimpleNamespace(
            columns_lr=torch.tensor(columns_lr, dtype=torch.float32),
            param_groups=[{"betas": betas, "eps": eps}])

    def values(self):
        return {name: getattr(self, attr).detach().cpu().double().numpy() for name, attr, _, _ in SPECS}


def _rand(rows, seed, device):
    g = torch.Generator().manual_seed(seed)
    return {name: torch.randn((rows, w), generator=g).to(device) for name, _, w, _ in SPECS}


def test_matches_reference_across_retention_eviction_and_readmission(gpu):
    announce("resident adam KAT")
    lrs = [0.01, 0.02, 0.03, 0.04, 0.05, 0.06]
    opt = GPUResidentAdam(batch_size=3, block_size=4, capacity_blocks=2, device="cuda")
    ref = O.ResidentAdamRef(batch_size=3, betas=(0.9, 0.999), eps=1e-15)

    def run(gs, ref_params, layout, ids, grads, it):
        stats = opt.step(iteration=it, gaussians=gs, sparse_grad_local_ids=ids,
                         sparse_grad_components=grads)
        rs = ref.step(ref_params, layout, to_np(ids), {k: to_np(v).astype(np.float64)
                                                       for k, v in grads.items()}, lrs)
        assert stats == rs
        for name, got in gs.values().items():
            np.testing.assert_allclose(got, ref_params[name], rtol=2e-5, atol=2e-6)
        return stats

    layout = [(10, slice(0, 4)), (20, slice(4, 7))]
    mgr = _Manager(layout, gpu)
    init = _rand(7, 10, gpu)
    gs = _Gaussians(mgr, init, lrs, eps=1e-15)
    ref_p = {k: to_np(v).astype(np.float64) for k, v in init.items()}
    opt.set_resident_blocks([10, 20])
    s = run(gs, ref_p, layout, torch.tensor([0, 2, 4, 6], device=gpu), _rand(4, 20, gpu), 1)
    assert s == {"updated_blocks": 2, "updated_block_ids": [10, 20], "touched_rows": 4, "cold_rows": 4}
    s = run(gs, ref_p, layout, torch.tensor([1, 4, 5], device=gpu), _rand(3, 21, gpu), 2)
    assert s["cold_rows"] == 0

    layout = [(20, slice(0, 3)), (30, slice(3, 7))]
    mgr.set_layout(layout)
    p2 = _rand(7, 11, gpu)
    for name, attr, _, _ in SPECS:
        setattr(gs, attr, torch.nn.Parameter(p2[name].clone()))
    ref_p = {k: to_np(v).astype(np.float64) for k, v in p2.items()}
    ref.evict_missing({20, 30})
    opt.set_resident_blocks([20, 30])
    s = run(gs, ref_p, layout, torch.tensor([0, 2, 3, 6], device=gpu), _rand(4, 22, gpu), 3)
    assert s == {"updated_blocks": 2, "updated_block_ids": [20, 30], "touched_rows": 4, "cold_rows": 2}

    layout = [(10, slice(0, 4))]
    mgr.set_layout(layout)
    p3 = _rand(4, 12, gpu)
    for name, attr, _, _ in SPECS:
        setattr(gs, attr, torch.nn.Parameter(p3[name].clone()))
    ref_p = {k: to_np(v).astype(np.float64) for k, v in p3.items()}
    ref.evict_missing({10})
    opt.set_resident_blocks([10])
    s = run(gs, ref_p, layout, torch.tensor([0, 3], device=gpu), _rand(2, 23, gpu), 4)
    assert s == {"updated_blocks": 1, "updated_block_ids": [10], "touched_rows": 2, "cold_rows": 2}
    agg = opt.get_stats()
    assert agg["cold_restarts"] == 4 and agg["state_evictions"] == 3
    assert agg["resident_state_blocks"] == 1


def _unified(rows, seed, device):
    g = torch.Generator().manual_seed(seed)
    return torch.randn((rows, 59), generator=g).to(device)


class _UnifiedGaussians:
    """Component attributes as column views of one [N,59] table (unified order)."""

    def __init__(self, manager, table, columns_lr, betas, eps):
        self.gpu_working_set_manager = manager
        self.table = table
        c = 0
        for name, attr, w, _ in SPECS:
            setattr(self, attr, table[:, c:c + w])
            c += w
        self.optimizer = types.SimpleNamespace(columns_lr=torch.tensor(columns_lr),
                                               param_groups=[{"betas": betas, "eps": eps}])


@pytest.mark.parametrize("idx_dtype", [torch.int64, torch.int32])
def test_unified_table_untouched_rows_bitwise(gpu, idx_dtype):
    announce(f"resident adam unified idx={idx_dtype}")
    rows, block = 50_000, 4096
    n_blocks = -(-rows // block)
    layout = [(b, slice(b * block, min(rows, (b + 1) * block))) for b in range(n_blocks)]
    mgr = _Manager(layout, gpu)
    table = _unified(rows, 0, gpu)
    before = table.clone()
    lrs = [1e-3, 0.05, 5e-3, 1e-3, 2.5e-3, 1.25e-4]
    gs = _UnifiedGaussians(mgr, table, lrs, (0.9, 0.999), 1e-15)
    opt = GPUResidentAdam(batch_size=4, block_size=block, device="cuda")
    opt.set_resident_blocks([b for b, _ in layout])
    g = torch.Generator().manual_seed(1)
    ids = torch.sort(torch.randperm(rows, generator=g)[: int(0.3 * rows)]).values
    grad_table = torch.randn((ids.numel(), 59), generator=g) * 1e-3
    grads, c = {}, 0
    for name, _, w, _ in SPECS:
        grads[name] = grad_table[:, c:c + w].to(gpu)
        c += w
    opt.step(1, gs, ids.to(gpu).to(idx_dtype), grads)
    untouched = torch.ones(rows, dtype=torch.bool)
    untouched[ids] = False
    assert torch.equal(table[untouched.to(gpu)], before[untouched.to(gpu)])
    # touched rows: first step is lr * g / (|g| + eps') per column
    lr_cols = np.concatenate([[lrs[gi]] * w for _, _, w, gi in SPECS])
    p, _, _ = O.adam_rows(to_np(before)[to_np(ids)].astype(np.float64),
                          grad_table.numpy().astype(np.float64), 0.0, 0.0, lr_cols, 0.9, 0.999,
                          1e-15, 4.0, 0.1, np.sqrt(0.001))
    np.testing.assert_allclose(to_np(table)[to_np(ids)], p, rtol=2e-5, atol=2e-6)


def test_sophia_matches_oracle(gpu):
    announce("resident sophia")
    rows, block = 9000, 4096
    layout = [(b, slice(b * block, min(rows, (b + 1) * block))) for b in range(3)]
    mgr = _Manager(layout, gpu)
    init = _rand(rows, 5, gpu)
    lrs = [0.01, 0.02, 0.03, 0.04, 0.05, 0.06]
    gs = _Gaussians(mgr, init, lrs, betas=(0.9, 0.99), eps=1e-12)
    opt = GPUResidentSophia(batch_size=2, block_size=block, device="cuda", rho=0.04,
                            hessian_interval=2)
    opt.set_resident_blocks([0, 1, 2])
    ref_p = {k: to_np(v).astype(np.float64) for k, v in init.items()}
    ref_m = {name: np.zeros((rows, w)) for name, _, w, _ in SPECS}
    ref_h = {name: np.zeros((rows, w)) for name, _, w, _ in SPECS}
    g = torch.Generator().manual_seed(6)
    for it in (1, 2, 3, 4):
        ids = torch.sort(torch.randperm(rows, generator=g)[:3000]).values
        grads = {name: (torch.randn((3000, w), generator=g) * 1e-2).to(gpu) for name, _, w, _ in SPECS}
        opt.step(it, gs, ids.to(gpu), grads)
        sel = ids.numpy()
        for name, _, _, gi in SPECS:
            p, m, h = O.sophia_update(ref_p[name][sel], to_np(grads[name]).astype(np.float64),
                                      ref_m[name][sel], ref_h[name][sel], lrs[gi], 0.9, 0.99,
                                      1e-12, 0.04, 2.0, update_h=(it % 2 == 0))
            ref_p[name][sel], ref_m[name][sel], ref_h[name][sel] = p, m, h
    for name, got in gs.values().items():
        np.testing.assert_allclose(got, ref_p[name], rtol=2e-5, atol=2e-6)


def test_row_outside_layout_raises(gpu):
    announce("resident adam bad row")
    layout = [(0, slice(0, 4))]
    mgr = _Manager(layout, gpu)
    gs = _Gaussians(mgr, _rand(8, 0, gpu), [0.01] * 6)
    opt = GPUResidentAdam(batch_size=1, block_size=4, device="cuda")
    opt.set_resident_blocks([0])
    with pytest.raises(RuntimeError, match="outside every resident block"):
        opt.step(1, gs, torch.tensor([1, 6], device=gpu), _rand(2, 1, gpu))
