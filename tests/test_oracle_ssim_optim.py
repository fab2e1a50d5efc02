"""Pins for the SSIM/loss oracle and the resident-optimizer oracle.

SSIM: window vs its closed form and the kernel's float32 literals; map vs a
conv2d SSIM (utils/loss_utils.py:45-85 restated with torch conv2d); backward
vs torch.autograd of that conv2d SSIM; the full TideGS loss gradient vs
autograd.
Optimizer: the known-answer stats sequence of
tests/test_gpu_resident_optimizer.py:155-214, a hand-derived first step, and
Sophia's closed-form special cases.
"""
import math
import types

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import optim_ref as O
from oracle import ssim_ref as S

# float32 literals used by the HIP kernel (tidegs_amd/csrc/ssim.hip c_gauss)
KERNEL_WINDOW = [0.001028380123898387, 0.0075987582094967365, 0.036000773310661316,
                 0.10936068743467331, 0.21300552785396576, 0.26601171493530273,
                 0.21300552785396576, 0.10936068743467331, 0.036000773310661316,
                 0.0075987582094967365, 0.001028380123898387]


def _conv_ssim_map(a, b, C1=0.01 ** 2, C2=0.03 ** 2):
    w1 = torch.tensor(S.gaussian_window(), dtype=a.dtype)
    win = (w1[:, None] * w1[None, :])[None, None].repeat(a.shape[1], 1, 1, 1)
    f = lambda x: F.conv2d(x, win, padding=5, groups=a.shape[1])  # noqa: E731
    mu1, mu2 = f(a), f(b)
    s11 = f(a * a) - mu1 ** 2
    s22 = f(b * b) - mu2 ** 2
    s12 = f(a * b) - mu1 * mu2
    return ((2 * mu1 * mu2 + C1) * (2 * s12 + C2)) / ((mu1 ** 2 + mu2 ** 2 + C1) * (s11 + s22 + C2))


def test_window_closed_form_and_kernel_literals():
    w = S.gaussian_window()
    x = np.arange(11) - 5
    ref = np.exp(-x ** 2 / 4.5)
    np.testing.assert_allclose(w, ref / ref.sum(), rtol=1e-15)
    w32 = S.gaussian_window(dtype=np.float32)
    np.testing.assert_array_equal(w32, np.array(KERNEL_WINDOW, np.float32))
    # float32 evaluation stays within one ulp of the exact taps
    assert np.all(np.abs(w32.astype(np.float64) - w) <= np.spacing(w32).astype(np.float64))


def test_ssim_map_and_backward_vs_conv2d_autograd():
    g = torch.Generator().manual_seed(0)
    a = torch.rand((2, 3, 23, 37), dtype=torch.float64, generator=g)
    b = torch.rand((2, 3, 23, 37), dtype=torch.float64, generator=g)
    m, d1, d2, d3 = S.ssim_fwd(a.numpy(), b.numpy(), dtype=np.float64)
    ref = _conv_ssim_map(a, b)
    np.testing.assert_allclose(m, ref.numpy(), atol=1e-12)
    gmap = torch.randn(a.shape, dtype=torch.float64, generator=g)
    aa = a.clone().requires_grad_()
    (gr,) = torch.autograd.grad((_conv_ssim_map(aa, b) * gmap).sum(), [aa])
    got = S.ssim_bwd(a.numpy(), b.numpy(), gmap.numpy(), d1, d2, d3, dtype=np.float64)
    np.testing.assert_allclose(got, gr.numpy(), atol=1e-11)


def test_tide_loss_grad_vs_autograd():
    g = torch.Generator().manual_seed(1)
    img = torch.rand((3, 19, 26), dtype=torch.float64, generator=g)
    gt = torch.rand((3, 19, 26), dtype=torch.float64, generator=g) * 300 - 20  # exercises clamp
    loss, grad = S.tide_loss(img.numpy(), gt.numpy(), dtype=np.float64)
    x = img.clone().requires_grad_()
    gtn = torch.clamp(gt / 255.0, 0.0, 1.0)
    L = 0.8 * (x - gtn).abs().mean() + 0.2 * (1 - _conv_ssim_map(x[None], gtn[None]).mean())
    (gr,) = torch.autograd.grad(L, [x])
    assert abs(loss - float(L)) < 1e-12
    np.testing.assert_allclose(grad, gr.numpy(), atol=1e-12)


def _np_params(rows, seed):
    rng = np.random.default_rng(seed)
    return {name: rng.normal(size=(rows, w)) for name, _, w, _ in O.COMPONENT_SPECS}


def test_resident_adam_reference_stats_sequence():
    # The block layouts and expected stats of tests/test_gpu_resident_optimizer.py:155-210.
    opt = O.ResidentAdamRef(batch_size=3, betas=(0.9, 0.999), eps=1e-15)
    lrs = [0.01, 0.02, 0.03, 0.04, 0.05, 0.06]
    p = _np_params(7, 10)
    layout = [(10, slice(0, 4)), (20, slice(4, 7))]
    s = opt.step(p, layout, np.array([0, 2, 4, 6]), _np_params(4, 20), lrs)
    assert s == {"updated_blocks": 2, "updated_block_ids": [10, 20], "touched_rows": 4, "cold_rows": 4}
    s = opt.step(p, layout, np.array([1, 4, 5]), _np_params(3, 21), lrs)
    assert s == {"updated_blocks": 2, "updated_block_ids": [10, 20], "touched_rows": 3, "cold_rows": 0}
    opt.evict_missing({20, 30})
    layout = [(20, slice(0, 3)), (30, slice(3, 7))]
    p = _np_params(7, 11)
    s = opt.step(p, layout, np.array([0, 2, 3, 6]), _np_params(4, 22), lrs)
    assert s == {"updated_blocks": 2, "updated_block_ids": [20, 30], "touched_rows": 4, "cold_rows": 2}
    opt.evict_missing({10})
    p = _np_params(4, 12)
    s = opt.step(p, [(10, slice(0, 4))], np.array([0, 3]), _np_params(2, 23), lrs)
    assert s == {"updated_blocks": 1, "updated_block_ids": [10], "touched_rows": 2, "cold_rows": 2}


def test_adam_first_step_is_lr_sign():
    # t = 1 from zero moments: update = lr * g / (|g| + eps') with eps' = eps,
    # i.e. lr * sign(g) up to eps.
    g = np.array([[0.3, -2.0, 1e-3]])
    p, m, v = O.adam_rows(np.zeros((1, 3)), g, np.zeros((1, 3)), np.zeros((1, 3)), lr=0.01,
                          b1=0.9, b2=0.999, eps=1e-15, bsz=2.0, bias1=0.1,
                          denom_scale=math.sqrt(0.001))
    np.testing.assert_allclose(p, -0.01 * np.sign(g), rtol=1e-9)
    np.testing.assert_allclose(m, 0.1 * g / 2.0, rtol=1e-12)
    np.testing.assert_allclose(v, 0.001 * (g / 2.0) ** 2, rtol=1e-12)


def test_sophia_closed_forms():
    p0 = np.array([1.0, 1.0, 1.0, 1.0])
    g = np.array([1e-3, -1e-3, 0.5, -0.5])
    m0 = np.zeros(4)
    h0 = np.full(4, 10.0)
    # no Hessian refresh: h unchanged, tiny ratios are not clipped
    p, m, h = O.sophia_update(p0, g, m0, h0, lr=0.1, b1=0.9, b2=0.99, eps=1e-12, rho=0.04,
                              bsz=1.0, update_h=False)
    np.testing.assert_array_equal(h, h0)
    np.testing.assert_allclose(m, 0.1 * g)
    np.testing.assert_allclose(p, p0 - 0.1 * (0.1 * g / 10.0))
    # zero curvature: ratio = m / eps saturates at +-rho
    p, m, h = O.sophia_update(p0, g, m0, np.zeros(4), lr=0.1, b1=0.0, b2=0.0, eps=1e-12,
                              rho=0.04, bsz=1.0, update_h=False)
    np.testing.assert_allclose(p, p0 - 0.1 * 0.04 * np.sign(g))
    # refresh with b2 = 0: h = g^2
    p, m, h = O.sophia_update(p0, g, m0, h0, lr=1.0, b1=0.0, b2=0.0, eps=1e-12, rho=1e9,
                              bsz=1.0, update_h=True)
    np.testing.assert_allclose(h, g * g)
    np.testing.assert_allclose(p, p0 - 1.0 / g)
