"""CPU restatement of clm_kernels' fused SSIM and TideGS's training loss.

Test oracle only (see ``oracle/__init__.py``).

* ``ssim_fwd`` restates ``clm_kernels/ssim.cu:187-286``: separable 11-tap
  Gaussian (sigma 1.5) with zero padding, x pass then y pass, SSIM map and the
  three partial-derivative maps.
* ``ssim_bwd`` restates ``ssim.cu:288-366``.
* ``tide_loss`` restates ``strategies/base_engine.py:464-488``:
  ``0.8 * L1 + 0.2 * (1 - mean SSIM)`` with ``gt = clamp(gt/255, 0, 1)``.

Pins (tests/test_oracle_ssim.py): the window against its closed form, the map
against the conv2d SSIM of ``utils/loss_utils.py:45-85`` (restated with
torch.nn.functional.conv2d), and the backward against torch.autograd of that
conv2d SSIM in float64.
"""
from __future__ import annotations

import numpy as np


def gaussian_window(size: int = 11, sigma: float = 1.5, dtype=np.float64) -> np.ndarray:
    """Normalised Gaussian taps.  For float32 this follows utils/loss_utils.py:26-32
    as torch evaluates it: exp() in double rounded to float32, the sum rounded once
    to float32, and the division in float32."""
    x = np.arange(size, dtype=np.float64) - size // 2
    g = np.exp(-(x ** 2) / (2 * sigma ** 2)).astype(dtype)
    total = dtype(g.astype(np.float64).sum())
    return (g / total).astype(dtype)


def _sep_conv(img: np.ndarray, w: np.ndarray) -> np.ndarray:
    """Zero-padded 'same' separable filter over the last two axes, x then y.
    In float32 the taps accumulate in order 0..10 in float32 (the kernel's
    arithmetic); in float64 the filter is scipy's correlate1d (double
    accumulation)."""
    if img.dtype == np.float64:
        from scipy.ndimage import correlate1d

        hx = correlate1d(img, w, axis=-1, mode="constant", cval=0.0)
        return correlate1d(hx, w, axis=-2, mode="constant", cval=0.0)
    r = len(w) // 2
    H, W = img.shape[-2:]
    pad = np.zeros(img.shape[:-2] + (H + 2 * r, W + 2 * r), dtype=img.dtype)
    pad[..., r:r + H, r:r + W] = img
    hx = np.zeros(img.shape[:-2] + (H + 2 * r, W), dtype=img.dtype)
    for t in range(len(w)):
        hx = hx + w[t] * pad[..., :, t:t + W]
    out = np.zeros(img.shape, dtype=img.dtype)
    for t in range(len(w)):
        out = out + w[t] * hx[..., t:t + H, :]
    return out


def ssim_fwd(img1, img2, C1=0.01 ** 2, C2=0.03 ** 2, dtype=np.float32):
    """Returns (ssim_map, dm_dmu1, dm_dsigma1_sq, dm_dsigma12), all [B,CH,H,W]."""
    a = np.asarray(img1, dtype=dtype)
    b = np.asarray(img2, dtype=dtype)
    w = gaussian_window(dtype=dtype)
    C1, C2 = dtype(C1), dtype(C2)
    mu1 = _sep_conv(a, w)
    mu2 = _sep_conv(b, w)
    s11 = _sep_conv(a * a, w) - mu1 * mu1
    s22 = _sep_conv(b * b, w) - mu2 * mu2
    s12 = _sep_conv(a * b, w) - mu1 * mu2
    C = 2 * mu1 * mu2 + C1
    D = 2 * s12 + C2
    A = mu1 * mu1 + mu2 * mu2 + C1
    B = s11 + s22 + C2
    m = (C * D) / (A * B)
    d_mu1 = ((mu2 * 2 * D) / (A * B) - (mu2 * 2 * C) / (A * B)
             - (mu1 * 2 * C * D) / (A * A * B) + (mu1 * 2 * C * D) / (A * B * B))
    d_s11 = (-C * D) / (A * B * B)
    d_s12 = (2 * C) / (A * B)
    return m, d_mu1, d_s11, d_s12


def ssim_bwd(img1, img2, dL_dmap, d_mu1, d_s11, d_s12, dtype=np.float32):
    """dL/dimg1 = G*(g dm/dmu1) + 2 x G*(g dm/dsigma1^2) + y G*(g dm/dsigma12)."""
    a = np.asarray(img1, dtype=dtype)
    b = np.asarray(img2, dtype=dtype)
    g = np.asarray(dL_dmap, dtype=dtype)
    w = gaussian_window(dtype=dtype)
    return (_sep_conv(g * d_mu1, w) + 2 * a * _sep_conv(g * d_s11, w)
            + b * _sep_conv(g * d_s12, w))


def tide_loss(image_chw, gt_chw_255, lambda_dssim=0.2, dtype=np.float32):
    """Loss value and dL/dimage ([3,H,W]) of the TideGS training loss."""
    img = np.asarray(image_chw, dtype=dtype)[None]
    gt = np.clip(np.asarray(gt_chw_255, dtype=dtype) / dtype(255.0), 0, 1)[None]
    n = img.size
    m, d1, d2, d3 = ssim_fwd(img, gt, dtype=dtype)
    l1 = np.abs(img - gt).mean(dtype=np.float64)
    loss = (1 - lambda_dssim) * l1 + lambda_dssim * (1 - m.mean(dtype=np.float64))
    g_map = np.full(img.shape, -lambda_dssim / n, dtype=dtype)
    grad = ssim_bwd(img, gt, g_map, d1, d2, d3, dtype=dtype)
    grad = grad + dtype((1 - lambda_dssim) / n) * np.sign(img - gt).astype(dtype)
    return float(loss), grad[0]
